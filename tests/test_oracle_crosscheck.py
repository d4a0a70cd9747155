"""Pins for the oracle beyond the literal vectors:
- the event-driven C restatement agrees with the literal queue-formulation restatement
  (oracle/queue_ref.py) on random small layers in every mode, including capacity
  truncation, pads, thresholds <= 0 and n_real > L;
- the conv candidate routing agrees with a brute-force dense construction (every
  neuron x every event, valid-tap mask), restating salt_core/tests/_reference.py:19-61;
- the shift-rounded multiply: closed form (exact 64-bit) vs the reference's int32
  hi/lo split, on random wide values (salt_core/tests/test_fixed_point.py:101-122), and
  the |round_shift(a*v)| <= |v| invariant (test_fixed_point.py:53-66).
"""
import numpy as np
import pytest

from oracle import oracle as O
from oracle import queue_ref as Q
from salt_amd.quant.codes import build_decay_table_int


def _rand_case(rng):
    fa = int(rng.integers(0, 16))
    fV = int(rng.integers(0, 4))
    iV = int(rng.integers(4, 31 - fV))
    tau = float(rng.choice([2.0, 4.0, 16.0, 40.0]))
    tab = build_decay_table_int(fa, tau)
    if tab.size == 0:
        tab = np.zeros(1, np.int32)
    rm = str(rng.choice(["round", "truncate"]))
    om = str(rng.choice(["wrap", "saturate"]))
    L = int(rng.integers(1, 40))
    nr = int(rng.integers(0, L + 3))
    t = np.sort(rng.integers(0, 30, L)).astype(np.float32)
    if rng.random() < 0.5:
        t[min(nr, L):] = 1e12
    if rng.random() < 0.5:
        kind = "fc"
        n_in, n_out = int(rng.integers(1, 6)), int(rng.integers(1, 6))
        src = rng.integers(0, n_in, L).astype(np.int32)
        q = rng.integers(-20, 21, (n_out, n_in)).astype(np.int32)
        N = n_out
        geom = dict(kind="fc", n_in=n_in, n_out=n_out)
    else:
        kind = "conv"
        while True:
            ic, h, w = int(rng.integers(1, 3)), int(rng.integers(1, 6)), int(rng.integers(1, 6))
            k, s, p = int(rng.integers(1, 4)), int(rng.integers(1, 3)), int(rng.integers(0, 2))
            if (h + 2 * p - k) // s + 1 >= 1 and (w + 2 * p - k) // s + 1 >= 1:
                break
        oc, mql = int(rng.integers(1, 3)), int(rng.integers(1, 12))
        src = rng.integers(0, ic * h * w, L).astype(np.int32)
        q = rng.integers(-20, 21, (oc, ic, k, k)).astype(np.int32)
        N = oc * ((h + 2 * p - k) // s + 1) * ((w + 2 * p - k) // s + 1)
        geom = dict(kind="conv", ic=ic, h_in=h, w_in=w, oc=oc, k=k, s=s, p=p, max_queue_len=mql)
    vk = int(rng.integers(0, 4))
    vth = None if vk == 0 else (int(rng.integers(-3, 40)) if vk == 1 else rng.integers(-2, 40, N).astype(np.int32))
    cap = int(rng.integers(1, 30))
    params = dict(q=q, table=tab, v_th=vth, f_a=fa, f_V=fV, i_V=iV, round_mode=rm, overflow_mode=om)
    return geom, params, t, src, nr, cap


def _queue(geom, prm, t, src, nr, cap):
    a = (prm["q"], prm["table"], prm["v_th"], prm["f_a"], prm["f_V"], prm["i_V"], t, src, nr, cap)
    kw = dict(round_mode=prm["round_mode"], overflow_mode=prm["overflow_mode"])
    if geom["kind"] == "fc":
        return Q.fc_forward(*a, **kw)
    g = {k: geom[k] for k in ("ic", "h_in", "w_in", "k", "s", "p", "max_queue_len")}
    return Q.conv_forward(*a, **g, **kw)


@pytest.mark.parametrize("seed", range(6))
def test_event_driven_oracle_equals_queue_formulation(seed):
    rng = np.random.default_rng(seed)
    hits = {"trunc_out": 0, "trunc_queue": 0, "pads": 0}
    for _ in range(60):
        geom, prm, t, src, nr, cap = _rand_case(rng)
        r = _queue(geom, prm, t, src, nr, cap)
        o = O.layer_forward(geom, prm, t[None], src[None], np.array([nr]), cap)
        np.testing.assert_array_equal(o["v_final"][0], r["v_final"])
        np.testing.assert_array_equal(o["v_min"][0], r["v_unfitted_min"])
        np.testing.assert_array_equal(o["v_max"][0], r["v_unfitted_max"])
        assert int(o["out_n"][0]) == r["out_n"]
        np.testing.assert_array_equal(o["out_times"][0], r["out_times"])
        np.testing.assert_array_equal(o["out_src"][0], r["out_src"])
        if geom["kind"] == "conv":
            assert int(o["needed_queue"][0]) == r["needed_queue"]
            hits["trunc_queue"] += r["needed_queue"] > geom["max_queue_len"]
        hits["trunc_out"] += r["out_n"] > cap
        hits["pads"] += nr < t.shape[0]
    assert all(v > 0 for v in hits.values()), hits  # the regimes were exercised


def _dense_conv_sequences(x, y, c, n_real, K, S, P, H, W):
    """Brute force: for every output position, the events whose tap is valid, in order
    (restates the mask of salt_core/tests/_reference.py:47-54)."""
    seqs = {}
    for oy in range(H):
        for ox in range(W):
            lst = []
            for j in range(n_real):
                ky = y[j] - oy * S + P
                kx = x[j] - ox * S + P
                if 0 <= ky < K and 0 <= kx < K:
                    lst.append((j, c[j], ky, kx))
            seqs[oy * W + ox] = lst
    return seqs


@pytest.mark.parametrize("seed", range(4))
def test_conv_routing_equals_dense_brute_force(seed):
    """Each conv neuron's register equals a per-neuron sequential scan over exactly the
    events the dense construction gives it, then the catch-up decay to the last time."""
    rng = np.random.default_rng(100 + seed)
    for _ in range(20):
        ic, h, w = int(rng.integers(1, 3)), int(rng.integers(2, 7)), int(rng.integers(2, 7))
        K, S, P = int(rng.integers(1, 4)), int(rng.integers(1, 3)), int(rng.integers(0, 2))
        H, W = (h + 2 * P - K) // S + 1, (w + 2 * P - K) // S + 1
        if H < 1 or W < 1:
            continue
        oc = 2
        L = int(rng.integers(1, 30))
        t = np.sort(rng.integers(0, 40, L)).astype(np.float32)
        src = rng.integers(0, ic * h * w, L).astype(np.int32)
        q = rng.integers(-30, 31, (oc, ic, K, K)).astype(np.int32)
        tab = build_decay_table_int(6, 8.0)
        prm = dict(q=q, table=tab, v_th=None, f_a=6, f_V=1, i_V=20, round_mode="round",
                   overflow_mode="wrap")
        geom = dict(kind="conv", ic=ic, h_in=h, w_in=w, oc=oc, k=K, s=S, p=P, max_queue_len=L + 1)
        o = O.layer_forward(geom, prm, t[None], src[None], np.array([L]), 4)
        x, y, c = src % (h * w) % w, src % (h * w) // w, src // (h * w)
        seqs = _dense_conv_sequences(x, y, c, L, K, S, P, H, W)
        T = t[L - 1]
        for o_c in range(oc):
            for pos in range(H * W):
                v, t_last = 0, np.float32(0)
                for j, cj, ky, kx in seqs[pos]:
                    a, ident = O.decay_lookup(np.float32(t[j] - t_last), tab)
                    v = O.process_event(v, a, ident, int(q[o_c, cj, ky, kx]), None, f_a=6,
                                        f_V=1, i_V=20)["v_final"]
                    t_last = t[j]
                if seqs[pos]:
                    a, ident = O.decay_lookup(np.float32(T - t_last), tab)
                    v = O.process_event(v, a, ident, 0, None, f_a=6, f_V=1, i_V=20)["v_final"]
                assert o["v_final"][0, o_c * H * W + pos] == v


def test_wide_mul_shift_closed_form_equals_reference_split():
    rng = np.random.default_rng(3)
    for n in (1, 4, 6, 10, 15):
        a = rng.integers(0, 2 ** n, 2000).astype(np.int32)
        v = rng.integers(-(2 ** 29), 2 ** 29, 2000).astype(np.int32)
        for mode in ("round", "truncate"):
            split = Q.wide_mul_shift(a, v, n, mode)
            closed = np.array([O.wide_mul_shift(int(ai), int(vi), n, mode) for ai, vi in zip(a, v)])
            exact = (a.astype(object) * v.astype(object) + ((1 << (n - 1)) if mode == "round" else 0)) >> n
            np.testing.assert_array_equal(split, closed)
            np.testing.assert_array_equal(closed, np.array(exact, dtype=np.int64))


def test_decay_never_grows_magnitude():
    rng = np.random.default_rng(0)
    v = rng.integers(-100000, 100000, 2000)
    a = rng.integers(0, 2 ** 6, 2000)
    for mode in ("round", "truncate"):
        r = np.array([O.wide_mul_shift(int(ai), int(vi), 6, mode) for ai, vi in zip(a, v)])
        assert np.all(np.abs(r) <= np.abs(v))


def test_stream_hash_is_order_sensitive():
    t = np.array([1.0, 2.0, 3.0], np.float32)
    s = np.array([5, 6, 7], np.int32)
    h = O.stream_hash(t, s, 3, 4)
    assert h != O.stream_hash(t[::-1].copy(), s[::-1].copy(), 3, 4)
    assert h != O.stream_hash(t, s, 2, 4)
    assert h == O.stream_hash(np.append(t, 9.0).astype(np.float32), np.append(s, 1).astype(np.int32), 3, 4)
