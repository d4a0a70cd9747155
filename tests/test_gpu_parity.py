"""GPU path vs the CPU oracle, bit for bit: spike streams (times, sources, counts),
final registers, per-neuron and per-stream extremes, needed queue lengths.  Geometries
are chosen to exercise each work decomposition: whole layer in one wave per stream
(direct output), channel groups and row bands (spike masks + compaction), FC slices."""
import numpy as np
import pytest

from salt_amd import ConvLayer, FCLayer, QuantizedLayerParams
from salt_amd.quant.codes import build_decay_table_int
from oracle import oracle as O
from helpers import assert_layer_equal, oracle_spec
from gpu_util import run_layer

pytestmark = pytest.mark.gpu

MODES = [("round", "wrap", 10, 0, 24), ("truncate", "saturate", 6, 2, 12), ("round", "saturate", 15, 3, 27),
         ("truncate", "wrap", 4, 1, 29), ("round", "wrap", 0, 0, 20)]


def _events(rng, B, L, n_src, t_max=200, dup=0.25):
    times = np.zeros((B, L), np.float32)
    src = rng.integers(0, n_src, (B, L)).astype(np.int32)
    n_real = rng.integers(max(1, L // 2), L + 1, B).astype(np.int32)
    n_real[0] = L
    if B > 1:
        n_real[1] = 0
    for b in range(B):
        gaps = np.where(rng.random(L) < dup, 0, rng.integers(1, max(2, 2 * t_max // L), L))
        times[b] = np.cumsum(gaps)
        times[b, n_real[b]:] = 1e12
    return times, src, n_real


def _params(rng, shape, n_neurons, oc, mode, bits, vth_kind):
    rm, om, fa, fV, iV = mode
    lim = {8: 127, 16: 2000, 32: 70000}[bits]
    q = rng.integers(-lim, lim + 1, shape)
    tab = build_decay_table_int(fa, 12.0)
    if tab.size == 0:
        tab = np.zeros(1, np.int32)
    hi = max(2, min(2 ** (iV + fV - 1) - 1, lim * (1 << fV)))
    if vth_kind == "none":
        vth = None
    elif vth_kind == "scalar":
        vth = np.int32(rng.integers(1, hi))
    elif vth_kind == "channel":
        vth = np.repeat(rng.integers(1, hi, oc), n_neurons // oc).astype(np.int32)
    else:
        vth = rng.integers(1, hi, n_neurons).astype(np.int32)
    return QuantizedLayerParams(q=q, decay_table_int=tab, v_th_int=vth, scale=np.float32(1.0),
                                f_a=fa, f_V=fV, i_V=iV, overflow_mode=om), rm


CONV_CASES = [
    # (ic, h, w, oc, k, s, p, B, L)  -- comment: expected plan
    (2, 10, 10, 2, 3, 1, 0, 16, 200),      # direct: one wave per stream
    (2, 12, 12, 8, 3, 1, 1, 8, 300),       # channel groups -> masks
    (2, 34, 34, 16, 5, 2, 0, 8, 400),      # N-MNIST conv1 geometry
    (16, 15, 15, 32, 3, 2, 0, 8, 400),     # N-MNIST conv2 geometry
    (1, 130, 130, 4, 3, 1, 0, 4, 800),     # row bands (state above the LDS budget)
    (3, 9, 11, 5, 4, 3, 2, 8, 150),        # odd sizes, stride 3, padding 2
    (1, 7, 7, 3, 1, 2, 0, 8, 100),         # k < s: some pixels reach no neuron
]


@pytest.mark.parametrize("case", CONV_CASES)
@pytest.mark.parametrize("mi", range(len(MODES)))
def test_conv_matches_oracle(case, mi):
    ic, h, w, oc, k, s, p, B, L = case
    rng = np.random.default_rng(1000 * mi + sum(case))
    layer = ConvLayer(name="c", ic=ic, h_in=h, w_in=w, oc=oc, k=k, s=s, p=p, init_k=1.0,
                      max_queue_len=int(rng.choice([L + 1, max(2, L // 20)])),
                      max_out_spikes=int(rng.choice([4 * L * oc, 7])))
    bits = [8, 16, 32][mi % 3]
    vk = ["scalar", "channel", "neuron", "none"][mi % 4]
    params, rm = _params(rng, layer.weight_shape, layer.n_neurons, oc, MODES[mi], bits, vk)
    times, src, n_real = _events(rng, B, L, ic * h * w)
    print("conv case", case, "mode", MODES[mi], "bits", bits, "vth", vk, "mql", layer.max_queue_len,
          "cap", layer.max_out_spikes, flush=True)
    out = run_layer(layer, params, times, src, n_real, round_mode=rm)
    geom, prm, cap = oracle_spec(layer, params, rm)
    ref = O.layer_forward(geom, prm, times, src, n_real, cap)
    assert_layer_equal(out, ref, tag=str(case))


FC_CASES = [(2312, 128, 4, 300), (37, 10, 16, 200), (100, 1000, 4, 120), (64, 1500, 3, 80), (5, 1, 8, 50)]


@pytest.mark.parametrize("case", FC_CASES)
@pytest.mark.parametrize("mi", range(len(MODES)))
def test_fc_matches_oracle(case, mi):
    n_in, n_out, B, L = case
    rng = np.random.default_rng(7 + 100 * mi + n_out)
    layer = FCLayer(name="f", n_in=n_in, n_out=n_out, init_k=1.0,
                    max_out_spikes=int(rng.choice([L * n_out, 5])))
    bits = [8, 16, 32][mi % 3]
    vk = ["scalar", "channel", "none"][mi % 3]
    params, rm = _params(rng, layer.weight_shape, n_out, n_out, MODES[mi], bits, vk)
    times, src, n_real = _events(rng, B, L, n_in)
    print("fc case", case, "mode", MODES[mi], "bits", bits, "vth", vk, flush=True)
    out = run_layer(layer, params, times, src, n_real, round_mode=rm)
    geom, prm, cap = oracle_spec(layer, params, rm)
    ref = O.layer_forward(geom, prm, times, src, n_real, cap)
    assert_layer_equal(out, ref, tag=str(case))



@pytest.mark.parametrize("bits", [8, 16, 32])
def test_fc_readouts_without_threshold_match_oracle(bits):
    """FC layers with no threshold (v_th None, the readout variant: full chunks of 64
    events unrolled, weights loaded first): weights of every width, from LDS (a small
    slice) and from global memory (a wide one, or two waves per stream), streams that
    end on a chunk boundary, inside one and that are empty, wrap and saturate with
    values pushed past the register range."""
    for mi, (n_in, n_out, B, L) in enumerate([(300, 10, 5, 64 * 5), (2312, 64, 3, 64 * 3 + 17),
                                              (37, 128, 4, 150), (1568, 10, 4, 64 * 2 + 1)]):
        rng = np.random.default_rng(5100 + 10 * bits + mi)
        layer = FCLayer(name="f", n_in=n_in, n_out=n_out, init_k=1.0, max_out_spikes=16)
        mode = MODES[(mi + bits // 8) % len(MODES)]
        params, rm = _params(rng, layer.weight_shape, n_out, n_out, mode, bits, "none")
        times, src, n_real = _events(rng, B, L, n_in)
        n_real[0], n_real[-1] = L, 0
        if B > 2:
            n_real[1] = 64
        print("fc readout", bits, (n_in, n_out, B, L), mode, flush=True)
        out = run_layer(layer, params, times, src, n_real, round_mode=rm)
        geom, prm, cap = oracle_spec(layer, params, rm)
        ref = O.layer_forward(geom, prm, times, src, n_real, cap)
        assert int(ref["out_n"].max()) == 0
        assert_layer_equal(out, ref, tag=f"readout {bits} {n_out}")


@pytest.mark.parametrize("waves", ["1", "2", "4"])
def test_fc_waves_per_stream_match_oracle(waves, monkeypatch):
    """Dense firing (thresholds of a few units) with the neurons of a stream on 1, 2 or 4
    waves (SALT_FC_WAVES): the waves' spikes merged per event in neuron order, a capacity
    cut inside a chunk, and, with one wave, slices of 1024 neurons writing spike masks."""
    monkeypatch.setenv("SALT_FC_WAVES", waves)
    for mi, (n_in, n_out, B, L) in enumerate([(37, 10, 6, 300), (64, 130, 4, 200), (100, 300, 4, 150),
                                              (50, 1024, 3, 130), (200, 1500, 2, 100)]):
        rng = np.random.default_rng(4400 + 10 * mi + int(waves))
        for cap in (L * n_out, 1 + L * n_out // 7):
            layer = FCLayer(name="f", n_in=n_in, n_out=n_out, init_k=1.0, max_out_spikes=cap)
            params, rm = _params(rng, layer.weight_shape, n_out, n_out, MODES[mi], [8, 16, 32][mi % 3],
                                 "scalar")
            params = params._replace(v_th_int=np.int32(rng.integers(1, 8)))
            times, src, n_real = _events(rng, B, L, n_in)
            print("fc waves", waves, (n_in, n_out, B, L), "cap", cap, flush=True)
            out = run_layer(layer, params, times, src, n_real, round_mode=rm)
            geom, prm, ocap = oracle_spec(layer, params, rm)
            ref = O.layer_forward(geom, prm, times, src, n_real, ocap)
            assert int(ref["out_n"].sum()) > 64 * B, "the case must fire densely"
            if n_out >= 300:  # chunks of more than two spikes per event: the dense placement
                assert (ref["out_n"] / np.maximum(n_real, 1)).max() > 2
            assert_layer_equal(out, ref, tag=f"waves {waves} {n_out} {cap}")

@pytest.mark.parametrize("spw", [2, 3, 4, 5])
def test_conv_streams_per_work_group_match_oracle(spw, monkeypatch):
    """Channel-slot kernel, several streams per work-group (forced through SALT_CONV_SPW): streams of different
    lengths, an empty one, and a last work-group with slots past the batch (B = 7, 11)
    give the oracle's streams, registers and extremes."""
    monkeypatch.setenv("SALT_CONV_PACKED", "0")  # the channel-slot kernel
    monkeypatch.setenv("SALT_CONV_SPW", str(spw))
    for mi, case in enumerate([(2, 34, 34, 16, 5, 2, 0, 7, 400), (16, 15, 15, 32, 3, 2, 0, 11, 400),
                               (2, 10, 10, 2, 3, 1, 0, 11, 200)]):
        ic, h, w, oc, k, s, p, B, L = case
        rng = np.random.default_rng(300 + 10 * spw + mi)
        layer = ConvLayer(name="c", ic=ic, h_in=h, w_in=w, oc=oc, k=k, s=s, p=p, init_k=1.0,
                          max_queue_len=int(rng.choice([L + 1, max(2, L // 20)])),
                          max_out_spikes=int(rng.choice([4 * L * oc, 9])))
        params, rm = _params(rng, layer.weight_shape, layer.n_neurons, oc, MODES[mi], 8,
                             ["scalar", "channel", "neuron"][mi])
        times, src, n_real = _events(rng, B, L, ic * h * w)
        n_real[3] = L // 7  # a short stream beside full ones
        print("spw", spw, "case", case, "n_real", n_real.tolist(), flush=True)
        out = run_layer(layer, params, times, src, n_real, round_mode=rm)
        geom, prm, cap = oracle_spec(layer, params, rm)
        ref = O.layer_forward(geom, prm, times, src, n_real, cap)
        assert_layer_equal(out, ref, tag=f"spw {spw} {case}")


def _clustered_sources(rng, B, L, ic, h, w, patch):
    """Sources in a few patch x patch squares, visited in bursts, so that consecutive
    events share, overlap or miss each other's candidate blocks in runs of every length."""
    src = np.zeros((B, L), np.int32)
    for b in range(B):
        i = 0
        while i < L:
            n = int(rng.integers(1, 12))
            y0, x0 = rng.integers(0, h - patch + 1), rng.integers(0, w - patch + 1)
            y = y0 + rng.integers(0, patch, n)
            x = x0 + rng.integers(0, patch, n)
            c = rng.integers(0, ic, n)
            src[b, i:i + n] = (c * h * w + y * w + x)[:L - i]
            i += n
    return src


@pytest.mark.parametrize("pair", ["0", "1"])
def test_conv_one_and_two_events_per_step_match_oracle(pair, monkeypatch):
    """Steps of one event and of two (forced through SALT_CONV_PAIR): uniform and
    clustered sources, whole-plane, sub-band and row-band plans, truncated and untruncated
    queues give the oracle's streams, registers and extremes."""
    monkeypatch.setenv("SALT_CONV_PACKED", "0")  # the channel-slot kernel
    monkeypatch.setenv("SALT_CONV_PAIR", pair)
    cases = [((2, 34, 34, 16, 5, 2, 0, 6, 500), None, False), ((2, 34, 34, 16, 5, 2, 0, 6, 500), None, True),
             ((16, 15, 15, 32, 3, 2, 0, 6, 400), None, True), ((2, 12, 12, 8, 3, 1, 1, 5, 300), "2,2", True),
             ((1, 130, 130, 4, 3, 1, 0, 3, 600), None, True), ((3, 20, 20, 6, 4, 2, 1, 5, 300), None, False)]
    for mi, (case, plan, clustered) in enumerate(cases):
        ic, h, w, oc, k, s, p, B, L = case
        if plan:
            monkeypatch.setenv("SALT_CONV_PLAN", plan)
        else:
            monkeypatch.delenv("SALT_CONV_PLAN", raising=False)
        rng = np.random.default_rng(700 + 10 * int(pair) + mi)
        layer = ConvLayer(name="c", ic=ic, h_in=h, w_in=w, oc=oc, k=k, s=s, p=p, init_k=1.0,
                          max_queue_len=int(rng.choice([L + 1, max(2, L // 25)])),
                          max_out_spikes=4 * L * oc)
        params, rm = _params(rng, layer.weight_shape, layer.n_neurons, oc, MODES[mi % 5], 8,
                             ["scalar", "channel", "neuron"][mi % 3])
        times, src, n_real = _events(rng, B, L, ic * h * w)
        if clustered:
            src = _clustered_sources(rng, B, L, ic, h, w, 2 * k)
        print("pair", pair, "case", case, "plan", plan, "clustered", clustered, flush=True)
        out = run_layer(layer, params, times, src, n_real, round_mode=rm)
        geom, prm, cap = oracle_spec(layer, params, rm)
        ref = O.layer_forward(geom, prm, times, src, n_real, cap)
        assert_layer_equal(out, ref, tag=f"pair {pair} {case} {plan} {clustered}")


@pytest.mark.parametrize("hwalk", ["0", "1"])
def test_conv_spikes_placed_by_the_helper_or_by_each_group_match_oracle(hwalk, monkeypatch):
    """Whole-plane plans whose spikes the helper wave places for every channel group, or
    each channel-group wave its own (forced through SALT_CONV_HWALK): one and two events
    per step, one to eight channel groups, sub-bands, dense firing, a capacity cut and an
    empty stream give the oracle's streams, registers and extremes."""
    monkeypatch.setenv("SALT_CONV_PACKED", "0")  # the channel-slot kernel
    monkeypatch.setenv("SALT_CONV_HWALK", hwalk)
    cases = [((2, 34, 34, 16, 5, 2, 0, 5, 500), "0", None), ((16, 15, 15, 32, 3, 2, 0, 5, 400), "0", None),
             ((2, 34, 34, 16, 5, 1, 0, 3, 300), "1", None), ((2, 12, 12, 8, 3, 1, 1, 5, 300), "0", "2,2"),
             ((4, 12, 12, 40, 5, 1, 2, 3, 200), "0", None)]  # 7 groups of 3 iterations
    for mi, (case, pair, plan) in enumerate(cases):
        ic, h, w, oc, k, s, p, B, L = case
        monkeypatch.setenv("SALT_CONV_PAIR", pair)
        if plan:
            monkeypatch.setenv("SALT_CONV_PLAN", plan)
        else:
            monkeypatch.delenv("SALT_CONV_PLAN", raising=False)
        rng = np.random.default_rng(1300 + 10 * int(hwalk) + mi)
        layer = ConvLayer(name="c", ic=ic, h_in=h, w_in=w, oc=oc, k=k, s=s, p=p, init_k=1.0,
                          max_queue_len=L + 1,
                          max_out_spikes=int(rng.choice([4 * L * oc, 50])))
        params, rm = _params(rng, layer.weight_shape, layer.n_neurons, oc, MODES[mi % 5], 8,
                             ["scalar", "channel", "neuron"][mi % 3])
        times, src, n_real = _events(rng, B, L, ic * h * w)
        src = _clustered_sources(rng, B, L, ic, h, w, 2 * k)
        n_real[1] = 0  # an empty stream
        print("hwalk", hwalk, "case", case, "pair", pair, "plan", plan, flush=True)
        out = run_layer(layer, params, times, src, n_real, round_mode=rm)
        geom, prm, cap = oracle_spec(layer, params, rm)
        ref = O.layer_forward(geom, prm, times, src, n_real, cap)
        assert int(ref["out_n"].sum()) > 0, "the case must fire"
        assert_layer_equal(out, ref, tag=f"hwalk {hwalk} {case} {pair} {plan}")


@pytest.mark.parametrize("pair", ["0", "1"])
def test_conv_many_iterations_per_step_match_oracle(pair, monkeypatch):
    """One channel group per stream (SALT_CONV_PLAN=1,1) puts every channel in one wave:
    3 iterations per event for conv1's geometry (8 with two-event steps) and 2 for
    conv2's (4 with two-event steps), clustered sources."""
    monkeypatch.setenv("SALT_CONV_PACKED", "0")  # the channel-slot kernel
    monkeypatch.setenv("SALT_CONV_PAIR", pair)
    monkeypatch.setenv("SALT_CONV_PLAN", "1,1")
    for mi, case in enumerate([(2, 34, 34, 16, 5, 2, 0, 5, 400), (16, 15, 15, 32, 3, 2, 0, 5, 400)]):
        ic, h, w, oc, k, s, p, B, L = case
        rng = np.random.default_rng(1100 + 10 * int(pair) + mi)
        layer = ConvLayer(name="c", ic=ic, h_in=h, w_in=w, oc=oc, k=k, s=s, p=p, init_k=1.0,
                          max_queue_len=int(rng.choice([L + 1, max(2, L // 25)])),
                          max_out_spikes=4 * L * oc)
        params, rm = _params(rng, layer.weight_shape, layer.n_neurons, oc, MODES[2 * mi], 8,
                             ["neuron", "channel"][mi])
        times, src, n_real = _events(rng, B, L, ic * h * w)
        src = _clustered_sources(rng, B, L, ic, h, w, 2 * k)
        print("iterations pair", pair, "case", case, flush=True)
        out = run_layer(layer, params, times, src, n_real, round_mode=rm)
        geom, prm, cap = oracle_spec(layer, params, rm)
        ref = O.layer_forward(geom, prm, times, src, n_real, cap)
        assert_layer_equal(out, ref, tag=f"iterations pair {pair} {case}")


@pytest.mark.parametrize("lists", ["0", "1"])
def test_conv_row_bands_with_and_without_event_lists(lists, monkeypatch):
    """Row-band plans (planes above the LDS size) whose work-groups decode their band's
    event list, or the whole stream (SALT_CONV_BANDLIST=0): same streams, registers and
    extremes as the oracle, for stride 1 and for stride 2 with padding (events meeting
    two bands), uniform and clustered sources, and streams longer than one segment of
    the list build (1024 events)."""
    monkeypatch.setenv("SALT_CONV_BANDLIST", lists)
    for mi, (case, clustered) in enumerate([((1, 130, 130, 4, 3, 1, 0, 3, 700), False),
                                            ((2, 200, 200, 4, 5, 2, 2, 3, 600), True),
                                            ((1, 130, 130, 4, 3, 1, 0, 2, 3500), True)]):
        ic, h, w, oc, k, s, p, B, L = case
        rng = np.random.default_rng(1300 + 10 * int(lists) + mi)
        layer = ConvLayer(name="c", ic=ic, h_in=h, w_in=w, oc=oc, k=k, s=s, p=p, init_k=1.0,
                          max_queue_len=int(rng.choice([L + 1, max(2, L // 25)])),
                          max_out_spikes=4 * L * oc)
        params, rm = _params(rng, layer.weight_shape, layer.n_neurons, oc, MODES[mi + 1], 8,
                             ["channel", "neuron", "scalar"][mi])
        times, src, n_real = _events(rng, B, L, ic * h * w)
        if clustered:
            src = _clustered_sources(rng, B, L, ic, h, w, 3 * k)
        print("band lists", lists, "case", case, flush=True)
        out = run_layer(layer, params, times, src, n_real, round_mode=rm)
        geom, prm, cap = oracle_spec(layer, params, rm)
        ref = O.layer_forward(geom, prm, times, src, n_real, cap)
        assert_layer_equal(out, ref, tag=f"band lists {lists} {case}")


def test_without_neuron_extremes_same_streams_and_registers():
    rng = np.random.default_rng(5)
    layer = ConvLayer(name="c", ic=2, h_in=34, w_in=34, oc=16, k=5, s=2, p=0, init_k=1.0,
                      max_queue_len=500, max_out_spikes=4000)
    params, rm = _params(rng, layer.weight_shape, layer.n_neurons, 16, MODES[0], 8, "scalar")
    times, src, n_real = _events(rng, 8, 400, 2 * 34 * 34)
    a = run_layer(layer, params, times, src, n_real, round_mode=rm, extremes=True)
    b = run_layer(layer, params, times, src, n_real, round_mode=rm, extremes=False)
    assert b.result.v_unfitted_min is None
    for x, y in [(a.stream.event_times, b.stream.event_times), (a.stream.event_source_idx, b.stream.event_source_idx),
                 (a.result.v_final, b.result.v_final), (a.result.stream_stats, b.result.stream_stats)]:
        assert bool((x == y).all())


def test_repeat_runs_are_bitwise_identical():
    """Determinism: spike order never depends on atomics or scheduling."""
    rng = np.random.default_rng(9)
    layer = ConvLayer(name="c", ic=1, h_in=130, w_in=130, oc=4, k=3, s=1, p=0, init_k=1.0,
                      max_queue_len=900, max_out_spikes=20000)
    params, rm = _params(rng, layer.weight_shape, layer.n_neurons, 4, MODES[0], 8, "scalar")
    times, src, n_real = _events(rng, 4, 800, 130 * 130)
    a = run_layer(layer, params, times, src, n_real, round_mode=rm)
    b = run_layer(layer, params, times, src, n_real, round_mode=rm)
    assert bool((a.stream.event_source_idx == b.stream.event_source_idx).all())
    assert bool((a.result.v_final == b.result.v_final).all())


@pytest.mark.parametrize("plan", ["1,2", "1,3", "2,2", "1,8"])
def test_conv_work_group_shapes_match_oracle(plan, monkeypatch):
    """Every work-group shape the planner can choose (channel groups x row sub-bands,
    forced through SALT_CONV_PLAN) gives the oracle's streams, registers and extremes."""
    monkeypatch.setenv("SALT_CONV_PACKED", "0")  # the channel-slot kernel
    monkeypatch.setenv("SALT_CONV_PLAN", plan)
    for mi, case in enumerate([(2, 34, 34, 16, 5, 2, 0, 8, 400), (16, 15, 15, 32, 3, 2, 0, 8, 400),
                               (2, 12, 12, 8, 3, 1, 1, 8, 300)]):
        ic, h, w, oc, k, s, p, B, L = case
        rng = np.random.default_rng(77 + mi)
        layer = ConvLayer(name="c", ic=ic, h_in=h, w_in=w, oc=oc, k=k, s=s, p=p, init_k=1.0,
                          max_queue_len=int(rng.choice([L + 1, max(2, L // 20)])),
                          max_out_spikes=4 * L * oc)
        params, rm = _params(rng, layer.weight_shape, layer.n_neurons, oc, MODES[mi], 8,
                             ["scalar", "neuron", "channel"][mi])
        times, src, n_real = _events(rng, B, L, ic * h * w)
        print("plan", plan, "case", case, flush=True)
        out = run_layer(layer, params, times, src, n_real, round_mode=rm)
        geom, prm, cap = oracle_spec(layer, params, rm)
        ref = O.layer_forward(geom, prm, times, src, n_real, cap)
        assert_layer_equal(out, ref, tag=f"{plan} {case}")


PACK_CASES = [
    # (ic, h, w, oc, k, s, p, B, L)
    (2, 34, 34, 16, 5, 2, 0, 7, 500),      # conv1 of the N-MNIST network: classes up to 3x3
    (16, 15, 15, 32, 3, 2, 0, 7, 400),     # conv2: classes up to 2x2, 32 channels
    (2, 20, 20, 6, 5, 1, 2, 5, 300),       # stride 1, padding: classes up to 5x5
    (3, 9, 11, 5, 4, 3, 2, 7, 200),        # stride 3 > k / 2, odd plane
    (1, 7, 7, 3, 1, 2, 0, 6, 120),         # k < s: pixels that reach no neuron
    (2, 12, 12, 40, 3, 1, 1, 5, 200),      # many channels: several iterations at 3x3
]


@pytest.mark.parametrize("shape", ["1,1", "1,3", "1,4", "2,1", "2,2", "2,3", "3,1", "4,2", "8,1"])
def test_conv_packed_shapes_match_oracle(shape, monkeypatch):
    """The packed conv kernel (valid candidates packed per class of candidate rectangle)
    with its channel groups x streams per work-group forced through SALT_CONV_PACK:
    uniform and clustered sources, truncated and untruncated queues, every threshold kind,
    both overflow modes, a short and an empty stream, and a last work-group with slots past
    the batch give the oracle's streams, registers and extremes."""
    monkeypatch.setenv("SALT_CONV_PACK", shape)
    for mi, case in enumerate(PACK_CASES):
        ic, h, w, oc, k, s, p, B, L = case
        rng = np.random.default_rng(2100 + 17 * mi + int(shape[0]) * 3 + int(shape[-1]))
        layer = ConvLayer(name="c", ic=ic, h_in=h, w_in=w, oc=oc, k=k, s=s, p=p, init_k=1.0,
                          max_queue_len=int(rng.choice([L + 1, max(2, L // 25)])),
                          max_out_spikes=int(rng.choice([4 * L * oc, 11])))
        params, rm = _params(rng, layer.weight_shape, layer.n_neurons, oc, MODES[mi % 5],
                             [8, 16, 32][mi % 3], ["scalar", "channel", "neuron", "none"][mi % 4])
        times, src, n_real = _events(rng, B, L, ic * h * w)
        n_real[2] = L // 9
        if mi % 2:
            src = _clustered_sources(rng, B, L, ic, h, w, 2 * k)
        print("packed", shape, "case", case, "mql", layer.max_queue_len, "cap", layer.max_out_spikes,
              flush=True)
        out = run_layer(layer, params, times, src, n_real, round_mode=rm)
        geom, prm, cap = oracle_spec(layer, params, rm)
        ref = O.layer_forward(geom, prm, times, src, n_real, cap)
        assert_layer_equal(out, ref, tag=f"packed {shape} {case}")
