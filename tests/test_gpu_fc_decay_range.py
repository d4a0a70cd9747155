"""FC layers on the GPU against the CPU oracle with event gaps that cover the whole decay
table: every gap 0 (identity), 1..n (each table entry) and above n (decay to 0), a first
event later than the table (its gap is measured from t = 0), and times that cross 2^24 ms,
where float32 holds only even integers.  Modes cover wrap and saturate with the high part
of the decay multiply within 24 bits (i_V + f_V - f_a = 24) and beyond (25).
References: salt_core/quant/codes.py:87-105 (three decay regimes),
salt_core/connectivity/fc.py:20-33 (gap to the previous real event, the first against 0),
salt_core/stream.py:24-46 (output order)."""
import numpy as np
import pytest

from salt_amd import FCLayer, QuantizedLayerParams
from salt_amd.quant.codes import build_decay_table_int
from oracle import oracle as O
from helpers import assert_layer_equal, oracle_spec
from gpu_util import run_layer

pytestmark = pytest.mark.gpu

# (round_mode, overflow_mode, f_a, f_V, i_V, tau): i_V + f_V - f_a = 24 or 25
MODES = [("round", "wrap", 5, 0, 29, 12.0), ("truncate", "wrap", 4, 1, 28, 20.0),
         ("round", "saturate", 5, 1, 28, 20.0), ("truncate", "saturate", 4, 2, 27, 12.0),
         ("round", "wrap", 10, 0, 24, 20.0)]

# (n_in, n_out): weights in LDS with one wave per stream, two waves reading global memory,
# eight-neuron-per-lane slices, and a layer wide enough for spike masks + compaction
SHAPES = [(40, 64), (2312, 200), (30, 1000), (64, 4500)]


def gap_stream(rng, n_table, t0, extra):
    """Integer gaps holding every value 0 .. 2 n_table + 5 once (shuffled), `extra` more
    drawn from {0, 1 .. n_table, long}; times = t0 + cumsum(gaps) as float32."""
    gaps = rng.permutation(np.arange(2 * n_table + 6))
    more = np.where(rng.random(extra) < 0.3, 0,
                    np.where(rng.random(extra) < 0.8, rng.integers(1, n_table + 1, extra),
                             rng.integers(n_table + 1, 10 ** 6, extra)))
    gaps = np.concatenate([gaps, more])
    return (t0 + np.cumsum(gaps)).astype(np.float32)


def float32_gaps(times, n_real):
    """The gaps the reference computes: float32 differences, the first against 0."""
    out = []
    for t, n in zip(times, n_real):
        r = t[:n].astype(np.float32)
        out.append(np.diff(np.concatenate([[np.float32(0)], r])).astype(np.float32))
    return np.concatenate(out)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("mi", range(len(MODES)))
def test_fc_gaps_span_the_decay_table(shape, mi):
    rm, om, fa, fV, iV, tau = MODES[mi]
    n_in, n_out = shape
    rng = np.random.default_rng(5100 + 37 * mi + n_out)
    table = build_decay_table_int(fa, tau)
    n = len(table)
    L = 2 * n + 6 + 120
    # stream 0: starts at 0; 1: first event after the table; 2: crosses 2^24 ms;
    # 3: entirely above 2^24 ms, with pads; 4: first gap inside the table, with pads
    starts = [0, n + 37, 2 ** 24 - (L * n) // 3, 2 ** 24 + 11, int(rng.integers(1, n + 1))]
    times = np.stack([gap_stream(rng, n, t0, L - (2 * n + 6)) for t0 in starts])
    n_real = np.full(len(starts), L, np.int32)
    n_real[3], n_real[4] = L - 17, L - 40
    for b in (3, 4):
        times[b, n_real[b]:] = 1e12
    src = rng.integers(0, n_in, times.shape).astype(np.int32)

    # register values that reach the top bits, so the high multiply needs its full width
    w = iV + fV
    q_lim = min(2 ** 30 >> fV, 2 ** (w - 2) >> fV)
    q = rng.integers(-q_lim // 4, q_lim // 4 + 1, (n_out, n_in)).astype(np.int32)
    vth = rng.integers(2 ** (w - 3), 2 ** (w - 1), n_out).astype(np.int32)
    vth[::3] = 2 ** (w - 1) - 1  # some neurons keep their value long
    # two neurons step by a quarter of the register per event: within a few events of
    # short gaps they reach the top quarter and wrap or saturate
    q[0], q[1] = q_lim, -q_lim
    vth[0] = vth[1] = 2 ** (w - 1) - 1
    params = QuantizedLayerParams(q=q, decay_table_int=table, v_th_int=vth, scale=np.float32(1.0),
                                  f_a=fa, f_V=fV, i_V=iV, overflow_mode=om)
    layer = FCLayer(name="f", n_in=n_in, n_out=n_out, init_k=1.0, max_out_spikes=L * n_out)

    g = float32_gaps(times, n_real)
    assert set(range(n + 1)) <= set(int(x) for x in g if x <= n), "every table index is used"
    assert (g > n).sum() >= n, "gaps beyond the table (decay code 0)"
    assert times[2, 0] < 2 ** 24 < times[2, L - 1] and times[3, 0] > 2 ** 24

    print("fc decay range", shape, MODES[mi], "table", n, "L", L, flush=True)
    out = run_layer(layer, params, times, src, n_real, round_mode=rm)
    geom, prm, cap = oracle_spec(layer, params, rm)
    ref = O.layer_forward(geom, prm, times, src, n_real, cap)
    assert_layer_equal(out, ref, tag=f"{shape} {MODES[mi]}")
    # values in the register's top quarter: with i_V + f_V - f_a = 25 their high part
    # (V >> f_a) needs more than 24 bits
    top = max(np.abs(out.result.v_unfitted_max.cpu().numpy()).max(),
              np.abs(out.result.v_unfitted_min.cpu().numpy().astype(np.int64)).max())
    assert top >= 2 ** (w - 2)
