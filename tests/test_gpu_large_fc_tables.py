"""FC weight tables above 2^31 bytes: the rows an event reads lie past any 32-bit signed
byte offset, in each of the kernel's weight-row address forms (scalar row base for slices
of four or more words per lane, a per-lane 64-bit address for narrow slices, the sliced
layout that writes spike masks).

An FC layer's result depends on its weights only through the rows (transposed: columns
of q) of the sources its events name (salt_core/connectivity/fc.py:20-61: every event
adds column q[:, s] to every neuron).  So the oracle runs a layer of just those columns,
with each source renamed to its column's place, and must match the GPU run on the full
table bit for bit.  The table is int32 (values beyond int16, so the codes stay 32-bit):
about 540 M codes, 2.16 GB, zero outside the columns used."""
import numpy as np
import pytest

from salt_amd import FCLayer, QuantizedLayerParams
from salt_amd.quant.codes import build_decay_table_int
from oracle import oracle as O
from helpers import assert_layer_equal, oracle_spec
from gpu_util import run_layer

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_in,n_out,form", [
    (524291, 1030, "scalar row base, 3 waves of 8 words per lane"),
    (128000, 4200, "sliced: 5 slices of 16 words per lane, spike masks"),
    (5400007, 100, "narrow: 2 waves of 1 word per lane, per-lane address"),
])
def test_fc_table_above_2gib_matches_oracle_on_the_columns_used(n_in, n_out, form):
    assert n_in * n_out * 4 > 2 ** 31
    rng = np.random.default_rng(n_in % 1000 + n_out)
    used = np.unique(np.concatenate([[0, n_in - 1, n_in - 2, n_in // 2],
                                     rng.integers(0, n_in, 36)])).astype(np.int64)
    q = np.zeros((n_out, n_in), np.int32)
    cols = rng.integers(-70000, 70001, (n_out, used.size))
    for j, c in enumerate(used):  # column by column: a fancy-index store is far slower here
        q[:, c] = cols[:, j]
    q[0, used[-1]] = 70000  # beyond int16: 32-bit codes
    B, L = 3, 200
    pick = rng.integers(0, used.size, (B, L))
    pick[0, :used.size] = np.arange(used.size)  # every column used, the last row included
    times = np.zeros((B, L), np.float32)
    n_real = np.array([L, L // 2, 0], np.int32)
    for b in range(B):
        gaps = np.where(rng.random(L) < 0.25, 0, rng.integers(1, 6, L))
        times[b] = np.cumsum(gaps)
        times[b, n_real[b]:] = 1e12
    cap = L * n_out
    params = QuantizedLayerParams(q=q, decay_table_int=build_decay_table_int(10, 12.0),
                                  v_th_int=np.int32(40000), scale=np.float32(1.0),
                                  f_a=10, f_V=0, i_V=24, overflow_mode="wrap")
    layer = FCLayer(name="f", n_in=n_in, n_out=n_out, init_k=1.0, max_out_spikes=cap)
    print("fc table", (n_in, n_out), form, "bytes", n_in * n_out * 4, flush=True)
    out = run_layer(layer, params, times, used[pick].astype(np.int32), n_real, round_mode="round")
    small = FCLayer(name="f", n_in=used.size, n_out=n_out, init_k=1.0, max_out_spikes=cap)
    sparams = params._replace(q=np.ascontiguousarray(q[:, used]))
    del q, params
    geom, prm, ocap = oracle_spec(small, sparams, "round")
    ref = O.layer_forward(geom, prm, times, pick.astype(np.int32), n_real, ocap)
    assert int(ref["out_n"].sum()) > 10 * L, "the case must fire"
    # the GPU names sources of the full table; the oracle names columns of the small one
    assert_layer_equal(out, ref, tag=f"table {n_in}x{n_out}")
