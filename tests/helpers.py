"""Shared test helpers: product layers/params -> oracle specs, GPU runs, comparisons."""
import numpy as np

from oracle import oracle as O


def oracle_spec(layer, params, round_mode="round"):
    """(geom, params, cap) for oracle.layer_forward from a salt_amd layer + params."""
    if hasattr(layer, "oc"):
        geom = dict(kind="conv", ic=layer.ic, h_in=layer.h_in, w_in=layer.w_in, oc=layer.oc,
                    k=layer.k, s=layer.s, p=layer.p, max_queue_len=layer.max_queue_len)
    else:
        geom = dict(kind="fc", n_in=layer.n_in, n_out=layer.n_out)
    v_th = params.v_th_int
    if v_th is not None:
        v_th = np.broadcast_to(np.asarray(v_th).astype(np.int64).astype(np.int32),
                               (layer.n_neurons,))
    p = dict(q=np.asarray(params.q), table=np.asarray(params.decay_table_int), v_th=v_th,
             f_a=params.f_a, f_V=params.f_V, i_V=params.i_V, round_mode=str(getattr(round_mode, "value", round_mode)),
             overflow_mode=str(getattr(params.overflow_mode, "value", params.overflow_mode)))
    return geom, p, layer.max_out_spikes


def oracle_network(network, params, events, round_mode="round", nthreads=0):
    specs = [oracle_spec(l, p, round_mode) for l, p in zip(network.layers, params)]
    return O.network_forward(specs, events.event_times, events.source_idx,
                             events.n_real_events, nthreads=nthreads)


def assert_layer_equal(gpu_out, ref, *, extremes=True, tag=""):
    """Bit-exact comparison of one layer's GPU LayerOutput (batched) against the oracle."""
    n = gpu_out.stream.n_real_events.cpu().numpy()
    np.testing.assert_array_equal(n, ref["out_n"], err_msg=f"{tag} spike counts")
    cap = ref["out_times"].shape[1]
    np.testing.assert_array_equal(gpu_out.stream.event_source_idx.cpu().numpy()[:, :cap],
                                  ref["out_src"], err_msg=f"{tag} spike sources")
    np.testing.assert_array_equal(gpu_out.stream.event_times.cpu().numpy()[:, :cap],
                                  ref["out_times"], err_msg=f"{tag} spike times")
    r = gpu_out.result
    np.testing.assert_array_equal(r.v_final.cpu().numpy(), ref["v_final"], err_msg=f"{tag} v_final")
    if extremes:
        np.testing.assert_array_equal(r.v_unfitted_min.cpu().numpy(), ref["v_min"], err_msg=f"{tag} v_min")
        np.testing.assert_array_equal(r.v_unfitted_max.cpu().numpy(), ref["v_max"], err_msg=f"{tag} v_max")
    st = r.stream_stats.cpu().numpy()
    np.testing.assert_array_equal(st[:, 0], ref["v_min"].min(axis=1), err_msg=f"{tag} stream vmin")
    np.testing.assert_array_equal(st[:, 1], ref["v_max"].max(axis=1), err_msg=f"{tag} stream vmax")
    if "needed_queue" in ref and st[:, 2].any():
        np.testing.assert_array_equal(st[:, 2], ref["needed_queue"], err_msg=f"{tag} needed queue")


def encode_aer(x, y, c, t_us) -> bytes:
    """Events -> N-MNIST 40-bit AER bytes (x, y, polarity<<7 | t[22:16], t[15:8], t[7:0]),
    built byte by byte with Python integers."""
    out = bytearray()
    for xi, yi, ci, ti in zip(x, y, c, t_us):
        xi, yi, ci, ti = int(xi), int(yi), int(ci), int(ti)
        assert 0 <= ti < 1 << 23 and ci in (0, 1)
        out += bytes([xi, yi, (ci << 7) | (ti >> 16), (ti >> 8) & 0xFF, ti & 0xFF])
    return bytes(out)


def write_nmnist_tree(root, per_digit_train=6, per_digit_test=3, seed=0, n_range=(40, 160)):
    """A small N-MNIST-shaped tree: root/{Train,Test}/<digit>/<five digits>.bin with random
    events (sorted microsecond times).  Returns {path: (x, y, c, t_us)}."""
    import os
    rng = np.random.default_rng(seed)
    files = {}
    for split, per in (("Train", per_digit_train), ("Test", per_digit_test)):
        for d in range(10):
            os.makedirs(os.path.join(root, split, str(d)), exist_ok=True)
            for k in range(per):
                n = int(rng.integers(*n_range))
                x, y = rng.integers(0, 34, n), rng.integers(0, 34, n)
                c = rng.integers(0, 2, n)
                t = np.sort(rng.integers(0, 300_000, n))
                path = os.path.join(root, split, str(d), f"{k * 7 + d:05d}.bin")
                with open(path, "wb") as f:
                    f.write(encode_aer(x, y, c, t))
                files[path] = (x, y, c, t)
    return files
