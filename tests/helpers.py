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
