"""The CPU oracle against the reference's own known-answer vectors (transcribed in
tests/golden/reference_literals.json with file:line citations)."""
import math

import numpy as np
import pytest

from oracle import oracle as O
from oracle import queue_ref as Q


def test_round_shift_literals(golden):
    for case in golden["round_shift"]:
        got = [O.round_shift(x, case["shift"], case["mode"]) for x in case["x"]]
        assert got == case["want"], case["cite"]
        got_q = Q.round_shift(np.array(case["x"]), case["shift"], case["mode"]).tolist()
        assert got_q == case["want"], case["cite"]


def test_wide_mul_shift_literals(golden):
    for case in golden["wide_mul_shift"]:
        assert O.wide_mul_shift(case["a"], case["v"], case["shift"], case["mode"]) == case["want"], case["cite"]
        assert int(Q.wide_mul_shift(case["a"], case["v"], case["shift"], case["mode"])) == case["want"]


def test_fit_to_bits_literals(golden):
    for case in golden["fit_to_bits"]:
        for x, want, ovf in zip(case["x"], case["want"], case["ovf"]):
            assert O.fit_to_bits(x, case["bits"], case["mode"]) == (want, ovf), case["cite"]


def test_process_event_literals(golden):
    for c in golden["process_event"]:
        r = O.process_event(c["v0"], c["a"], c["ident"], c["q"], c["v_th"], f_a=c["f_a"],
                            f_V=c["f_V"], i_V=c["i_V"], round_mode=c["round"],
                            overflow_mode=c["overflow"])
        if "want_v" in c:
            assert r["v_final"] == c["want_v"], c["cite"]
        if "want_spike" in c:
            assert r["is_spiked"] == c["want_spike"], c["cite"]
        if "want_ovf" in c:
            assert r["overflowed"] == c["want_ovf"], c["cite"]
        if "want_unfitted" in c:
            assert r["v_unfitted"] == c["want_unfitted"], c["cite"]


def test_run_layer_literals_queue_formulation(golden):
    """The literal queue restatement (scan over columns) reproduces the reference's
    hand-computed chains."""
    for c in golden["run_layer"]:
        r = Q.run_layer(np.array(c["a"], np.int32), np.array(c["ident"]), np.array(c["q"], np.int32),
                        np.array(c["v_th"]), f_a=c["f_a"], f_V=c["f_V"], i_V=c["i_V"])
        assert r["v_final"].tolist() == c["want_v_final"], c["cite"]
        if "want_spike_any" in c:
            assert r["spike_mask"].any(axis=1).tolist() == c["want_spike_any"], c["cite"]
        if "want_ovf_any" in c:
            assert r["overflowed"].any(axis=1).tolist() == c["want_ovf_any"], c["cite"]
        if "want_vmax" in c:
            assert r["v_unfitted_max"].tolist() == c["want_vmax"], c["cite"]
            assert r["v_unfitted_min"].tolist() == c["want_vmin"], c["cite"]


def test_decay_lookup_literals(golden):
    from salt_amd.quant.codes import build_decay_table_int
    for c in golden["decay_lookup"]:
        table = build_decay_table_int(c["f_a"], c["tau"])
        got = [O.decay_lookup(dt, table) for dt in c["dt"]]
        assert [g[1] for g in got] == c["ident"], c["cite"]
        assert [g[0] for g in got][1:] == c["a_from_index_1"], c["cite"]
        a_q, id_q = Q.apply_decay_table_int(np.array(c["dt"], np.float32), table)
        assert id_q.tolist() == c["ident"] and a_q[1:].tolist() == c["a_from_index_1"]


def _layer_case(c):
    if c["kind"] == "fc":
        geom = dict(kind="fc", n_in=c["n_in"], n_out=c["n_out"])
    else:
        geom = {k: c[k] for k in ("ic", "h_in", "w_in", "oc", "k", "s", "p", "max_queue_len")}
        geom["kind"] = "conv"
    from salt_amd.quant.codes import build_decay_table_int
    params = dict(q=np.array(c["q"]), table=build_decay_table_int(c["f_a"], c["tau"]),
                  v_th=c["v_th"], f_a=c["f_a"], f_V=c["f_V"], i_V=c["i_V"],
                  round_mode="round", overflow_mode=c.get("overflow", "wrap"))
    return geom, params


@pytest.mark.parametrize("section", ["layers", "stream_order"])
def test_layer_literals(golden, section):
    for c in golden[section]:
        geom, params = _layer_case(c)
        r = O.layer_forward(geom, params, np.array([c["times"]], np.float32),
                            np.array([c["src"]], np.int32), np.array([c["n_real"]]),
                            c["max_out_spikes"])
        if "want_v_final" in c:
            assert r["v_final"][0].tolist() == c["want_v_final"], c["cite"]
        if "want_n" in c:
            assert int(r["out_n"][0]) == c["want_n"], c["cite"]
        if "want_out_src" in c:
            n = len(c["want_out_src"])
            assert r["out_src"][0, :n].tolist() == c["want_out_src"], c["cite"]
        if "want_out_times" in c:
            n = len(c["want_out_times"])
            assert r["out_times"][0, :n].tolist() == c["want_out_times"], c["cite"]
        if "want_needed_queue" in c:
            assert int(r["needed_queue"][0]) == c["want_needed_queue"], c["cite"]


def test_decay_table_literals(golden):
    from salt_amd.quant.codes import build_decay_table_int, delta_t_max
    for c in golden["decay_table"]:
        t = build_decay_table_int(c["f_a"], c["tau"])
        assert t.dtype == np.int32
        assert t[:len(c["prefix"])].tolist() == c["prefix"], c["cite"]
        assert t.shape == (delta_t_max(c["f_a"], c["tau"]),)
        if "length" in c:
            assert t.shape[0] == c["length"] and int(t[-1]) == c["last"], c["cite"]
    t = build_decay_table_int(8, 16.0)  # salt_core/tests/test_quant_codes.py:77-81
    assert t.min() >= 0 and t.max() <= 255 and np.all(np.diff(t) <= 0)


def test_delta_t_max_boundary(golden):
    """salt_core/tests/test_quant_codes.py:49-58: the boundary definition itself."""
    from salt_amd.quant.codes import delta_t_max
    for f_a, tau in golden["delta_t_max_boundary"]["cases"]:
        d = delta_t_max(f_a, tau)
        eps = 2.0 ** -(f_a + 1)
        base = 1.0 - 1.0 / tau
        assert base ** d >= eps and base ** (d + 1) < eps
