"""Overflow analysis on the GPU, with the properties example/tests/test_quant_run.py checks
on a trained model, here on a synthetic N-MNIST-shaped model with narrowed registers:
narrowing makes registers overflow; widening leaves samples without overflow bit-exact;
min_extra_bits removes every overflow and each layer's count is the least that does;
headroom is negative exactly for overflowing layers; overflow_events point at overflowed
samples and layers.  Also batched = per-sample (salt_core/tests/test_network.py:79-96)."""
import numpy as np
import pytest
import torch

from salt_amd import QuantBackend
from salt_amd.capacity import GrowthPolicy
from salt_amd.decoder import MembraneRegressionDecoder
from salt_amd.network import InputEvents
from salt_amd.quant_run import (MAX_OVERFLOW_EVENTS, headroom_bits, min_extra_bits,
                                overflow_events, quant_forward_split, reference_arrays,
                                with_extra_i_V)
from test_gpu_model_folder import _net, _raw

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
SHRINK = 6
BATCH = 6


@pytest.fixture(scope="module")
def setup():
    net, params = _net(mql=160)
    raw = _raw(21, 18)
    dec = MembraneRegressionDecoder()
    narrow = with_extra_i_V(params, [-SHRINK] * len(params))
    print("overflow analysis: base and narrowed runs", flush=True)
    out = quant_forward_split(net, dec, params, "round", raw, BATCH, device=DEV)
    narrow_out = quant_forward_split(net, dec, narrow, "round", raw, BATCH, device=DEV)
    policies = {l.name: GrowthPolicy() for l in net.layers}
    return dict(net=net, params=params, raw=raw, dec=dec, narrow=narrow, out=out,
                narrow_out=narrow_out, policies=policies)


def test_narrowed_registers_overflow(setup):
    assert setup["narrow_out"].overflowed.any()
    assert setup["narrow_out"].overflowed.sum() > setup["out"].overflowed.sum()


def test_wider_i_V_keeps_samples_without_overflow(setup):
    wide = quant_forward_split(setup["net"], setup["dec"],
                               with_extra_i_V(setup["params"], [3] * 3), "round", setup["raw"],
                               BATCH, device=DEV)
    clean = ~setup["out"].overflowed.any(axis=1)
    assert clean.any()
    for key, value in reference_arrays(setup["out"]).items():
        np.testing.assert_array_equal(getattr(wide, key)[clean], value[clean], err_msg=key)


def test_min_extra_bits_removes_all_overflow_and_is_minimal(setup):
    print("min_extra_bits", flush=True)
    extra, rounds = min_extra_bits(setup["net"], setup["dec"], setup["narrow"], "round",
                                   setup["raw"], BATCH, setup["policies"], setup["narrow_out"],
                                   device=DEV)
    fixed = quant_forward_split(setup["net"], setup["dec"], with_extra_i_V(setup["narrow"], extra),
                                "round", setup["raw"], BATCH, device=DEV)
    assert rounds >= 1 and all(e >= 0 for e in extra)
    assert not fixed.overflowed.any()
    for i, e in enumerate(extra):
        if e == 0:
            continue
        one_less = list(extra)
        one_less[i] -= 1
        again = quant_forward_split(setup["net"], setup["dec"],
                                    with_extra_i_V(setup["narrow"], one_less), "round",
                                    setup["raw"], BATCH, device=DEV)
        assert again.overflowed.any(), f"layer {i}"


def test_headroom_negative_exactly_for_overflowed_layers(setup):
    headroom = headroom_bits(setup["narrow"], setup["narrow_out"])
    for h, ov in zip(headroom, setup["narrow_out"].overflowed.any(axis=0)):
        assert (h is not None and h < 0) == bool(ov)


def test_overflow_events_point_at_overflowed_samples_and_layers(setup):
    print("overflow_events", flush=True)
    events = overflow_events(setup["net"], setup["narrow"], "round", setup["raw"],
                             setup["narrow_out"])
    names = [l.name for l in setup["net"].layers]
    assert 0 < len(events) <= MAX_OVERFLOW_EVENTS
    for ev in events:
        assert setup["narrow_out"].overflowed[ev["sample"], names.index(ev["layer"])]
        low, high = ev["register_range"]
        assert ev["true_min"] < low or ev["true_max"] > high
        assert ev["v_after"] == 0 if ev["spiked"] else low <= ev["v_after"] <= high


def test_batched_equals_per_sample(setup):
    net, params, raw = setup["net"], setup["params"], setup["raw"]
    be = QuantBackend("round")
    batched = net.apply_batched(params, raw, backend=be)
    for i in (0, 5, 17):
        one = InputEvents(*(np.asarray(a)[i] for a in raw))
        single = net.apply(params, one, backend=be)
        for rb, rs in zip(batched.results, single.results):
            assert torch.equal(rb.v_final[i], rs.v_final)
            assert torch.equal(rb.v_unfitted_min[i], rs.v_unfitted_min)
            assert torch.equal(rb.spike_count[i], rs.spike_count)
        assert bool(batched.fits[i]) == bool(single.fits)
