"""Capacity knobs and growth (salt_amd.capacity), with the worked examples of
salt_core/tests/test_capacity_fit.py.  CPU only."""
import numpy as np
import pytest
import torch

from salt_amd import ConvLayer, FCLayer
from salt_amd.capacity import (Capacity, GrowthPolicy, LayerDiag, grown_to_fit,
                               grown_to_fit_batch, reduce_over_batch, shrunk_to_observed)
from salt_amd.quant_run import grown_for_needed

CONV = ConvLayer(name="conv", ic=1, h_in=4, w_in=4, oc=1, k=3, s=1, p=1, init_k=1.0, chunk_size=4,
                 max_queue_len=10, max_out_spikes=20, max_extra_steps=10)
CONV2 = ConvLayer(name="conv2", ic=1, h_in=4, w_in=4, oc=1, k=3, s=1, p=1, init_k=1.0,
                  chunk_size=4, max_queue_len=10, max_out_spikes=20, max_extra_steps=10)
FC = FCLayer(name="out", n_in=16, n_out=2, init_k=1.0)
POLICIES = {"conv": GrowthPolicy(), "conv2": GrowthPolicy(), "out": GrowthPolicy()}


def _diag(queue, out_spikes, steps, spike_count=(0, 0, 0)):
    return LayerDiag(spike_count=torch.tensor(spike_count, dtype=torch.float32),
                     firing_rate=torch.zeros(3),
                     needed={"max_queue_len": torch.tensor(queue),
                             "max_out_spikes": torch.tensor(out_spikes),
                             "max_extra_steps": torch.tensor(steps)})


def _fc_diag(out_spikes=(0, 0, 0)):
    return LayerDiag(spike_count=torch.zeros(3), firing_rate=torch.zeros(3),
                     needed={"max_out_spikes": torch.tensor(out_spikes),
                             "max_extra_steps": torch.zeros(3, dtype=torch.int64)})


def _needed(queue, out_spikes, steps):
    return {"max_queue_len": queue, "max_out_spikes": out_spikes, "max_extra_steps": steps}


def test_reduce_over_batch():
    r = reduce_over_batch(_diag([3, 9, 5], [1, 2, 7], [4, 4, 6], spike_count=[100, 200, 300]))
    assert {k: int(v) for k, v in r.needed.items()} == _needed(9, 7, 6)
    assert float(r.spike_count) == 200.0


def test_capacities_and_replace():
    assert dict(CONV.capacity) == _needed(10, 20, 10)
    grown = CONV.with_capacity(CONV.capacity.replace(max_queue_len=30))
    assert (grown.max_queue_len, grown.max_out_spikes, grown.max_extra_steps) == (30, 20, 10)
    assert dict(FC.capacity) == {"max_out_spikes": 8192, "max_extra_steps": 0}
    with pytest.raises(KeyError):
        CONV.capacity.replace(queue=5)


def test_fits_checks_every_knob_per_sample():
    fits = CONV.capacity.fits(_diag([10, 11, 3], [20, 1, 1], [10, 2, 12]))
    assert fits.tolist() == [True, False, False]


def test_everything_fits_returns_the_same_list():
    layers = [CONV, FC]
    assert grown_to_fit_batch(layers, POLICIES, [_diag([10, 3, 3], [20, 1, 1], [10, 2, 2]),
                                                 _fc_diag()]) is layers


def test_one_overflowing_sample_grows_the_layer():
    # ceil(11 * 1.5) = 17; max_extra_steps -> 17 - ceil(17 / 4) = 12
    grown = grown_to_fit_batch([CONV, FC], POLICIES, [_diag([2, 11, 2], [1, 1, 1], [1, 1, 1]),
                                                      _fc_diag()])
    assert (grown[0].max_queue_len, grown[0].max_out_spikes, grown[0].max_extra_steps) == (17, 20, 12)
    assert grown[1] is FC


def test_only_the_overflowing_layer_grows():
    # conv2: ceil(15 * 1.5) = 23, extra steps 23 - ceil(23 / 4) = 17
    grown = grown_to_fit_batch([CONV, CONV2, FC], POLICIES,
                               [_diag([2, 3, 2], [1, 1, 1], [1, 1, 1]),
                                _diag([2, 15, 2], [1, 1, 1], [1, 1, 1]), _fc_diag()])
    assert grown[0] is CONV and grown[2] is FC
    assert dict(grown[1].capacity) == _needed(23, 20, 17)


def test_two_layers_grow_in_one_call():
    grown = grown_to_fit_batch([CONV, CONV2, FC], POLICIES,
                               [_diag([12, 3, 2], [1, 1, 1], [1, 1, 1]),
                                _diag([2, 3, 2], [1, 25, 1], [1, 1, 1]), _fc_diag()])
    assert dict(grown[0].capacity) == _needed(18, 20, 13)
    assert dict(grown[1].capacity) == _needed(10, 38, 10)


def test_policy_grown_and_shrunk():
    cap = Capacity(max_queue_len=100, max_out_spikes=2000, max_extra_steps=100)
    assert GrowthPolicy().grown(cap, _needed(50, 10, 100), chunk_size=4) == cap
    assert dict(GrowthPolicy().grown(cap, _needed(777, 10, 0), chunk_size=4)) == _needed(1166, 2000, 874)
    g = GrowthPolicy(max_extra_steps_grow_factor=2.0).grown(cap, _needed(50, 10, 107), chunk_size=4)
    assert dict(g) == _needed(100, 2000, 214)
    assert dict(GrowthPolicy().shrunk(cap, _needed(10, 600, 40))) == _needed(100, 900, 100)
    assert GrowthPolicy().shrunk(cap, _needed(0, 0, 40))["max_out_spikes"] == 1


def test_grown_to_fit_changes_only_capacity_fields():
    diag = LayerDiag(spike_count=0, firing_rate=0.0, needed=_needed(11, 1, 1))
    [grown] = grown_to_fit([CONV], POLICIES, [diag])
    assert grown is not CONV and grown == CONV.with_capacity(grown.capacity)
    assert grown.max_queue_len == 17


def test_shrunk_to_observed_returns_same_list_when_nothing_shrinks():
    layers = [CONV, FC]
    observed = {"conv": _needed(10, 20, 10), "out": {"max_out_spikes": 8192, "max_extra_steps": 0}}
    assert shrunk_to_observed(layers, POLICIES, observed) is layers


def test_with_chunk_size():
    conv = ConvLayer(name="conv", ic=1, h_in=4, w_in=4, oc=1, k=3, s=1, p=1, init_k=1.0,
                     chunk_size=4, max_queue_len=30, max_out_spikes=20, max_extra_steps=3)
    two = conv.with_chunk_size(2)
    assert (two.chunk_size, two.max_extra_steps, two.max_queue_len) == (2, 15, 30)
    assert FC.with_chunk_size(3) == FCLayer(name="out", n_in=16, n_out=2, init_k=1.0, chunk_size=3)


def test_grown_for_needed_uses_the_largest_need_over_all_samples():
    needed = {"conv": _needed(np.array([3, 12, 5]), np.array([1, 2, 3]), np.zeros(3, int)),
              "out": {"max_out_spikes": np.array([0, 9000, 1]), "max_extra_steps": np.zeros(3, int)}}
    grown = grown_for_needed([CONV, FC], POLICIES, needed)
    assert dict(grown[0].capacity) == _needed(18, 20, 13)
    assert grown[1].max_out_spikes == 13500
