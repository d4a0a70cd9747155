"""salt_amd: the integer event-by-event forward pass of salt_core/quant on MI355X.

The Python side mirrors the reference's host API (EventStream, InputEvents, Network,
ConvLayer/FCLayer, QuantizedLayerParams, QuantBackend); all event processing runs in
hand-written gfx950 kernels in libsalt_hip.so, reached through the C-ABI of
include/salt_hip.h.
"""
from salt_amd.capacity import Capacity, LayerDiag
from salt_amd.layers import ConvLayer, ConvSpec, FCLayer, FCSpec, LayerOutput, conv, fc
from salt_amd.network import InputEvents, Network, NetworkOutput, run_network
from salt_amd.quant import (QUANT, OverflowMode, QuantBackend, QuantizedLayerParams,
                            QuantLayerResult, RoundMode, build_decay_table_int, delta_t_max)
from salt_amd.stream import PAD_TIME, EventStream

__all__ = ["Capacity", "LayerDiag", "ConvLayer", "ConvSpec", "FCLayer", "FCSpec", "LayerOutput",
           "conv", "fc", "InputEvents", "Network", "NetworkOutput", "run_network", "QUANT",
           "OverflowMode", "QuantBackend", "QuantizedLayerParams", "QuantLayerResult",
           "RoundMode", "build_decay_table_int", "delta_t_max", "PAD_TIME", "EventStream"]
