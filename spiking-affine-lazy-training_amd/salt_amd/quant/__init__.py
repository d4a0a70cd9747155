"""The integer backend (salt_core/quant) on the GPU."""
from salt_amd.quant.backend import QUANT, QuantBackend, QuantLayerResult
from salt_amd.quant.codes import build_decay_table_int, delta_t_max
from salt_amd.quant.fixed_point import (MAX_REGISTER_BITS, MAX_SHIFT_BITS, OverflowMode,
                                        RoundMode)
from salt_amd.quant.params import QuantizedLayerParams

__all__ = ["QUANT", "QuantBackend", "QuantLayerResult", "QuantizedLayerParams", "RoundMode",
           "OverflowMode", "MAX_SHIFT_BITS", "MAX_REGISTER_BITS", "build_decay_table_int",
           "delta_t_max"]
