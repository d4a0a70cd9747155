"""QuantizedLayerParams: one layer's integer parameters, the same fields as
salt_core/quant/params.py:9-21.  Arrays may be numpy arrays or torch tensors."""
from typing import Any, NamedTuple

from salt_amd.quant.fixed_point import OverflowMode


class QuantizedLayerParams(NamedTuple):
    q: Any                 # integer weight codes, shape = layer.weight_shape
    decay_table_int: Any   # build_decay_table_int(f_a, layer.tau), dt = 1..n
    v_th_int: Any          # scalar or (n_neurons,) integer threshold; None = never fires
    scale: Any             # per-neuron weight step s_c, used only by readout
    f_a: int               # fraction bits of the decay code
    f_V: int               # fraction bits of the register
    i_V: int               # integer bits of the register (incl. sign)
    overflow_mode: OverflowMode | str = OverflowMode.WRAP
