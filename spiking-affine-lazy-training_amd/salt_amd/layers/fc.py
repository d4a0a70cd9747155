"""FCLayer / FCSpec / fc: the fully connected layer of salt_core/layers/fc.py with the same
fields.  forward runs the integer event-driven kernel through QuantBackend."""
import math
from collections.abc import Mapping
from dataclasses import dataclass, field, replace
from typing import Any, ClassVar

from salt_amd.capacity import Capacity
from salt_amd.layers.base import LayerOutput, check_leading_axis


@dataclass(frozen=True)
class FCLayer:
    """salt_core/layers/fc.py:23-135."""
    name: str
    n_in: int
    n_out: int
    init_k: float
    tau: float = 16.0
    v_th: float = 1.0
    alpha: float = 2.0
    chunk_size: int = 1
    max_out_spikes: int = 8192
    max_extra_steps: int = 0

    @property
    def n_neurons(self) -> int:
        return self.n_out

    @property
    def input_shape(self) -> tuple[int, ...]:
        return (self.n_in,)

    @property
    def output_shape(self) -> tuple[int, ...]:
        return (self.n_out,)

    @property
    def fan_in(self) -> int:
        return self.n_in

    @property
    def weight_shape(self) -> tuple[int, ...]:
        return (self.n_out, self.n_in)

    @property
    def capacity(self) -> Capacity:
        return Capacity(max_out_spikes=self.max_out_spikes, max_extra_steps=self.max_extra_steps)

    def with_capacity(self, capacity: Capacity) -> "FCLayer":
        return replace(self, **capacity)

    def with_chunk_size(self, chunk_size: int) -> "FCLayer":
        """New chunk_size, max_extra_steps unchanged (salt_core/layers/fc.py:130-136)."""
        return replace(self, chunk_size=chunk_size)

    def unflatten_neurons(self, values):
        check_leading_axis(values, self.n_out, "n_out")
        return values.reshape(self.n_out, 1, 1, *values.shape[1:])

    def broadcast_channels(self, values):
        check_leading_axis(values, self.n_out, "n_out")
        return values

    def forward(self, params, in_stream, *, backend=None, trace: bool = False) -> LayerOutput:
        """Integer forward of this layer over a (batched) EventStream."""
        from salt_amd.quant.backend import resolve_backend
        be = resolve_backend(backend)
        out = be.layer_forward(self, params, in_stream)
        if trace:
            out = out._replace(trace=be.layer_trace(self, params, in_stream))
        return out


@dataclass(frozen=True)
class FCSpec:
    """FCLayer without n_in, completed by Network.build (salt_core/layers/fc.py:139-154)."""
    n_out: int
    name: str | None = None
    options: Mapping[str, Any] = field(default_factory=dict)
    name_prefix: ClassVar[str] = "fc"

    def build(self, input_shape: tuple[int, ...], name: str) -> FCLayer:
        return FCLayer(name=name, n_in=math.prod(input_shape), n_out=self.n_out, **self.options)


def fc(n_out: int, *, name: str | None = None, **options: Any) -> FCSpec:
    """salt_core/layers/fc.py:157-158."""
    return FCSpec(n_out=n_out, name=name, options=options)
