"""ConvLayer / ConvSpec / conv: the conv layer of salt_core/layers/conv.py with the same
fields, geometry and neuron numbering (oc*h_out*w_out + y*w_out + x).  forward runs the
integer event-driven kernel through QuantBackend."""
from collections.abc import Mapping
from dataclasses import dataclass, field, replace
from typing import Any, ClassVar

from salt_amd.capacity import Capacity
from salt_amd.layers.base import LayerOutput, check_leading_axis, safe_extra_steps


@dataclass(frozen=True)
class ConvLayer:
    """salt_core/layers/conv.py:22-187.  h_out = (h_in + 2p - k) // s + 1."""
    name: str
    ic: int
    h_in: int
    w_in: int
    oc: int
    k: int
    s: int
    p: int
    init_k: float
    tau: float = 16.0
    v_th: float = 1.0
    alpha: float = 2.0
    chunk_size: int = 1
    max_queue_len: int = 128
    max_out_spikes: int = 8192
    max_extra_steps: int | None = None

    def __post_init__(self) -> None:
        if self.h_out < 1 or self.w_out < 1:
            raise ValueError(
                f"{self.name} 幾何退化:輸入 {self.h_in}x{self.w_in}、k={self.k} s={self.s} "
                f"p={self.p} -> 輸出 {self.h_out}x{self.w_out}")
        if self.max_extra_steps is None:
            object.__setattr__(self, "max_extra_steps",
                               safe_extra_steps(self.max_queue_len, self.chunk_size))

    @property
    def h_out(self) -> int:
        return (self.h_in + 2 * self.p - self.k) // self.s + 1

    @property
    def w_out(self) -> int:
        return (self.w_in + 2 * self.p - self.k) // self.s + 1

    @property
    def n_neurons(self) -> int:
        return self.oc * self.h_out * self.w_out

    @property
    def input_shape(self) -> tuple[int, ...]:
        return (self.ic, self.h_in, self.w_in)

    @property
    def output_shape(self) -> tuple[int, ...]:
        return (self.oc, self.h_out, self.w_out)

    @property
    def fan_in(self) -> int:
        return self.ic * self.k * self.k

    @property
    def weight_shape(self) -> tuple[int, ...]:
        return (self.oc, self.ic, self.k, self.k)

    @property
    def capacity(self) -> Capacity:
        return Capacity(max_queue_len=self.max_queue_len, max_out_spikes=self.max_out_spikes,
                        max_extra_steps=self.max_extra_steps)

    def with_capacity(self, capacity: Capacity) -> "ConvLayer":
        return replace(self, **capacity)

    def with_chunk_size(self, chunk_size: int) -> "ConvLayer":
        """New chunk_size with max_extra_steps reset to the value that always suffices
        (salt_core/layers/conv.py:179-186)."""
        return replace(self, chunk_size=chunk_size,
                       max_extra_steps=safe_extra_steps(self.max_queue_len, chunk_size))

    def unflatten_neurons(self, values):
        """(n_neurons, ...) -> (oc, h_out, w_out, ...) (salt_core/layers/conv.py:104-112)."""
        check_leading_axis(values, self.n_neurons, "n_neurons")
        return values.reshape(self.oc, self.h_out, self.w_out, *values.shape[1:])

    def broadcast_channels(self, values):
        """(oc, ...) -> (n_neurons, ...) (salt_core/layers/conv.py:114-122)."""
        check_leading_axis(values, self.oc, "oc")
        return values.repeat(self.h_out * self.w_out, axis=0)

    def forward(self, params, in_stream, *, backend=None, trace: bool = False) -> LayerOutput:
        """Integer forward of this layer over a (batched) EventStream."""
        from salt_amd.quant.backend import resolve_backend
        be = resolve_backend(backend)
        out = be.layer_forward(self, params, in_stream)
        if trace:
            out = out._replace(trace=be.layer_trace(self, params, in_stream))
        return out


@dataclass(frozen=True)
class ConvSpec:
    """ConvLayer without its input plane, completed by Network.build
    (salt_core/layers/conv.py:189-211)."""
    oc: int
    k: int
    s: int
    p: int
    name: str | None = None
    options: Mapping[str, Any] = field(default_factory=dict)
    name_prefix: ClassVar[str] = "conv"

    def build(self, input_shape: tuple[int, ...], name: str) -> ConvLayer:
        if len(input_shape) != 3:
            raise ValueError(f"{name}:conv 要空間輸入 (C, H, W),前一層的輸出是攤平的 {input_shape}")
        ic, h_in, w_in = input_shape
        return ConvLayer(name=name, ic=ic, h_in=h_in, w_in=w_in, oc=self.oc, k=self.k, s=self.s,
                         p=self.p, **self.options)


def conv(oc: int, k: int, s: int, p: int, *, name: str | None = None, **options: Any) -> ConvSpec:
    """salt_core/layers/conv.py:214-216."""
    return ConvSpec(oc=oc, k=k, s=s, p=p, name=name, options=options)
