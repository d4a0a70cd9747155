"""Shared layer pieces: LayerOutput and the shape checks of salt_core/layers/base.py."""
from typing import Any, NamedTuple


class LayerOutput(NamedTuple):
    """One layer's forward output (salt_core/layers/base.py:65-70)."""
    stream: Any   # EventStream fed to the next layer
    result: Any   # QuantLayerResult
    diag: Any     # LayerDiag
    trace: Any    # LayerForwardTrace when forward ran with trace=True, else None


def base_scan_steps(queue_len: int, chunk_size: int) -> int:
    """ceil(queue_len / chunk_size) (salt_core/float/affine.py:73-75); kept so that the
    capacity knobs of a layer match the reference's."""
    return -(-queue_len // chunk_size)


def safe_extra_steps(queue_len: int, chunk_size: int) -> int:
    """salt_core/float/affine.py:78-80."""
    return queue_len - base_scan_steps(queue_len, chunk_size)


def check_leading_axis(values, expected: int, what: str) -> None:
    """salt_core/layers/base.py:82-85."""
    if values.ndim == 0 or values.shape[0] != expected:
        raise ValueError(f"第 0 軸長度要等於 {what}={expected},拿到的形狀是 {values.shape}")
