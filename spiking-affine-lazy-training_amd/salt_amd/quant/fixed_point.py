"""Fixed-point conventions of the integer path (host side): rounding and overflow
modes and the width limits, as salt_core/quant/fixed_point.py:15-29 defines them.
The arithmetic itself runs in the HIP kernels (libsalt_hip.so)."""
import enum

# The low product a*lo has up to 2*shift_bits bits plus the half-step (fixed_point.py:15).
MAX_SHIFT_BITS = 15
# Register value plus one weight contribution must fit int32 (fixed_point.py:17).
MAX_REGISTER_BITS = 30


class RoundMode(str, enum.Enum):
    """Rounding after the decay multiply (fixed_point.py:20-23); strings accepted."""
    ROUND = "round"
    TRUNCATE = "truncate"


class OverflowMode(str, enum.Enum):
    """Register write-back when out of range (fixed_point.py:26-29); strings accepted."""
    WRAP = "wrap"
    SATURATE = "saturate"


def check_shift_bits(shift_bits: int) -> None:
    """ValueError as wide_mul_shift raises it (fixed_point.py:57-60)."""
    if shift_bits > MAX_SHIFT_BITS:
        raise ValueError(f"shift_bits={shift_bits} 超過 {MAX_SHIFT_BITS},低位乘積"
                         f"(2*shift_bits 位元)會溢位 int32 (shift_bits above MAX_SHIFT_BITS)")
    if shift_bits < 0:
        raise ValueError(f"shift_bits={shift_bits} is negative")


def check_total_bits(total_bits: int) -> None:
    """ValueError as fit_to_bits raises it (fixed_point.py:79-82)."""
    if total_bits > MAX_REGISTER_BITS:
        raise ValueError(f"total_bits={total_bits} 超過 {MAX_REGISTER_BITS},暫存器值加上"
                         "權重貢獻之後可能溢位 int32 (total_bits above MAX_REGISTER_BITS)")
    if total_bits < 1:
        raise ValueError(f"total_bits={total_bits} below 1")
