// Device-side building blocks shared by the layer kernels of libsalt_hip.so
// (gfx950, 64-lane wavefronts).  The fixed-point helpers restate
// salt_core/quant/fixed_point.py and salt_core/quant/codes.py of the reference.
#pragma once

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "salt_hip.h"

namespace salt {

constexpr int kWave = 64;
// Events per compaction segment: spike masks become a stream segment by segment, so that
// a stream's walk and its padding spread over many waves.
constexpr int kCompactSeg = 2048;
constexpr float kPadTime = 1e12f;  // salt_core/stream.py:13

// MI355X hands the work-groups of a launch to its 8 XCDs in turn (linear id i to XCD
// i % 8), and each XCD has an L2 of its own.  xcd_order(i, n) renumbers the n work-groups
// so that each XCD runs one contiguous range of the new numbers: work-groups that read the
// same data (the row bands of one stream) then fetch it into one L2 instead of eight.  A
// bijection on [0, n); results never depend on it.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_order(int i, int n) {
  const int q = n / kXcds, r = n - q * kXcds;
  const int x = i % kXcds, k = i / kXcds;
  return x * q + min(x, r) + k;
}

// Quantisation parameters of one layer, uniform over the launch.
struct Quant {
  int fa;        // shift_bits of the decay multiply (f_a)
  int fV;        // fractional bits of the register (f_V)
  int wbits;     // register width i_V + f_V
  int rc;        // rounding constant: 2^(f_a-1) for round, 0 for truncate
  int half;      // 2^(wbits-1)
  int n_table;   // decay table entries (dt = 1 .. n_table)
  int vth_kind;  // SALT_VTH_*
  int vth_scalar;
  const int32_t* vth;
};

// Decay multiply D = A*(V >> f_a) + ((A*(V & (2^f_a-1)) + c) >> f_a), which is the
// split multiply of salt_core/quant/fixed_point.py:47-65 (bit-identical to
// (A*V + c) >> f_a with an exact product).  A < 2^15 and the low part < 2^15, so the
// low product is a 24-bit unsigned multiply-add; F24: the high part fits 24 bits too.
// (The trace kernel's form; the layer kernels use decay_mul_wide.)
template <bool F24>
__device__ __forceinline__ int32_t decay_mul(int32_t v, int32_t a, int fa, int rc) {
  const int32_t hi = v >> fa;
  const uint32_t lo = (uint32_t)v & ((1u << fa) - 1u);
  const int32_t t2 = (int32_t)((__umul24((uint32_t)a, lo) + (uint32_t)rc) >> fa);
  return F24 ? __mul24(a, hi) + t2 : a * hi + t2;
}

// The same value as one 64-bit multiply-add: V*A = hi*A*2^f_a + lo*A, so
// (V*A + c) >> f_a = hi*A + ((lo*A + c) >> f_a) exactly; |V| < 2^29 and A <= 2^f_a keep
// the product in 64 bits and the result in 32.  Two instructions on gfx950
// (v_mad_i64_i32 and a 64-bit shift) against six for the split form, which pays off in
// every layer loop (measured on MI355X: conv, the firing FC and the readout).
__device__ __forceinline__ int32_t decay_mul_wide(int32_t v, int32_t a, int fa, int rc) {
  return (int32_t)(((int64_t)v * a + rc) >> fa);
}

// Write-back into the (i_V + f_V)-bit register, salt_core/quant/fixed_point.py:68-90:
// saturate clamps, wrap keeps the low wbits bits sign-extended.
template <bool SAT>
__device__ __forceinline__ int32_t fit_bits(int32_t u, const Quant& qz) {
  if (SAT) return min(max(u, -qz.half), qz.half - 1);
  return __builtin_amdgcn_sbfe(u, 0, qz.wbits);
}

// Extended decay table in LDS: [0] = 2^f_a (dt = 0, the identity column, which the
// decay multiply maps to V exactly), [1..n] = decay_table_int, [n+1] = 0 (dt > n).
// Index = min(dt, n + 1): salt_core/quant/codes.py:87-105.
__device__ __forceinline__ void load_ext_table(int32_t* ext, const int32_t* table,
                                               int n_table, int fa, int lane, int nthreads) {
  for (int i = lane; i < n_table + 2; i += nthreads)
    ext[i] = i == 0 ? (1 << fa) : (i <= n_table ? table[i - 1] : 0);
}

// Times are float32 holding integer ms in [0, 2^31) (checked on the host); the unsigned
// conversion is exact up to 2^32, so even a time rounded up to 2^31 by the float32 cast
// keeps its value.  Differences are taken in 32-bit wrap-around arithmetic and read as
// unsigned: for non-decreasing times that is the exact gap, which equals the reference's
// float32 difference wherever the gap selects a table entry (gaps up to 2^21 are exact
// in float32 differences of such times).  Spike times go back to float through
// ms_time().
__device__ __forceinline__ int time_ms(float t) { return (int)(uint32_t)t; }
__device__ __forceinline__ float ms_time(int t) { return (float)(uint32_t)t; }

// Extended-table index of a gap: 0 (identity), 1..n (table), n + 1 (decay to 0).
__device__ __forceinline__ int decay_slot(int dt, int n_table) {
  return (int)min((uint32_t)dt, (uint32_t)n_table + 1u);
}

__device__ __forceinline__ int floordiv_pos(int a, int s) {  // s > 0
  return a >= 0 ? a / s : -((-a + s - 1) / s);
}

// n / d for 0 <= n < 2^22 and d >= 1, with rcp = 1 / d as float (within one ulp): the
// float product is within one of n / d, so its truncation is the quotient or one off,
// and one integer correction either way makes it exact.  A few instructions against a
// generic 32-bit division's two dozen.
__host__ __device__ inline int div_small(int n, int d, float rcp) {
  int q = (int)((float)n * rcp);
  const int r = n - q * d;
  q += r >= d ? 1 : 0;
  q -= r < 0 ? 1 : 0;
  return q;
}

__device__ __forceinline__ int wave_min(int v) {
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ int wave_max(int v) {
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
  return v;
}

// Inclusive prefix sum over the 64 lanes with DPP (no LDS round trip): Hillis-Steele
// within each row of 16 lanes (row_shr 1, 2, 4, 8), then row 0's total into row 1 and
// row 2's into row 3 (row_bcast:15), then rows 0-1's total into rows 2-3 (row_bcast:31).
// Lanes without a source, and rows outside the row mask, add 0.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

// Number of set bits of m below this lane (v_mbcnt).
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// v_writelane, which this compiler exposes as an LLVM intrinsic but not as a builtin:
// lane `lane` of the result <- the wave-uniform `v`, other lanes <- `old`.  (The compiler
// puts the lane select in M0, since a VALU instruction reads one scalar operand here.)
extern "C" __device__ int salt_writelane_i32(int v, int lane, int old) __asm(
    "llvm.amdgcn.writelane.i32");

// lo/hi of lane e <- the wave-uniform 64-bit value v; other lanes keep theirs.  The value
// comes straight from the compare's scalar result and the lane from the scalar loop
// counter, so no scalar instruction waits for a vector one.
__device__ __forceinline__ void stage_to_lane(uint32_t& lo, uint32_t& hi, uint64_t v, int e) {
  lo = (uint32_t)salt_writelane_i32((int)(uint32_t)v, e, (int)lo);
  hi = (uint32_t)salt_writelane_i32((int)(uint32_t)(v >> 32), e, (int)hi);
}
// The low half alone (slices of 32 neurons or fewer).
__device__ __forceinline__ void stage_to_lane_lo(uint32_t& lo, uint64_t v, int e) {
  lo = (uint32_t)salt_writelane_i32((int)(uint32_t)v, e, (int)lo);
}

__device__ __forceinline__ int rdlane(int v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}

__device__ __forceinline__ int32_t load_code_bits(const void* p, size_t i, int bits) {
  if (bits == 8) return (int32_t) static_cast<const int8_t*>(p)[i];
  if (bits == 16) return (int32_t) static_cast<const int16_t*>(p)[i];
  return static_cast<const int32_t*>(p)[i];
}

}  // namespace salt
