// Launchers of the layer kernels.  Each kernel family is instantiated in its own
// translation unit (conv_inst.hip once per iteration count, fc_inst.hip once per
// weight width) so that the build compiles them in parallel.
#pragma once

#include "conv_kernel.hpp"
#include "conv_packed.hpp"
#include "fc_kernel.hpp"

namespace salt {

constexpr int kLdsMax = 160 * 1024;  // gfx950 LDS per workgroup

// Conv flags: bit 5 = two events per step (needs bit 3), bit 4 = no queue truncation
// possible (max_queue_len >= stream length), bit 3 = candidate masks fit 32 bits,
// bit 2 = saturate, bit 1 = per-neuron extremes, bit 0 = per-neuron thresholds.
enum : int {
  kConvPair = 32, kConvNoTrunc = 16, kConvM32 = 8, kConvSat = 4, kConvExt = 2, kConvVthN = 1
};
constexpr int kConvFlagCombos = 64;

// Iteration counts with an instantiated kernel family.
#define SALT_CONV_NITS(X) X(1) X(2) X(3) X(4) X(8)
#define SALT_DECLARE_CONV(N)                                                           \
  hipError_t launch_conv_nit##N(const ConvArgs& a, int flags, dim3 grid, dim3 block,   \
                                size_t lds, hipStream_t st);
SALT_CONV_NITS(SALT_DECLARE_CONV)
#undef SALT_DECLARE_CONV

// Packed conv flags: bit 3 = no queue truncation possible, bit 2 = threshold array (per
// channel or per neuron), bit 1 = per-neuron extremes, bit 0 = saturate.
enum : int { kPackNoTrunc = 8, kPackVtha = 4, kPackExt = 2, kPackSat = 1 };
constexpr int kPackFlagCombos = 16;

// Iteration bounds with an instantiated packed kernel family.
#define SALT_PACK_IMAXES(X) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8)
#define SALT_DECLARE_PACK(N)                                                           \
  hipError_t launch_pack_imax##N(const PackArgs& a, int flags, dim3 grid, dim3 block,  \
                                 size_t lds, hipStream_t st);
SALT_PACK_IMAXES(SALT_DECLARE_PACK)
#undef SALT_DECLARE_PACK

// FC flags: bit 2 = no threshold (a readout), bit 1 = saturate, bit 0 = weights in LDS.
enum : int { kFcNoFire = 4, kFcSat = 2, kFcWlds = 1 };

#define SALT_DECLARE_FC(B)                                                             \
  hipError_t launch_fc_q##B(const FcArgs& a, int npl, int flags, dim3 grid, int waves, \
                            size_t lds, hipStream_t st);
SALT_DECLARE_FC(8)
SALT_DECLARE_FC(16)
SALT_DECLARE_FC(32)
#undef SALT_DECLARE_FC

// Sets the dynamic-LDS limit of a kernel once, then launches it.
template <typename Args>
hipError_t launch_with_lds(const void* kern, void (*fn)(Args), bool* attr_set, dim3 grid,
                           dim3 block, size_t lds, hipStream_t st, const Args& a) {
  if (!*attr_set) {
    const hipError_t e =
        hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax);
    if (e != hipSuccess) return e;
    *attr_set = true;
  }
  hipLaunchKernelGGL(fn, grid, block, lds, st, a);
  return hipGetLastError();
}

}  // namespace salt
