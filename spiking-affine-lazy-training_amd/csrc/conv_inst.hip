// Instantiates the conv kernels for one iteration count (SALT_NIT, set by build.sh).
#include <array>
#include <utility>

#include "launch.hpp"

#ifndef SALT_NIT
#error "SALT_NIT must be defined"
#endif

namespace salt {
namespace {

template <int NIT, int F>
hipError_t conv_entry(const ConvArgs& a, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
  constexpr bool kSat = (F & kConvSat) != 0,
                 kExt = (F & kConvExt) != 0, kVthN = (F & kConvVthN) != 0,
                 kM32 = (F & kConvM32) != 0, kNoTrunc = (F & kConvNoTrunc) != 0,
                 kPair = (F & kConvPair) != 0;
  if constexpr (kPair && !kM32) {
    return hipErrorInvalidValue;  // pairs need candidate masks of 32 bits or less
  } else {
    static bool attr_set = false;
    auto fn = conv_layer_kernel<NIT, kSat, kExt, kVthN, kM32, kNoTrunc, kPair>;
    return launch_with_lds(reinterpret_cast<const void*>(fn), fn, &attr_set, grid, block, lds,
                           st, a);
  }
}

using ConvFn = hipError_t (*)(const ConvArgs&, dim3, dim3, size_t, hipStream_t);

template <int NIT, int... F>
constexpr std::array<ConvFn, sizeof...(F)> conv_table(std::integer_sequence<int, F...>) {
  return {{&conv_entry<NIT, F>...}};
}

}  // namespace

#define SALT_CAT2(a, b) a##b
#define SALT_CAT(a, b) SALT_CAT2(a, b)

hipError_t SALT_CAT(launch_conv_nit, SALT_NIT)(const ConvArgs& a, int flags, dim3 grid,
                                               dim3 block, size_t lds, hipStream_t st) {
  static constexpr auto table =
      conv_table<SALT_NIT>(std::make_integer_sequence<int, kConvFlagCombos>{});
  return table[flags & (kConvFlagCombos - 1)](a, grid, block, lds, st);
}

}  // namespace salt
