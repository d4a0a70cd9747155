// Instantiates the packed conv kernels for one iteration bound (SALT_PACK_IMAX, set by
// build.sh): 16 variants each (saturate, neuron extremes, threshold array, no truncation).
#include <array>
#include <utility>

#include "launch.hpp"

#ifndef SALT_PACK_IMAX
#error "SALT_PACK_IMAX must be defined"
#endif

namespace salt {
namespace {

template <int IMAX, int F>
hipError_t pack_entry(const PackArgs& a, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
  constexpr bool kSat = (F & kPackSat) != 0, kExt = (F & kPackExt) != 0,
                 kVtha = (F & kPackVtha) != 0, kNoTrunc = (F & kPackNoTrunc) != 0;
  static bool attr_set = false;
  auto fn = conv_packed_kernel<IMAX, kSat, kExt, kVtha, kNoTrunc>;
  return launch_with_lds(reinterpret_cast<const void*>(fn), fn, &attr_set, grid, block, lds, st,
                         a);
}

using PackFn = hipError_t (*)(const PackArgs&, dim3, dim3, size_t, hipStream_t);

template <int IMAX, int... F>
constexpr std::array<PackFn, sizeof...(F)> pack_table(std::integer_sequence<int, F...>) {
  return {{&pack_entry<IMAX, F>...}};
}

}  // namespace

#define SALT_CAT2(a, b) a##b
#define SALT_CAT(a, b) SALT_CAT2(a, b)

hipError_t SALT_CAT(launch_pack_imax, SALT_PACK_IMAX)(const PackArgs& a, int flags, dim3 grid,
                                                      dim3 block, size_t lds, hipStream_t st) {
  static constexpr auto table =
      pack_table<SALT_PACK_IMAX>(std::make_integer_sequence<int, kPackFlagCombos>{});
  return table[flags & (kPackFlagCombos - 1)](a, grid, block, lds, st);
}

}  // namespace salt
