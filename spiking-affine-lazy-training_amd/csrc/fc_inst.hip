// Instantiates the FC kernels for one weight width (SALT_QBITS, set by build.sh).
#include <array>
#include <utility>

#include "launch.hpp"

#ifndef SALT_QBITS
#error "SALT_QBITS must be defined"
#endif

namespace salt {
namespace {

#if SALT_QBITS == 8
using QType = int8_t;
#elif SALT_QBITS == 16
using QType = int16_t;
#else
using QType = int32_t;
#endif

template <int NPL, int F>
hipError_t fc_entry(const FcArgs& a, dim3 grid, int waves, size_t lds, hipStream_t st) {
  constexpr bool kSat = (F & kFcSat) != 0, kWlds = (F & kFcWlds) != 0;
  constexpr bool kNoFire = (F & kFcNoFire) != 0;
  static bool attr_set = false;
  auto fn = fc_layer_kernel<QType, NPL, kSat, kWlds, kNoFire>;
  return launch_with_lds(reinterpret_cast<const void*>(fn), fn, &attr_set, grid,
                         dim3(kWave * waves), lds, st, a);
}

using FcFn = hipError_t (*)(const FcArgs&, dim3, int, size_t, hipStream_t);

template <int NPL, int... F>
constexpr std::array<FcFn, sizeof...(F)> fc_table(std::integer_sequence<int, F...>) {
  return {{&fc_entry<NPL, F>...}};
}

}  // namespace

#define SALT_CAT2(a, b) a##b
#define SALT_CAT(a, b) SALT_CAT2(a, b)

hipError_t SALT_CAT(launch_fc_q, SALT_QBITS)(const FcArgs& a, int npl, int flags, dim3 grid,
                                             int waves, size_t lds, hipStream_t st) {
  // layers without a threshold (readouts) are narrow: their variant exists for slices of
  // up to 128 neurons; wider ones run the general kernel, whose thresholds never fire
  static constexpr auto t1 = fc_table<1>(std::make_integer_sequence<int, 8>{});
  static constexpr auto t2 = fc_table<2>(std::make_integer_sequence<int, 8>{});
  static constexpr auto t4 = fc_table<4>(std::make_integer_sequence<int, 4>{});
  static constexpr auto t8 = fc_table<8>(std::make_integer_sequence<int, 4>{});
  static constexpr auto t16 = fc_table<16>(std::make_integer_sequence<int, 4>{});
  switch (npl) {
    case 1: return t1[flags & 7](a, grid, waves, lds, st);
    case 2: return t2[flags & 7](a, grid, waves, lds, st);
    case 4: return t4[flags & 3](a, grid, waves, lds, st);
    case 8: return t8[flags & 3](a, grid, waves, lds, st);
    default: return t16[flags & 3](a, grid, waves, lds, st);
  }
}

}  // namespace salt
