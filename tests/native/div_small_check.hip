// Host check of div_small (csrc/salt_device.hpp), the conv decode's division: every
// n < 2^22 against exact integer division, for small divisors, the powers of two and
// their neighbours, and the divisors of the benchmark geometries.  Exit status 0 = exact.
#include <cstdio>

#include "salt_device.hpp"

int main() {
  int ds[512], nd = 0;
  for (int d = 1; d <= 300; ++d) ds[nd++] = d;
  for (int k = 9; k <= 21; ++k) {
    ds[nd++] = (1 << k) - 1;
    ds[nd++] = 1 << k;
    ds[nd++] = (1 << k) + 1;
    ds[nd++] = 3 << (k - 2);
  }
  ds[nd++] = 1156;     // 34 x 34
  ds[nd++] = 16384;    // 128 x 128
  ds[nd++] = 4194303;  // 2^22 - 1
  long bad = 0;
  for (int i = 0; i < nd; ++i) {
    const int d = ds[i];
    const float rcp = 1.0f / (float)d;
    for (int n = 0; n < (1 << 22); ++n)
      if (salt::div_small(n, d, rcp) != n / d && bad++ < 5)
        std::printf("n=%d d=%d: %d, not %d\n", n, d, salt::div_small(n, d, rcp), n / d);
  }
  std::printf("%d divisors, %ld mismatches\n", nd, bad);
  return bad != 0;
}
