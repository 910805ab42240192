// CPU check of mdma_amd/csrc/libm_expf.h: mdma::libm_expf against the C
// library's expf on every f32 bit pattern (split over threads), and the
// table of 2^(i/32) against exp2l. Prints "mismatches N table_errors M".
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <thread>
#include <vector>

#include "../mdma_amd/csrc/libm_expf.h"

int main() {
  int table_errors = 0;
  for (uint32_t i = 0; i < 32; i++) {
    const double v = (double)exp2l((long double)i / 32);
    uint64_t u;
    memcpy(&u, &v, 8);
    if (u - ((uint64_t)i << 47) != mdma::exp2_table(i)) table_errors++;
  }
  const unsigned n = std::thread::hardware_concurrency() ? std::thread::hardware_concurrency() : 4;
  std::atomic<uint64_t> bad{0};
  std::vector<std::thread> th;
  for (unsigned w = 0; w < n; w++)
    th.emplace_back([&, w] {
      uint64_t b = 0;
      for (uint64_t u = w; u < (1ull << 32); u += n) {
        const uint32_t bits = (uint32_t)u;
        float x;
        memcpy(&x, &bits, 4);
        const float g = expf(x), m = mdma::libm_expf(x);
        uint32_t gb, mb;
        memcpy(&gb, &g, 4);
        memcpy(&mb, &m, 4);
        if (gb != mb && !(isnan(g) && isnan(m))) b++;
      }
      bad += b;
    });
  for (auto &t : th) t.join();
  printf("mismatches %llu table_errors %d\n", (unsigned long long)bad.load(), table_errors);
  return 0;
}
