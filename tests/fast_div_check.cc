// Checks the multiply-high division of the tiled-copy kernel (FastDivU32,
// kernels/tiled_copy.h) against '/' on the CPU: every divisor up to 4096
// with every n up to 2^16, plus the divisors the layouts use, powers of two
// and their neighbours, and large divisors, each against edge and random n.
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#include "tiled_copy.h"

int main() {
  using kvx::FastDivHost;
  using kvx::MakeFastDivU32;
  uint64_t checked = 0;
  auto check = [&](uint32_t d, uint32_t n) {
    const uint32_t q = FastDivHost(MakeFastDivU32(d), n);
    ++checked;
    if (q != n / d) {
      std::printf("mismatch: %u / %u = %u, got %u\n", n, d, n / d, q);
      return false;
    }
    return true;
  };
  for (uint32_t d = 1; d <= 4096; ++d) {
    for (uint32_t n = 0; n < (1u << 16); ++n) {
      if (!check(d, n)) return 1;
    }
  }
  std::vector<uint32_t> divs = {1, 2, 3, 7, 8, 100, 128, 257, 1000, 4095, 14336, 65535,
                                65536, 65537, 1000003, 0x7fffffffu, 0x80000000u};
  for (int s = 1; s <= 31; ++s) {
    const uint32_t p = 1u << s;
    divs.push_back(p - 1);
    divs.push_back(p);
    divs.push_back(p + 1);
  }
  std::mt19937_64 rng(42);
  for (int i = 0; i < 2000; ++i) divs.push_back(1 + static_cast<uint32_t>(rng() % 0x80000000u));
  for (uint32_t d : divs) {
    if (d == 0) continue;
    const uint32_t edges[] = {0u, 1u, d - 1, d, d + 1, 2 * d - 1, 0xfffffffeu, 0xffffffffu,
                              0x80000000u, 0x7fffffffu};
    for (uint32_t n : edges) {
      if (!check(d, n)) return 1;
    }
    for (uint32_t q = 0; q < 64; ++q) {
      const uint64_t m = static_cast<uint64_t>(d) * (0xffffffffu / d - q);
      for (int o = -1; o <= 1; ++o) {
        const uint64_t n = m + o;
        if (n <= 0xffffffffu && !check(d, static_cast<uint32_t>(n))) return 1;
      }
    }
    for (int i = 0; i < 2000; ++i) {
      if (!check(d, static_cast<uint32_t>(rng()))) return 1;
    }
  }
  std::printf("fast div ok (%llu checks)\n", static_cast<unsigned long long>(checked));
  return 0;
}
