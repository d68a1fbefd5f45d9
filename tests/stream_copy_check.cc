// Checks kvx::StreamCopy against memcpy: sizes around the streaming threshold
// and the 128-byte step, every destination and source offset within a cache
// line, guard bytes on both sides of the destination untouched.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "stream_copy.h"

int main() {
  const size_t kMin = kvx::kStreamCopyMinBytes;
  const size_t sizes[] = {0, 1, 63, 4096, kMin - 1, kMin, kMin + 1, kMin + 63, kMin + 127,
                          kMin + 128, kMin + 129, 3 * kMin + 77, (4u << 20) + 5};
  const size_t kGuard = 256;
  std::vector<uint8_t> src((4u << 20) + 4096), dst, want;
  uint32_t x = 12345;
  for (uint8_t& b : src) {
    x = x * 1664525u + 1013904223u;
    b = static_cast<uint8_t>(x >> 24);
  }
  int cases = 0;
  for (size_t n : sizes) {
    dst.assign(n + 64 + 2 * kGuard, 0);
    // Every destination offset for the streamed sizes below 1 MiB, a few above.
    const size_t step = n < kMin ? 7 : n < (1u << 20) ? 1 : 9;
    for (size_t doff = 0; doff < 64; doff += step) {
      for (size_t soff : {size_t{0}, size_t{3}, size_t{32}, size_t{61}}) {
        std::memset(dst.data(), 0xA5, dst.size());
        want = dst;
        std::memcpy(want.data() + kGuard + doff, src.data() + soff, n);
        kvx::PrefetchSource(src.data() + soff, n);
        kvx::StreamCopy(dst.data() + kGuard + doff, src.data() + soff, n);
        kvx::StreamFence();
        if (dst != want) {
          std::printf("mismatch: bytes %zu dst offset %zu src offset %zu\n", n, doff, soff);
          return 1;
        }
        ++cases;
      }
    }
  }
  std::printf("stream copy ok: %d cases\n", cases);
  return 0;
}
