// Checks kvx::HostCopyPool: every byte of every segment arrives and nothing
// outside the segments is written, for pools of 0-7 workers, batches of many
// small segments (taken four at a time), of segments split into 4 MiB pieces,
// of mixed sizes (0 bytes to 9 MiB), many batches in a row, and two threads
// calling Copy on one pool at once. Built with -fsanitize=thread it also
// checks the pool's handoffs for data races.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <thread>
#include <vector>

#include "host_copy_pool.h"

namespace {

// The ThreadSanitizer build runs lighter batches (it is many times slower);
// every handoff pattern still occurs.
#ifdef KVX_CHECK_LIGHT
constexpr int kSmall = 160, kRounds = 30, kCallerRounds = 3;
constexpr size_t kBig = 4u << 20;
#else
constexpr int kSmall = 1200, kRounds = 300, kCallerRounds = 20;
constexpr size_t kBig = 9u << 20;
#endif

struct Arena {
  std::vector<uint8_t> src, dst;
  explicit Arena(size_t n) : src(n), dst(n, 0xA5) {
    uint32_t x = static_cast<uint32_t>(n) * 2654435761u + 1;
    for (uint8_t& b : src) {
      x = x * 1664525u + 1013904223u;
      b = static_cast<uint8_t>(x >> 24);
    }
  }
};

// Non-overlapping segments: `sizes` laid out one after another with gaps of
// `gap` bytes (left untouched), shuffled, at the same offsets in src and dst.
std::vector<kvx::HostCopyPool::Segment> Layout(Arena& a, const std::vector<size_t>& sizes,
                                               size_t gap, std::mt19937_64& rng,
                                               std::vector<std::pair<size_t, size_t>>* spans) {
  std::vector<kvx::HostCopyPool::Segment> segs;
  size_t off = 0;
  for (size_t s : sizes) {
    off += gap + (rng() % 64);
    segs.push_back({a.dst.data() + off, a.src.data() + off, s});
    spans->push_back({off, s});
    off += s;
  }
  std::shuffle(segs.begin(), segs.end(), rng);
  return segs;
}

bool Check(const Arena& a, const std::vector<std::pair<size_t, size_t>>& spans, const char* what) {
  std::vector<uint8_t> covered(a.dst.size(), 0);
  for (auto [off, n] : spans) {
    if (memcmp(a.dst.data() + off, a.src.data() + off, n) != 0) {
      std::printf("%s: segment at %zu (%zu bytes) differs\n", what, off, n);
      return false;
    }
    memset(covered.data() + off, 1, n);
  }
  for (size_t i = 0; i < a.dst.size(); ++i) {
    if (!covered[i] && a.dst[i] != 0xA5) {
      std::printf("%s: byte %zu outside the segments written\n", what, i);
      return false;
    }
  }
  return true;
}

}  // namespace

int main() {
  std::mt19937_64 rng(11);
  int checks = 0;
  for (int threads : {0, 1, 3, 7}) {
    kvx::HostCopyPool pool(threads);
    // Many small segments: random 32 KiB blocks (four at a time once there
    // are 64 per thread) and a few odd sizes.
    {
      std::vector<size_t> sizes(kSmall, 32768);
      for (size_t k = 0; k < sizes.size(); k += 97) sizes[k] = 1 + rng() % 70000;
      std::vector<std::pair<size_t, size_t>> spans;
      Arena a(kSmall * (32768 + 200) + (1 << 20));
      pool.Copy(Layout(a, sizes, 100, rng, &spans));
      if (!Check(a, spans, "small segments")) return 1;
      ++checks;
    }
    // Large segments split into 4 MiB pieces, and empty ones.
    {
      std::vector<size_t> sizes = {kBig + 5, 0, (4u << 20) - 1, 1, 0, 1 << 20};
      std::vector<std::pair<size_t, size_t>> spans;
      Arena a(kBig + (6u << 20));
      pool.Copy(Layout(a, sizes, 128, rng, &spans));
      if (!Check(a, spans, "large segments")) return 1;
      ++checks;
    }
    // Many batches in a row on one pool: every handoff between batches.
    {
      Arena a(1u << 20);  // at most 40 segments of < 9000 bytes plus gaps
      for (int round = 0; round < kRounds; ++round) {
        std::vector<size_t> sizes(1 + rng() % 40);
        for (size_t& s : sizes) s = rng() % 9000;
        std::vector<std::pair<size_t, size_t>> spans;
        std::fill(a.dst.begin(), a.dst.end(), 0xA5);
        pool.Copy(Layout(a, sizes, 16, rng, &spans));
        if (!Check(a, spans, "batch sequence")) return 1;
      }
      ++checks;
    }
    // Two callers at once on one pool: their batches run one after another.
    {
      Arena a(kSmall / 2 * 16600 + (1 << 20)), b(30 * 300100 + (1 << 20));
      std::vector<std::pair<size_t, size_t>> sa, sb;
      std::mt19937_64 ra(1), rb(2);
      std::vector<size_t> za(kSmall / 2, 16384), zb(30, 300000);
      auto ga = Layout(a, za, 64, ra, &sa);
      auto gb = Layout(b, zb, 64, rb, &sb);
      std::thread t1([&] { for (int r = 0; r < kCallerRounds; ++r) pool.Copy(ga); });
      std::thread t2([&] { for (int r = 0; r < kCallerRounds; ++r) pool.Copy(gb); });
      t1.join();
      t2.join();
      if (!Check(a, sa, "caller 1") || !Check(b, sb, "caller 2")) return 1;
      ++checks;
    }
  }
  std::printf("host copy pool ok: %d checks\n", checks);
  return 0;
}
