// The C-ABI's device-address checks on the CPU, no GPU calls: the address
// lookup is replaced (kvx::SetAddressQueryForTesting) by a map of made-up
// allocations, and every entry point that takes raw device addresses and
// can be called without a device object is driven with host, unknown,
// managed, wrong-device and overrunning addresses. Each must return
// KVX_INVALID_ARGUMENT with a message naming the argument, before anything
// is issued. No C-ABI call here is given addresses that should pass (such a
// call would go on to the device with made-up addresses); the checker
// itself is shown to pass good ranges, once per allocation.
#include <cstdint>
#include <cstdio>
#include <climits>
#include <cstring>
#include <string>

#include "device_memory.h"
#include "kvx.h"

namespace {

constexpr uint64_t kDev0 = 0x7f0000000000ull;  // device 0, 4 GiB
constexpr uint64_t kDev0Size = 4ull << 30;
constexpr uint64_t kDev1 = 0x7e0000000000ull;  // device 1, 1 GiB
constexpr uint64_t kHost = 0x600000000000ull;  // pinned host, 1 GiB
constexpr uint64_t kManaged = 0x610000000000ull;

kvx::AddressInfo FakeQuery(uint64_t a) {
  kvx::AddressInfo i;
  if (a >= kDev0 && a < kDev0 + kDev0Size) {
    i = {kvx::MemKind::kDevice, 0, kDev0, kDev0Size};
  } else if (a >= kDev1 && a < kDev1 + (1ull << 30)) {
    i = {kvx::MemKind::kDevice, 1, kDev1, 1ull << 30};
  } else if (a >= kHost && a < kHost + (1ull << 30)) {
    i = {kvx::MemKind::kHost, 0, 0, 0};
  } else if (a >= kManaged && a < kManaged + (1ull << 30)) {
    i = {kvx::MemKind::kOther, 0, 0, 0};
  }
  return i;
}

int failures = 0;

// rc must be INVALID_ARGUMENT with `needle` in the message.
void Refused(int rc, const char* needle, const char* what) {
  const char* msg = kvx_last_error();
  if (rc != KVX_INVALID_ARGUMENT || msg == nullptr || std::strstr(msg, needle) == nullptr) {
    std::printf("FAIL %s: rc %d, message '%s' (want INVALID_ARGUMENT with '%s')\n", what, rc,
                msg ? msg : "", needle);
    ++failures;
  }
}

kvx_tiled_layout Layout2d(int64_t h, int64_t w) {
  kvx_tiled_layout l;
  std::memset(&l, 0, sizeof(l));
  l.itemsize = 2;
  l.rank = 2;
  l.dims[0] = h;
  l.dims[1] = w;
  l.minor_to_major[0] = 1;
  l.minor_to_major[1] = 0;
  l.num_tiles = 1;
  l.tile_rank[0] = 2;
  l.tile_dims[0][0] = 8;
  l.tile_dims[0][1] = 128;
  return l;
}

}  // namespace

int main() {
  kvx::SetAddressQueryForTesting(FakeQuery);
  kvx_future* f = nullptr;

  // Tile / detile: both buffers, every kind of bad address.
  const kvx_tiled_layout l = Layout2d(64, 256);  // 32 KiB either side
  Refused(kvx_tile_buffer(0, &l, kHost, kDev0, nullptr, &f), "src_linear: host memory",
          "tile: host source");
  Refused(kvx_tile_buffer(0, &l, kDev0, 0x1000, nullptr, &f), "dst_tiled: not a device",
          "tile: unknown destination");
  Refused(kvx_detile_buffer(0, &l, kManaged, kDev0, nullptr, &f), "src_tiled: managed",
          "detile: managed source");
  Refused(kvx_detile_buffer(0, &l, kDev0, kDev1, nullptr, &f), "not of device 0",
          "detile: destination on device 1");
  Refused(kvx_tile_buffer(0, &l, kDev0 + kDev0Size - 100, kDev0, nullptr, &f), "past the end",
          "tile: source overruns its allocation");

  // Strided copies and plans: every row of an entry.
  kvx_strided_entry e;
  std::memset(&e, 0, sizeof(e));
  e.src = kDev0;
  e.dst = kDev0 + (1ull << 30);
  e.size_bytes = 4096;
  e.count = 16;
  e.src_stride_bytes = 8192;
  e.dst_stride_bytes = 4096;
  kvx_strided_entry bad = e;
  bad.dst = kHost;
  Refused(kvx_copy_strided(0, &bad, 1, nullptr, &f), "entry 0: strided entry destination: host",
          "strided: host destination");
  bad = e;
  bad.src_stride_bytes = 1ll << 30;  // rows 1..15 run past the 4 GiB allocation
  bad.src = kDev0 + (2ull << 30);
  Refused(kvx_copy_strided(0, &bad, 1, nullptr, &f), "past the end", "strided: rows overrun");
  kvx_strided_entry two[2] = {e, e};
  two[1].src = kDev1;
  Refused(kvx_copy_strided(0, two, 2, nullptr, &f), "entry 1", "strided: entry 1 on device 1");
  kvx_strided_plan* plan = nullptr;
  Refused(kvx_strided_plan_create(0, &bad, 1, &plan), "past the end", "plan: rows overrun");

  // Raw block kernels: every table and buffer, all on one device.
  Refused(kvx_gather_blocks(kHost, 4, 32768, 16, kDev0, 8, kDev0 + 4096, KVX_LAYER_MAJOR, 0,
                            nullptr),
          "storage_table: host memory", "gather_blocks: host table");
  Refused(kvx_scatter_blocks(kDev0, 4, 32768, 16, kDev0 + 64, 8, kDev1, KVX_LAYER_MAJOR, 0,
                             nullptr),
          "staging: memory of device 1", "scatter_blocks: staging on device 1");
  Refused(kvx_gather_blocks(kDev0, 4, 32768, 16, kDev0 + 64, 8,
                            kDev0 + kDev0Size - 32768, KVX_LAYER_MAJOR, 0, nullptr),
          "past the end", "gather_blocks: staging overruns");
  Refused(kvx_gather_blocks(kDev0, 4, 32768, 16, kDev0 + 64, 8, kDev0 + 4096, KVX_LAYER_MAJOR,
                            kHost, nullptr),
          "error: host memory", "gather_blocks: host error word");

  // Manager and weight synchronizer: every storage / tensor at create.
  uint64_t ptrs[2] = {kDev0, kHost};
  int64_t bytes[2] = {1 << 20, 1 << 20};
  kvx_manager_config mc;
  std::memset(&mc, 0, sizeof(mc));
  mc.device = 0;
  mc.host_alloc = KVX_HOST_MALLOC;
  mc.num_layers = 2;
  mc.num_shards = 1;
  mc.device_ptrs = ptrs;
  mc.device_bytes = bytes;
  mc.major_dim = 32;
  mc.host_blocks = 4;
  kvx_manager* m = nullptr;
  Refused(kvx_manager_create(&mc, &m), "device_ptrs[1]: host memory", "manager: host storage");
  ptrs[1] = kDev0 + kDev0Size - (1 << 19);
  Refused(kvx_manager_create(&mc, &m), "device_ptrs[1]: range runs past",
          "manager: storage overruns");
  kvx_weight_sync_config wc;
  std::memset(&wc, 0, sizeof(wc));
  wc.device = 1;
  wc.host_alloc = KVX_HOST_MALLOC;
  wc.num_layers = 2;
  wc.num_shards = 1;
  ptrs[0] = kDev1;
  ptrs[1] = kDev0;
  wc.device_ptrs = ptrs;
  wc.device_bytes = bytes;
  kvx_weight_sync* w = nullptr;
  Refused(kvx_weight_sync_create(&wc, &w), "device_ptrs[1]: memory of device 0",
          "weight sync: tensor on device 0");

  // Good ranges pass: any device for -1, then only that device; one lookup
  // per allocation.
  static int lookups = 0;
  kvx::SetAddressQueryForTesting([](uint64_t a) {
    ++lookups;
    return FakeQuery(a);
  });
  kvx::DeviceRangeChecker any(-1);
  bool ok = any.Check(kDev1 + 64, 4096, "a").ok() && any.device() == 1 &&
            any.Check(kDev1 + 8192, 1 << 20, "b").ok() && !any.Check(kDev0, 64, "c").ok() &&
            any.Check(kHost, 0, "empty").ok();
  if (!ok || lookups != 2) {
    std::printf("FAIL checker: pass path (lookups %d)\n", lookups);
    ++failures;
  }
  uint64_t ext = 0;
  if (!kvx::StridedExtent(4096, 16, 8192, &ext) || ext != 15 * 8192 + 4096 ||
      kvx::StridedExtent(1, INT64_MAX, 2, &ext)) {
    std::printf("FAIL StridedExtent\n");
    ++failures;
  }

  kvx::SetAddressQueryForTesting(nullptr);
  if (failures == 0) std::printf("device address checks: all passed\n");
  return failures == 0 ? 0 : 1;
}
