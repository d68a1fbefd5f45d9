// Host-side checks of the tiled-copy job builder (PlanTiled /
// AppendTiledJobs in libkvx) on the CPU, no device calls:
//   * buffers not aligned to the element size are rejected for every form
//     (the vector form would otherwise get fewer bytes per vector than one
//     element);
//   * the 32-bit unit limits hold at the vector width the buffers' alignment
//     actually allows, not only at the plan's widest one: a tensor whose
//     units fit at 16-byte vectors but not at 1-byte ones is refused at the
//     narrow width instead of wrapping its unit indices.
#include <cstdint>
#include <cstdio>
#include <vector>

#include "tiled_layout.h"

using kvx::Code;
using kvx::TiledJob;
using kvx::TiledLayout;

namespace {

int failures = 0;

void expect(bool ok, const char* what) {
  if (!ok) {
    std::printf("FAIL: %s\n", what);
    ++failures;
  }
}

TiledLayout Layout(int s, std::vector<int64_t> dims, std::vector<std::vector<int64_t>> tiles,
                   std::vector<int> mtm = {}) {
  TiledLayout l;
  l.itemsize = s;
  l.dims = dims;
  if (mtm.empty()) {
    for (int i = static_cast<int>(dims.size()) - 1; i >= 0; --i) mtm.push_back(i);
  }
  l.minor_to_major = mtm;
  l.tiles = tiles;
  return l;
}

// Builds the jobs of the whole tensor in one direction; returns the status
// code and checks that every vector job's units fit 32-bit indices.
Code Jobs(const kvx::TiledPlan& p, uint64_t tiled, uint64_t linear, bool tile,
          std::vector<TiledJob>* out = nullptr) {
  std::vector<TiledJob> zero, jobs;
  kvx::Status st = kvx::AppendTiledJobs(p, tiled, linear, 0, p.logical_bytes, tile,
                                        /*zero_pass=*/true, &zero, &jobs);
  for (const TiledJob& j : jobs) {
    if (j.vec != 0) {
      expect(j.dev.lo + j.dev.count <= (uint64_t{1} << 32), "vector job units fit 32 bits");
    }
  }
  if (out != nullptr) *out = jobs;
  return st.code();
}

}  // namespace

int main() {
  const uint64_t base = uint64_t{1} << 20;
  // Element-size alignment, both directions, both buffers.
  {
    auto p = kvx::PlanTiled(Layout(2, {40, 384}, {{8, 128}, {2, 1}}));
    expect(p.ok() && p->standard, "bf16 T(8,128)(2,1) plans as standard");
    for (bool tile : {true, false}) {
      expect(Jobs(*p, base, base + 1, tile) == Code::kInvalidArgument, "bf16 linear +1 refused");
      expect(Jobs(*p, base + 1, base, tile) == Code::kInvalidArgument, "bf16 tiled +1 refused");
      expect(Jobs(*p, base, base + 2, tile) == Code::kOk, "bf16 linear +2 accepted");
      expect(Jobs(*p, base + 8, base, tile) == Code::kOk, "bf16 tiled +8 accepted");
    }
  }
  {
    auto p = kvx::PlanTiled(Layout(4, {3, 20, 200}, {{8, 128}}));
    expect(p.ok() && p->standard, "f32 T(8,128) plans as standard");
    for (bool tile : {true, false}) {
      expect(Jobs(*p, base, base + 2, tile) == Code::kInvalidArgument, "f32 linear +2 refused");
      expect(Jobs(*p, base + 6, base, tile) == Code::kInvalidArgument, "f32 tiled +6 refused");
      std::vector<TiledJob> jobs;
      expect(Jobs(*p, base + 4, base, tile, &jobs) == Code::kOk, "f32 tiled +4 accepted");
      for (const TiledJob& j : jobs) expect(j.vec == 0 || j.vec >= 4, "f32 vector >= element");
    }
  }
  {
    auto p = kvx::PlanTiled(Layout(1, {40, 384}, {{8, 128}, {4, 1}}));
    expect(p.ok() && p->standard, "int8 T(8,128)(4,1) plans as standard");
    for (bool tile : {true, false}) {
      expect(Jobs(*p, base + 1, base + 3, tile) == Code::kOk, "int8 any byte offset accepted");
    }
  }
  {
    auto p = kvx::PlanTiled(Layout(2, {6, 40, 24}, {{8, 8}}, {0, 2, 1}));
    expect(p.ok() && !p->standard, "permuted bf16 plans as general");
    expect(Jobs(*p, base, base + 1, true) == Code::kInvalidArgument, "general linear +1 refused");
    expect(Jobs(*p, base + 4, base + 2, false) == Code::kOk, "general +4/+2 accepted");
  }
  // 32-bit unit limits at the chosen width: 8 GiB of int8 in T(8,128) has
  // 2^29 units of 16 bytes but 2^33 of one byte, and more than 2^32
  // elements, so the element-by-element form cannot take it either.
  {
    auto p = kvx::PlanTiled(Layout(1, {65536, 131072}, {{8, 128}}));
    expect(p.ok() && p->standard && p->gen.empty(), "8 GiB int8 plans as standard only");
    for (bool tile : {true, false}) {
      std::vector<TiledJob> jobs;
      expect(Jobs(*p, base, base, tile, &jobs) == Code::kOk, "8 GiB int8, aligned buffers");
      expect(!jobs.empty() && jobs[0].vec == 16, "8 GiB int8 moves 16-byte vectors");
      expect(Jobs(*p, base, base + 4, tile, &jobs) == Code::kOk, "8 GiB int8, 4-byte aligned");
      expect(Jobs(*p, base, base + 1, tile) == Code::kUnimplemented,
             "8 GiB int8 at 1-byte vectors refused (2^33 units)");
      expect(Jobs(*p, base + 2, base, tile) == Code::kUnimplemented,
             "8 GiB int8 at 2-byte vectors refused (2^32 units)");
    }
  }
  if (failures == 0) std::printf("tiled jobs: all checks passed\n");
  return failures == 0 ? 0 : 1;
}
