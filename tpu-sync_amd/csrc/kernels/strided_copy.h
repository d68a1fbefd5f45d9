// Host-side interface of the strided-entry copy kernel (gfx950).
//
// An entry is the reference's strided push entry
// (ShardPushEntryProto{src_offset, dst_offset, size, count, src_stride,
// dst_stride}, tpu_sync/rpc/raiden_service.proto:104-131) with absolute
// device addresses: for c in [0, count): copy `size` bytes from
// src + c * src_stride to dst + c * dst_stride, the expansion
// WeightSynchronizerBase::PushWeightsResharded performs on the host
// (tpu_sync/weight_sync/weight_synchronizer_base.cc:626-666). One launch
// executes any number of entries: a per-tensor offset-table pack (count 1
// per tensor), its unpack, and column splits of row-major matrices (count =
// rows) all have this form.
#ifndef KVX_KERNELS_STRIDED_COPY_H_
#define KVX_KERNELS_STRIDED_COPY_H_

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <vector>

namespace kvx {

struct StridedCopy {
  uint64_t src = 0;
  uint64_t dst = 0;
  int64_t size = 0;        // bytes per row
  int64_t count = 1;       // rows (the reference treats count <= 0 as 1)
  int64_t src_stride = 0;  // bytes between source rows
  int64_t dst_stride = 0;  // bytes between destination rows
};

// Device-side form of one entry, built on the host (64 bytes).
struct StridedEntryDev {
  uint64_t src;
  uint64_t dst;
  uint64_t src_stride;
  uint64_t dst_stride;
  uint64_t div_magic;      // floor(2^32 / vecs) + 1: row = (k * magic) >> 32
  uint32_t count;          // rows
  uint32_t vecs;           // vectors per row
  uint32_t tile_begin;     // first workgroup of the entry
  uint32_t rows_per_tile;  // > 0: whole rows per workgroup
  uint32_t tiles_per_row;  // > 0: a row spans this many workgroups
  uint32_t pad;
};
static_assert(sizeof(StridedEntryDev) == 64, "device table layout");

// Builds the device table for `copies` with vector width `vec_bytes`;
// returns false if an entry violates the kernel's limits. *grid receives the
// workgroup count. Entries whose rows span more than one tile come first in
// the table (in the copies' order, then the others in theirs); *long_tiles
// (if not null) receives their tiles, the first of the grid.
bool BuildStridedTable(const std::vector<StridedCopy>& copies, int vec_bytes,
                       std::vector<StridedEntryDev>* table, uint32_t* grid,
                       uint32_t* long_tiles = nullptr);

// Largest vector width (16, 8, 4, 2 or 1) dividing every address, size and
// stride of `copies`.
int StridedVectorBytes(const std::vector<StridedCopy>& copies);

// Launches the copy of a device-resident table of `n` entries (built by
// BuildStridedTable, `tiles` from its *grid, `long_tiles` from its
// *long_tiles) on `stream`. max_workgroups > 0 caps the grid (each workgroup
// then walks tiles with a stride of the grid), for copies bound by PCIe
// rather than HBM; otherwise the launch reserves LDS so that at most 2 of
// its workgroups share a CU, and at 16-byte vectors moves the long-row tiles
// sliced (0: every tile contiguous).
hipError_t LaunchStridedCopy(const StridedEntryDev* table_dev, uint32_t n,
                             uint32_t tiles, int vec_bytes, hipStream_t stream,
                             uint32_t max_workgroups = 0, uint32_t long_tiles = 0);

}  // namespace kvx

#endif  // KVX_KERNELS_STRIDED_COPY_H_
