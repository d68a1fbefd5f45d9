// Host block allocator with lock state and LRU-by-access-counter eviction.
//
// Same contract as the reference's LogicalBlockManager
// (tpu_sync/kv_cache/logical_block_manager.h:35-93,
// tpu_sync/kv_cache/logical_block_manager.cc:31-235): Allocate hands out
// free ids in ascending order first, then reclaims unlocked allocated ids in
// (last_access_counter, id) order; every mutating call validates the whole
// batch before it changes any state. Not thread-safe: callers lock.
//
// Free ids are kept in an ordered set and evictable ids in an ordered set
// keyed by (counter, id), so Allocate costs O(k log N) for k ids instead of
// the reference's O(N) scan plus sort; the ids chosen are identical.
#ifndef KVX_HOST_LOGICAL_BLOCK_MANAGER_H_
#define KVX_HOST_LOGICAL_BLOCK_MANAGER_H_

#include <cstdint>
#include <set>
#include <utility>
#include <vector>

#include "status.h"

namespace kvx {

class LogicalBlockManager {
 public:
  explicit LogicalBlockManager(int num_blocks);

  StatusOr<std::vector<int>> Allocate(int num_blocks_to_allocate,
                                      bool lock = false);
  Status AllocateTarget(const std::vector<int>& block_ids);
  Status Unlock(const std::vector<int>& block_ids);
  Status Deallocate(const std::vector<int>& block_ids);
  Status AccessBlock(int block_id);

  bool IsAllocated(int block_id) const;
  bool IsLocked(int block_id) const;
  int total_blocks() const { return total_blocks_; }
  int num_free_blocks() const { return static_cast<int>(free_.size()); }
  int num_allocated_blocks() const { return total_blocks_ - num_free_blocks(); }
  int num_locked_blocks() const { return num_locked_; }

 private:
  struct BlockState {
    bool is_allocated = false;
    bool is_locked = false;
    uint64_t last_access_counter = 0;
  };
  bool InRange(int id) const { return id >= 0 && id < total_blocks_; }
  void SetEvictable(int id, bool evictable);

  int total_blocks_;
  uint64_t access_counter_ = 0;
  int num_locked_ = 0;
  std::vector<BlockState> blocks_;
  std::set<int> free_;
  std::set<std::pair<uint64_t, int>> evictable_;
};

}  // namespace kvx

#endif  // KVX_HOST_LOGICAL_BLOCK_MANAGER_H_
