#include "logical_block_manager.h"

#include <string>

namespace kvx {

LogicalBlockManager::LogicalBlockManager(int num_blocks)
    : total_blocks_(num_blocks < 0 ? 0 : num_blocks),
      blocks_(static_cast<size_t>(total_blocks_)) {
  for (int i = 0; i < total_blocks_; ++i) free_.insert(free_.end(), i);
}

void LogicalBlockManager::SetEvictable(int id, bool evictable) {
  const auto key = std::make_pair(blocks_[id].last_access_counter, id);
  if (evictable) {
    evictable_.insert(key);
  } else {
    evictable_.erase(key);
  }
}

StatusOr<std::vector<int>> LogicalBlockManager::Allocate(
    int num_blocks_to_allocate, bool lock) {
  if (num_blocks_to_allocate <= 0) {
    return InvalidArgumentError("Requested blocks must be > 0, got " +
                                std::to_string(num_blocks_to_allocate));
  }
  if (num_blocks_to_allocate > total_blocks_) {
    return InvalidArgumentError(
        "Requested blocks (" + std::to_string(num_blocks_to_allocate) +
        ") exceed total blocks (" + std::to_string(total_blocks_) + ")");
  }
  const size_t want = static_cast<size_t>(num_blocks_to_allocate);
  if (free_.size() + evictable_.size() < want) {
    return ResourceExhaustedError(
        "Insufficient available blocks. Requested: " +
        std::to_string(num_blocks_to_allocate) +
        ", Free: " + std::to_string(free_.size()) +
        ", Evictable: " + std::to_string(evictable_.size()));
  }
  std::vector<int> ids;
  ids.reserve(want);
  // Free ids first, ascending.
  while (ids.size() < want && !free_.empty()) {
    ids.push_back(*free_.begin());
    free_.erase(free_.begin());
  }
  // Then unlocked allocated ids, least recently accessed first (ties by id).
  while (ids.size() < want) {
    const int id = evictable_.begin()->second;
    evictable_.erase(evictable_.begin());
    ids.push_back(id);
  }
  ++access_counter_;
  for (int id : ids) {
    BlockState& b = blocks_[id];
    if (b.is_locked) --num_locked_;
    b.is_allocated = true;
    b.is_locked = lock;
    b.last_access_counter = access_counter_;
    if (lock) {
      ++num_locked_;
    } else {
      SetEvictable(id, true);
    }
  }
  return ids;
}

Status LogicalBlockManager::AllocateTarget(const std::vector<int>& block_ids) {
  std::vector<bool> seen(static_cast<size_t>(total_blocks_), false);
  for (int id : block_ids) {
    if (!InRange(id)) {
      return InvalidArgumentError("Invalid block ID: " + std::to_string(id));
    }
    if (blocks_[id].is_allocated) {
      return FailedPreconditionError("Already allocated block ID: " +
                                     std::to_string(id));
    }
    if (seen[id]) {
      return InvalidArgumentError("Duplicate block ID: " + std::to_string(id));
    }
    seen[id] = true;
  }
  ++access_counter_;
  for (int id : block_ids) {
    free_.erase(id);
    BlockState& b = blocks_[id];
    b.is_allocated = true;
    b.is_locked = true;
    b.last_access_counter = access_counter_;
    ++num_locked_;
  }
  return OkStatus();
}

Status LogicalBlockManager::Unlock(const std::vector<int>& block_ids) {
  for (int id : block_ids) {
    if (!InRange(id)) {
      return InvalidArgumentError("Invalid block ID: " + std::to_string(id));
    }
    if (!blocks_[id].is_allocated) {
      return InvalidArgumentError("Cannot unlock unallocated block ID: " +
                                  std::to_string(id));
    }
  }
  for (int id : block_ids) {
    BlockState& b = blocks_[id];
    if (b.is_locked) {
      b.is_locked = false;
      --num_locked_;
      SetEvictable(id, true);
    }
  }
  return OkStatus();
}

Status LogicalBlockManager::Deallocate(const std::vector<int>& block_ids) {
  for (int id : block_ids) {
    if (!InRange(id)) {
      return InvalidArgumentError("Invalid block ID: " + std::to_string(id));
    }
    if (!blocks_[id].is_allocated) {
      return InvalidArgumentError("Cannot deallocate unallocated block ID: " +
                                  std::to_string(id));
    }
  }
  for (int id : block_ids) {
    BlockState& b = blocks_[id];
    if (!b.is_allocated) continue;  // repeated id in one call
    if (b.is_locked) {
      --num_locked_;
    } else {
      SetEvictable(id, false);
    }
    b.is_allocated = false;
    b.is_locked = false;
    free_.insert(id);
  }
  return OkStatus();
}

Status LogicalBlockManager::AccessBlock(int block_id) {
  if (!InRange(block_id)) {
    return InvalidArgumentError("Invalid block ID: " +
                                std::to_string(block_id));
  }
  if (!blocks_[block_id].is_allocated) {
    return InvalidArgumentError("Cannot access unallocated block ID: " +
                                std::to_string(block_id));
  }
  ++access_counter_;
  BlockState& b = blocks_[block_id];
  if (!b.is_locked) SetEvictable(block_id, false);
  b.last_access_counter = access_counter_;
  if (!b.is_locked) SetEvictable(block_id, true);
  return OkStatus();
}

bool LogicalBlockManager::IsAllocated(int block_id) const {
  return InRange(block_id) && blocks_[block_id].is_allocated;
}

bool LogicalBlockManager::IsLocked(int block_id) const {
  return InRange(block_id) && blocks_[block_id].is_locked;
}

}  // namespace kvx
