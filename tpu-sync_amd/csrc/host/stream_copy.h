// Host-to-host copy with non-temporal (streaming) stores, for the bounce
// lanes' moves between pinned bounce buffers and pageable host memory.
#pragma once

#include <cstddef>

namespace kvx {

// Copies `bytes` from `src` to `dst` (non-overlapping). Copies of at least
// kStreamCopyMinBytes write the destination with streaming stores, which skip
// the read-for-ownership of every destination line an ordinary store pays:
// the copy then moves 2x its bytes through host memory instead of 3x, which
// matters while the DMA engines share that memory. Smaller copies use memcpy.
// Streaming stores are weakly ordered: call StreamFence() before another
// thread, or a DMA, may read the destination.
void StreamCopy(void* dst, const void* src, size_t bytes);

// Store fence: every streaming store this thread issued is globally visible
// once it returns.
void StreamFence();

// Prefetches the first min(bytes, kPrefetchBytes) of `src` into the cache,
// for a copy that follows: its page walks and line fills then overlap the
// copy before it.
void PrefetchSource(const void* src, size_t bytes);

constexpr size_t kStreamCopyMinBytes = 4096;
constexpr size_t kPrefetchBytes = 32768;

}  // namespace kvx
