// Pin-aware LRU index of the host tier: the counterpart of the reference's
// LRUCache (tpu_sync/kv_cache/lru_cache.h:41-369), with the same observable
// behaviour, which callers depend on (eviction order, candidate resurrection,
// which operations reorder what):
//   * three lists -- active (MRU at the front), pinned, and eviction
//     candidates (oldest at the front);
//   * Put on a full cache demotes the active tail to the candidate list and
//     returns it; when every entry is pinned the key is silently not inserted;
//   * candidates stay indexed: Get / GetAndPin / Pin resurrect them, Peek and
//     Contains do not see them, Erase reclaims them;
//   * Unpin to zero moves the entry to the active front;
//   * GetEvictableKeys lists candidates oldest first, then the active tail.
//
// Implementation: nodes live in one pooled vector with intrusive prev/next
// indices and recycled slots, so Put/Evict/Pin never allocate after warm-up;
// the three lists are circular with sentinel nodes 0..2. Not thread-safe:
// callers lock (the store holds its mutex around every call).
#ifndef KVX_HOST_LRU_CACHE_H_
#define KVX_HOST_LRU_CACHE_H_

#include <cstddef>
#include <cstdint>
#include <functional>
#include <optional>
#include <unordered_map>
#include <utility>
#include <vector>

namespace kvx {

enum class NodeLocation : uint8_t { kLru = 0, kPinned = 1, kCandidate = 2 };

template <typename Key, typename Value, typename Hash = std::hash<Key>>
class LRUCache {
 public:
  explicit LRUCache(size_t capacity) : capacity_(capacity) { Reset(); }
  LRUCache(const LRUCache&) = delete;
  LRUCache& operator=(const LRUCache&) = delete;
  LRUCache(LRUCache&&) noexcept = default;
  LRUCache& operator=(LRUCache&&) noexcept = default;

  size_t capacity() const { return capacity_; }
  // Entries including eviction candidates.
  size_t size() const { return index_.size(); }
  size_t active_size() const { return len_[kActive] + len_[kPin]; }
  // Capacity not held by pinned entries, clamped at zero (pinning a
  // candidate can push the pinned list past the capacity).
  size_t available_space() const {
    return capacity_ > len_[kPin] ? capacity_ - len_[kPin] : 0;
  }
  bool empty() const { return index_.empty(); }

  bool Contains(const Key& key) const {
    auto it = index_.find(key);
    return it != index_.end() && nodes_[it->second].loc != NodeLocation::kCandidate;
  }

  void Clear() {
    index_.clear();
    Reset();
  }

  // Inserts or updates; see the class comment for the full-cache behaviour.
  std::optional<std::pair<Key, Value>> Put(Key key, Value value) {
    auto it = index_.find(key);
    if (it != index_.end()) {
      nodes_[it->second].value = std::move(value);
      ToFront(it->second);
      return std::nullopt;
    }
    std::optional<std::pair<Key, Value>> demoted;
    if (active_size() >= capacity_) {
      demoted = Evict();
      if (!demoted.has_value()) return std::nullopt;
    }
    Insert(std::move(key), std::move(value), /*front=*/true);
    return demoted;
  }

  // Inserts at (or moves to) the least-recently-used end. A full cache
  // demotes its tail first; the key is inserted even if nothing could be
  // demoted.
  void PutBack(Key key, Value value) {
    auto it = index_.find(key);
    if (it != index_.end()) {
      nodes_[it->second].value = std::move(value);
      ToBack(it->second);
      return;
    }
    if (active_size() >= capacity_) (void)Evict();
    Insert(std::move(key), std::move(value), /*front=*/false);
  }

  // Promotes to the MRU position (resurrecting a candidate).
  Value* Get(const Key& key) {
    auto it = index_.find(key);
    if (it == index_.end()) return nullptr;
    ToFront(it->second);
    return &nodes_[it->second].value;
  }

  const Value* Peek(const Key& key) const {
    auto it = index_.find(key);
    if (it == index_.end() || nodes_[it->second].loc == NodeLocation::kCandidate) {
      return nullptr;
    }
    return &nodes_[it->second].value;
  }
  Value* PeekMutable(const Key& key) {
    return const_cast<Value*>(static_cast<const LRUCache*>(this)->Peek(key));
  }
  const Value* PeekIncludingCandidates(const Key& key) const {
    auto it = index_.find(key);
    return it == index_.end() ? nullptr : &nodes_[it->second].value;
  }
  Value* PeekMutableIncludingCandidates(const Key& key) {
    auto it = index_.find(key);
    return it == index_.end() ? nullptr : &nodes_[it->second].value;
  }

  // Adds one pin; the first pin moves the entry (active or candidate) to the
  // front of the pinned list.
  Value* GetAndPin(const Key& key) {
    auto it = index_.find(key);
    if (it == index_.end()) return nullptr;
    Node& n = nodes_[it->second];
    if (n.pins == 0) {
      Unlink(it->second);
      LinkAfter(kPin, it->second);
      n.loc = NodeLocation::kPinned;
    }
    ++n.pins;
    return &n.value;
  }
  bool Pin(const Key& key) { return GetAndPin(key) != nullptr; }

  // Drops one pin (clamped at zero); true whenever the key exists.
  bool Unpin(const Key& key) {
    auto it = index_.find(key);
    if (it == index_.end()) return false;
    Node& n = nodes_[it->second];
    if (n.pins > 0 && --n.pins == 0) {
      Unlink(it->second);
      LinkAfter(kActive, it->second);
      n.loc = NodeLocation::kLru;
    }
    return true;
  }

  int GetPinCount(const Key& key) const {
    auto it = index_.find(key);
    return it == index_.end() ? 0 : nodes_[it->second].pins;
  }

  // Up to `count` unpinned keys, oldest first: candidates, then the active
  // list from its tail.
  std::vector<Key> GetEvictableKeys(size_t count) const {
    std::vector<Key> keys;
    for (uint32_t i = nodes_[kCand].next; i != kCand && keys.size() < count;
         i = nodes_[i].next) {
      keys.push_back(nodes_[i].key);
    }
    for (uint32_t i = nodes_[kActive].prev; i != kActive && keys.size() < count;
         i = nodes_[i].prev) {
      keys.push_back(nodes_[i].key);
    }
    return keys;
  }

  // Removes an unpinned entry (active or candidate).
  bool Erase(const Key& key) {
    auto it = index_.find(key);
    if (it == index_.end() || nodes_[it->second].pins > 0) return false;
    const uint32_t i = it->second;
    Unlink(i);
    index_.erase(it);
    Release(i);
    return true;
  }

  // Demotes the active tail to the back of the candidate list.
  std::optional<std::pair<Key, Value>> Evict() {
    const uint32_t i = nodes_[kActive].prev;
    if (i == kActive) return std::nullopt;
    Unlink(i);
    LinkBefore(kCand, i);
    nodes_[i].loc = NodeLocation::kCandidate;
    return std::make_pair(nodes_[i].key, nodes_[i].value);
  }

  std::vector<Key> GetEvictCandidateKeys() const {
    std::vector<Key> keys;
    for (uint32_t i = nodes_[kCand].next; i != kCand; i = nodes_[i].next) {
      keys.push_back(nodes_[i].key);
    }
    return keys;
  }

  // Calls fn(key, value, location) for every entry (no particular order).
  template <typename Fn>
  void ForEach(Fn&& fn) const {
    for (const auto& kv : index_) {
      const Node& n = nodes_[kv.second];
      fn(n.key, n.value, n.loc);
    }
  }

 private:
  // Sentinels of the three circular lists.
  static constexpr uint32_t kActive = 0;
  static constexpr uint32_t kPin = 1;
  static constexpr uint32_t kCand = 2;

  struct Node {
    Key key{};
    Value value{};
    int pins = 0;
    NodeLocation loc = NodeLocation::kLru;
    uint32_t prev = 0;
    uint32_t next = 0;
  };

  void Reset() {
    nodes_.assign(3, Node{});
    for (uint32_t s = 0; s < 3; ++s) nodes_[s].prev = nodes_[s].next = s;
    free_.clear();
    len_[0] = len_[1] = len_[2] = 0;
  }

  static uint32_t ListOf(NodeLocation loc) {
    return loc == NodeLocation::kLru ? kActive
           : loc == NodeLocation::kPinned ? kPin : kCand;
  }

  void Unlink(uint32_t i) {
    Node& n = nodes_[i];
    nodes_[n.prev].next = n.next;
    nodes_[n.next].prev = n.prev;
    --len_[ListOf(n.loc)];
  }
  // Links i right after `at` (a sentinel: the list front) and counts it in
  // the sentinel's list.
  void LinkAfter(uint32_t at, uint32_t i) {
    Node& n = nodes_[i];
    n.prev = at;
    n.next = nodes_[at].next;
    nodes_[n.next].prev = i;
    nodes_[at].next = i;
    ++len_[at];
  }
  // Links i right before sentinel `at` (the list back).
  void LinkBefore(uint32_t at, uint32_t i) {
    Node& n = nodes_[i];
    n.next = at;
    n.prev = nodes_[at].prev;
    nodes_[n.prev].next = i;
    nodes_[at].prev = i;
    ++len_[at];
  }

  // MRU promotion: a pinned entry moves to the pinned front, anything else
  // (active or candidate) to the active front.
  void ToFront(uint32_t i) {
    Node& n = nodes_[i];
    Unlink(i);
    if (n.pins > 0) {
      LinkAfter(kPin, i);
      n.loc = NodeLocation::kPinned;
    } else {
      LinkAfter(kActive, i);
      n.loc = NodeLocation::kLru;
    }
  }
  void ToBack(uint32_t i) {
    Node& n = nodes_[i];
    Unlink(i);
    if (n.pins > 0) {
      LinkBefore(kPin, i);
      n.loc = NodeLocation::kPinned;
    } else {
      LinkBefore(kActive, i);
      n.loc = NodeLocation::kLru;
    }
  }

  void Insert(Key key, Value value, bool front) {
    uint32_t i;
    if (!free_.empty()) {
      i = free_.back();
      free_.pop_back();
    } else {
      i = static_cast<uint32_t>(nodes_.size());
      nodes_.emplace_back();
    }
    Node& n = nodes_[i];
    n.key = key;
    n.value = std::move(value);
    n.pins = 0;
    n.loc = NodeLocation::kLru;
    if (front) {
      LinkAfter(kActive, i);
    } else {
      LinkBefore(kActive, i);
    }
    index_.emplace(std::move(key), i);
  }

  void Release(uint32_t i) {
    nodes_[i].key = Key{};
    nodes_[i].value = Value{};
    nodes_[i].pins = 0;
    free_.push_back(i);
  }

  size_t capacity_;
  std::vector<Node> nodes_;
  std::vector<uint32_t> free_;
  size_t len_[3] = {0, 0, 0};
  std::unordered_map<Key, uint32_t, Hash> index_;
};

}  // namespace kvx

#endif  // KVX_HOST_LRU_CACHE_H_
