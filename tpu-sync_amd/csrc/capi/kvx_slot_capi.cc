// extern "C" surface of the copy-spec builders and the staging-slot pool
// (declared in include/kvx.h).
#include <cstdint>
#include <vector>

#include "../host/copy_plan.h"
#include "capi_internal.h"

using kvx_capi::BadArray;
using kvx_capi::Done;
using kvx_capi::Fail;

namespace {

std::vector<int64_t> Vec(const int64_t* p, int64_t n) {
  return n > 0 ? std::vector<int64_t>(p, p + n) : std::vector<int64_t>();
}

void PutSpec(const kvx::CopySpec& s, int64_t* src, int64_t* dst, int64_t* sizes,
             int64_t* n_runs) {
  for (size_t i = 0; i < s.sizes.size(); ++i) {
    src[i] = s.src_offsets[i];
    dst[i] = s.dst_offsets[i];
    sizes[i] = s.sizes[i];
  }
  *n_runs = static_cast<int64_t>(s.sizes.size());
}

bool BadSpecOut(int64_t n, const int64_t* a, const int64_t* b, const int64_t* c,
                const int64_t* count) {
  return count == nullptr || BadArray(a, n) || BadArray(b, n) || BadArray(c, n);
}

int PutPlan(const kvx::CopyPlan& p, int64_t n, kvx_load_plan_out* o) {
  if (o == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null plan output");
  if (BadArray(o->producer_remote_block_ids, n) || BadArray(o->transport_host_block_ids, n) ||
      BadArray(o->h2d_local_block_ids, n) || BadArray(o->h2d_host_block_ids, n) ||
      BadArray(o->h2d_src, n) || BadArray(o->h2d_dst, n) || BadArray(o->h2d_sizes, n)) {
    return Fail(KVX_INVALID_ARGUMENT, "null plan array with a positive length");
  }
  for (size_t i = 0; i < p.producer_remote_block_ids.size(); ++i) {
    o->producer_remote_block_ids[i] = p.producer_remote_block_ids[i];
    o->transport_host_block_ids[i] = p.transport_host_block_ids[i];
  }
  for (size_t i = 0; i < p.h2d_local_block_ids.size(); ++i) {
    o->h2d_local_block_ids[i] = p.h2d_local_block_ids[i];
    o->h2d_host_block_ids[i] = p.h2d_host_block_ids[i];
  }
  o->num_h2d = static_cast<int64_t>(p.h2d_local_block_ids.size());
  PutSpec(p.h2d_copy, o->h2d_src, o->h2d_dst, o->h2d_sizes, &o->num_runs);
  return KVX_OK;
}

}  // namespace

extern "C" {

int kvx_offsets_impl(const int64_t* ids, int64_t n, int32_t source_is_compact,
                     int64_t* out_src, int64_t* out_dst, int64_t* out_sizes,
                     int64_t* n_runs) {
  if (BadArray(ids, n) || BadSpecOut(n, out_src, out_dst, out_sizes, n_runs)) {
    return Fail(KVX_INVALID_ARGUMENT, "null array with a positive length");
  }
  PutSpec(kvx::OffsetsImpl(Vec(ids, n), source_is_compact != 0), out_src, out_dst,
          out_sizes, n_runs);
  return KVX_OK;
}

int kvx_build_coalesced_copy_spec(const int64_t* src_ids, const int64_t* dst_ids,
                                  int64_t n, int64_t* out_src, int64_t* out_dst,
                                  int64_t* out_sizes, int64_t* n_runs) {
  if (BadArray(src_ids, n) || BadArray(dst_ids, n) ||
      BadSpecOut(n, out_src, out_dst, out_sizes, n_runs)) {
    return Fail(KVX_INVALID_ARGUMENT, "null array with a positive length");
  }
  auto r = kvx::BuildCoalescedCopySpec(Vec(src_ids, n), Vec(dst_ids, n));
  if (!r.ok()) return Fail(r.status());
  PutSpec(*r, out_src, out_dst, out_sizes, n_runs);
  return KVX_OK;
}

int kvx_build_load_copy_plan(const int64_t* remote, const int64_t* local,
                             const int64_t* host, int64_t n, kvx_load_plan_out* out) {
  if (BadArray(remote, n) || BadArray(local, n) || BadArray(host, n)) {
    return Fail(KVX_INVALID_ARGUMENT, "null array with a positive length");
  }
  auto r = kvx::BuildLoadCopyPlan(Vec(remote, n), Vec(local, n), Vec(host, n));
  if (!r.ok()) return Fail(r.status());
  return PutPlan(*r, n, out);
}

int kvx_manager_initialize_slot_pool(kvx_manager* m, int64_t num_slots) {
  if (m == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null manager");
  return Done(m->impl->InitializeSlotPool(num_slots));
}

int kvx_manager_acquire_slot(kvx_manager* m, int64_t* out_slot_idx) {
  if (m == nullptr || out_slot_idx == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null argument");
  auto r = m->impl->AcquireSlot();
  if (!r.ok()) return Fail(r.status());
  *out_slot_idx = r->slot_idx;
  return KVX_OK;
}

void kvx_manager_release_slot(kvx_manager* m, int64_t slot_idx) {
  if (m != nullptr) m->impl->ReleaseSlot(slot_idx);
}

int64_t kvx_manager_num_free_slots(kvx_manager* m) {
  return m == nullptr ? -1 : m->impl->num_free_slots();
}

int kvx_manager_slot_block_ids(kvx_manager* m, int64_t slot_idx, int64_t* out, int64_t cap,
                               int64_t* n_out) {
  if (m == nullptr || n_out == nullptr || BadArray(out, cap)) {
    return Fail(KVX_INVALID_ARGUMENT, "null argument");
  }
  auto r = m->impl->SlotBlockIds(slot_idx);
  if (!r.ok()) return Fail(r.status());
  *n_out = static_cast<int64_t>(r->size());
  for (int64_t i = 0; i < *n_out && i < cap; ++i) out[i] = (*r)[static_cast<size_t>(i)];
  return KVX_OK;
}

int kvx_manager_layer_spans(kvx_manager* m, int64_t slot_idx, int64_t num_blocks,
                            kvx_host_span* out, int64_t cap, int64_t* n_out) {
  if (m == nullptr || n_out == nullptr || BadArray(out, cap)) {
    return Fail(KVX_INVALID_ARGUMENT, "null argument");
  }
  auto r = m->impl->LayerSpans(slot_idx, num_blocks);
  if (!r.ok()) return Fail(r.status());
  *n_out = static_cast<int64_t>(r->size());
  for (int64_t i = 0; i < *n_out && i < cap; ++i) {
    const kvx::KVCacheHostSpan& s = (*r)[static_cast<size_t>(i)];
    out[i] = kvx_host_span{reinterpret_cast<uint64_t>(s.ptr),
                           static_cast<int64_t>(s.nbytes),
                           s.slot_idx,
                           s.base_major,
                           s.num_major,
                           static_cast<int64_t>(s.layer_idx),
                           static_cast<int64_t>(s.shard_idx)};
  }
  return KVX_OK;
}

int kvx_manager_issue_h2d(kvx_manager* m, int64_t slot_idx, int64_t num_blocks,
                          const int64_t* local_ids, int64_t n, void* stream,
                          kvx_future** out, int64_t* out_total_bytes,
                          int64_t* out_copy_segments) {
  if (m == nullptr || out == nullptr || BadArray(local_ids, n)) {
    return Fail(KVX_INVALID_ARGUMENT, "null argument");
  }
  auto r = m->impl->IssueH2D(slot_idx, num_blocks, Vec(local_ids, n),
                             static_cast<hipStream_t>(stream));
  if (!r.ok()) return Fail(r.status());
  if (out_total_bytes != nullptr) *out_total_bytes = r->total_bytes;
  if (out_copy_segments != nullptr) *out_copy_segments = r->copy_segments;
  *out = new kvx_future{std::move(r->future)};
  return KVX_OK;
}

int kvx_manager_stage_for_push(kvx_manager* m, const int64_t* src_ids, int64_t n,
                               void* stream, int64_t* out_slot_idx, int64_t* out_host_ids,
                               kvx_future** out_layer_futures, int64_t* out_copy_segments) {
  if (m == nullptr || out_slot_idx == nullptr || BadArray(src_ids, n) ||
      BadArray(out_host_ids, n) || out_layer_futures == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null argument");
  }
  auto r = m->impl->StageForPush(Vec(src_ids, n), static_cast<hipStream_t>(stream));
  if (!r.ok()) return Fail(r.status());
  *out_slot_idx = r->slot_idx;
  for (size_t i = 0; i < r->host_block_ids.size(); ++i) out_host_ids[i] = r->host_block_ids[i];
  const size_t layers = m->impl->num_layers();
  for (size_t l = 0; l < layers; ++l) {
    out_layer_futures[l] =
        new kvx_future{l < r->layer_futures.size() ? r->layer_futures[l] : kvx::CopyFuture()};
  }
  if (out_copy_segments != nullptr) *out_copy_segments = r->copy_segments;
  return KVX_OK;
}

int kvx_manager_prepare_load(kvx_manager* m, const int64_t* remote_ids,
                             const int64_t* local_ids, int64_t n, const int64_t* host_ids,
                             int64_t* out_slot_idx, int64_t* out_host_ids,
                             kvx_load_plan_out* out_plan) {
  if (m == nullptr || out_slot_idx == nullptr || BadArray(remote_ids, n) ||
      BadArray(local_ids, n) || BadArray(out_host_ids, n)) {
    return Fail(KVX_INVALID_ARGUMENT, "null argument");
  }
  std::vector<int64_t> host;
  if (host_ids != nullptr) host = Vec(host_ids, n);
  auto r = m->impl->PrepareLoad(Vec(remote_ids, n), Vec(local_ids, n),
                                host_ids != nullptr ? &host : nullptr);
  if (!r.ok()) return Fail(r.status());
  const int rc = PutPlan(r->plan, n, out_plan);
  if (rc != KVX_OK) {
    if (r->slot_idx >= 0) m->impl->ReleaseSlot(r->slot_idx);
    return rc;
  }
  *out_slot_idx = r->slot_idx;
  for (size_t i = 0; i < r->host_block_ids.size(); ++i) out_host_ids[i] = r->host_block_ids[i];
  return KVX_OK;
}

}  // extern "C"
