// Shared-arena handoff (copy_shared_kv's data path, split_pd_engine.cpp:49-115)
// on the C ABI: host checks, then one run-list kernel per handoff.
#include <algorithm>
#include <stdexcept>
#include <string>
#include <unordered_map>

#include "serving/pd_handoff.h"

namespace serving {
namespace {
using base::error::InvalidArgument;

base::Status abi_error(const char* what) {
  return base::error::InternalError(std::string(what) + ": " + pbe_last_error());
}
}  // namespace

base::Status CopySharedKV(const SharedArenaBinding& arena, uint64_t source_epoch,
                          const KVBlockManifest& manifest, void* stream, uint64_t* copied) {
  if (copied) *copied = 0;
  if (source_epoch == 0 || source_epoch != arena.epoch) return InvalidArgument("PD arena epoch mismatch");
  base::Status status = manifest.validate();
  if (!status) return status;
  const KVPoolDescriptor& pool = manifest.dst_pool;
  // The shared arena holds plain BF16 pages (qwen2.cpp:1124).
  if (pool.dtype != base::DataType::kDataTypeBf16 || pool.storage_mode != base::BlockStorageMode::kPlain)
    return InvalidArgument("PD shared layout mismatch");
  const int32_t layers = pool.layer_num;
  const auto& first = manifest.layer_mappings.front();
  for (size_t i = 0; i < manifest.layer_mappings.size(); ++i) {
    const auto& m = manifest.layer_mappings[i];
    if (m.layer_idx != static_cast<int32_t>(i)) return InvalidArgument("PD shared layout mismatch");
    if (i > 0 && m.src_block_ids != first.src_block_ids)
      return InvalidArgument("PD page-major layer IDs disagree");
    if (i > 0 && m.dst_block_ids != first.dst_block_ids)
      return InvalidArgument("PD destination is not page-major");
  }
  const pbe_kv_shape shape{layers, pool.kv_head_num, pool.head_size, pool.block_size};
  const int64_t n = static_cast<int64_t>(first.src_block_ids.size());
  int64_t bad = -1;
  if (pbe_validate_ids(first.src_block_ids.data(), n, &shape, 2, arena.view.bytes, &bad) != PBE_OK)
    return InvalidArgument("PD source block outside shared page layout");
  if (pbe_validate_ids(first.dst_block_ids.data(), n, &shape, 2, arena.view.bytes, &bad) != PBE_OK)
    return InvalidArgument("PD destination block outside shared page layout");
  uint64_t bytes = 0;
  const int rc = pbe_copy_shared_kv(&arena.view, first.src_block_ids.data(), first.dst_block_ids.data(),
                                    n, &shape, arena.device, stream, &bytes);
  if (rc == PBE_ERR_INVALID) return InvalidArgument(pbe_last_error());
  if (rc != PBE_OK) return abi_error("PD copy launch failed; discard the IPC domain");
  if (copied) *copied = bytes;
  return base::error::Success();
}

base::Status TakeOverSharedKV(base::SharedKVPageGroup* group, const SharedArenaBinding& arena,
                              const base::SharedKVPageGroup::PageTakeover& takeover,
                              const KVPoolDescriptor& pool, void* stream,
                              std::vector<int32_t>* block_table, uint64_t* copied) {
  if (copied) *copied = 0;
  if (!group || !block_table) return InvalidArgument("takeover group or block table is null");
  block_table->clear();
  if (pool.layer_num != group->layers()) return InvalidArgument("PD layer count mismatch");
  try {
    group->adopt(takeover);
  } catch (const base::ChunkAllocationError& e) {
    return InvalidArgument(e.what());
  } catch (const std::exception& e) {
    return InvalidArgument(e.what());
  }
  const int layers = group->layers();
  std::vector<int32_t> fresh;
  for (size_t i = 0; i < takeover.copy_ids.size(); ++i) {
    const int id = group->allocate(0);
    if (id < 0) {
      for (int32_t f : fresh) group->retire(0, f);  // layer 0 retire rolls back the reservations
      return InvalidArgument("model_kv_quota_exhausted");
    }
    fresh.push_back(id);
  }
  for (int l = 1; l < layers; ++l)
    for (size_t i = 0; i < fresh.size(); ++i) group->allocate(l);
  std::unordered_map<int32_t, int32_t> replace;
  for (size_t i = 0; i < fresh.size(); ++i) replace[takeover.copy_ids[i]] = fresh[i];
  for (int32_t id : takeover.page_ids) {
    auto r = replace.find(id);
    block_table->push_back(r == replace.end() ? id : r->second);
  }
  if (fresh.empty()) return base::error::Success();
  KVBlockManifest manifest;
  manifest.client_request_id.value = "page-takeover";
  manifest.handoff_id.value = 1;
  manifest.src_pool = manifest.dst_pool = pool;
  manifest.computed_tokens = static_cast<int32_t>(fresh.size()) * pool.block_size;
  manifest.prompt_tokens = manifest.computed_tokens;
  for (int l = 0; l < layers; ++l) manifest.layer_mappings.push_back({l, takeover.copy_ids, fresh});
  return CopySharedKV(arena, takeover.epoch, manifest, stream, copied);
}

SharedArenaKVTransferConnector::SharedArenaKVTransferConnector(SharedArenaBinding arena, void* stream)
    : arena_(arena), stream_(stream) {
  if (!stream_) {
    if (pbe_stream_create(arena_.device, &stream_) != PBE_OK)
      throw std::runtime_error(std::string("shared-arena connector stream: ") + pbe_last_error());
    owns_stream_ = true;
  }
}

SharedArenaKVTransferConnector::~SharedArenaKVTransferConnector() {
  // A copy whose completion cannot be proven may still write the arena.
  if (pbe_stream_synchronize(arena_.device, stream_) != PBE_OK) std::terminate();
  for (auto& r : records_)
    if (r.done) pbe_event_destroy(r.done);
  if (owns_stream_) pbe_stream_destroy(arena_.device, stream_);
}

base::Status SharedArenaKVTransferConnector::submit(const KVBlockManifest& manifest, HandoffId* handle) {
  return submit_from(arena_.epoch, manifest, handle);
}

base::Status SharedArenaKVTransferConnector::submit_from(uint64_t source_epoch,
                                                         const KVBlockManifest& manifest,
                                                         HandoffId* handle) {
  if (handle == nullptr) return InvalidArgument("shared-arena connector submit handle is null");
  *handle = {next_handoff_id_++};
  uint64_t bytes = 0;
  base::Status status = CopySharedKV(arena_, source_epoch, manifest, stream_, &bytes);
  if (!status) {
    records_.push_back({*handle, KVTransferStatus::Failed(status.get_err_msg()), nullptr, false, ""});
    return status;
  }
  pbe_event* done = nullptr;
  if (pbe_event_create(arena_.device, 0, &done) != PBE_OK || pbe_event_record(done, stream_) != PBE_OK) {
    if (done) pbe_event_destroy(done);
    // The copy is queued but its completion cannot be observed: fence the stream.
    if (pbe_stream_synchronize(arena_.device, stream_) != PBE_OK) std::terminate();
    records_.push_back({*handle, KVTransferStatus::Completed(), nullptr, false, ""});
    copied_bytes_ += bytes;
    return base::error::Success();
  }
  copied_bytes_ += bytes;
  records_.push_back({*handle, KVTransferStatus::Pending(), done, false, ""});
  return base::error::Success();
}

SharedArenaKVTransferConnector::Record* SharedArenaKVTransferConnector::find(HandoffId handle) {
  for (auto& r : records_)
    if (r.handle.value == handle.value) return &r;
  return nullptr;
}

KVTransferStatus SharedArenaKVTransferConnector::settle(Record& r, bool wait) {
  if (r.status.done() || !r.done) return r.status;
  const int rc = wait ? pbe_event_synchronize(r.done) : pbe_event_query(r.done);
  if (rc == PBE_NOT_READY) return r.status;
  pbe_event_destroy(r.done);
  r.done = nullptr;
  if (rc != PBE_OK) r.status = KVTransferStatus::Failed(pbe_last_error());
  else if (r.cancel_requested) r.status = KVTransferStatus::Cancelled(r.cancel_reason);
  else r.status = KVTransferStatus::Completed();
  return r.status;
}

KVTransferStatus SharedArenaKVTransferConnector::poll(HandoffId handle) {
  Record* r = find(handle);
  if (!r) return KVTransferStatus::Failed("shared-arena connector unknown handoff id");
  return settle(*r, false);
}

void SharedArenaKVTransferConnector::cancel(HandoffId handle, const std::string& reason) {
  Record* r = find(handle);
  if (r && !r->status.done()) {
    r->cancel_requested = true;
    r->cancel_reason = reason;
  }
}

KVTransferStatus SharedArenaKVTransferConnector::drain(HandoffId handle) {
  Record* r = find(handle);
  if (!r) return KVTransferStatus::Failed("unknown handoff id");
  return settle(*r, true);
}

void SharedArenaKVTransferConnector::release(HandoffId handle) {
  auto it = std::find_if(records_.begin(), records_.end(),
                         [&](const Record& r) { return r.handle.value == handle.value; });
  if (it != records_.end() && it->status.done() && it->done == nullptr) records_.erase(it);
}

}  // namespace serving
