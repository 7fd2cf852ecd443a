// Generic plan form of the handoff over arena pools:
// bind_manifest_transfers (infMain/source/serving/pd_handoff_common.cpp:64-153)
// and InProcKVBlockCopyConnector (infMain/source/serving/pd_handoff.cpp:80-213),
// with the per-op memcpy loop replaced by one op-list kernel per handoff.
#include <algorithm>
#include <numeric>
#include <stdexcept>
#include <string>

#include "cache/layout_codec.h"
#include "cache/page_schema.h"
#include "serving/pd_handoff.h"

namespace serving {
namespace {
using base::error::InvalidArgument;

// Byte address of `offset` in a (possibly segmented) view; the span
// [offset, offset+len) must stay inside one segment.
bool address_of(const pbe_arena_view& v, uint64_t offset, uint64_t len, uint8_t** out) {
  if (v.segment_bytes == 0 || offset > v.bytes || len > v.bytes - offset) return false;
  const uint64_t seg = offset / v.segment_bytes, in = offset % v.segment_bytes;
  if (seg >= v.nseg || len > v.segment_bytes - in) return false;
  *out = static_cast<uint8_t*>(v.base[seg]) + in;
  return true;
}

// Component address of (layer, kind) of block `id` in a page-major pool.
bool component_address(const ArenaKVPool& p, const cache::ComponentDescriptor& c, int32_t id,
                       uint8_t** out) {
  const KVPoolDescriptor& d = p.pool;
  const auto storage = base::MakeKVCacheStorageSpec(d.dtype, d.storage_mode);
  const uint64_t half = static_cast<uint64_t>(d.block_size) * d.kv_head_num * d.head_size *
                        base::DataTypeSize(storage.storage_dtype);
  const uint64_t plane = 2ull * c.layer + (c.kind == cache::ComponentKind::kValue ||
                                            c.kind == cache::ComponentKind::kValueScale);
  if (id < 0 || id % (2 * d.layer_num)) return false;
  if (c.kind == cache::ComponentKind::kKey || c.kind == cache::ComponentKind::kValue)
    return address_of(p.view, (static_cast<uint64_t>(id) + plane) * half, half, out);
  // scales: [page][layer][K|V][token][head] fp32
  if (!p.scales) return false;
  const uint64_t rows = static_cast<uint64_t>(d.block_size) * d.kv_head_num;
  const uint64_t page = static_cast<uint64_t>(id) / (2ull * d.layer_num);
  const uint64_t off = (page * 2ull * d.layer_num + plane) * rows * 4u;
  if (off > p.scale_bytes || rows * 4u > p.scale_bytes - off) return false;
  *out = static_cast<uint8_t*>(p.scales) + off;
  return true;
}
}  // namespace

base::Status BindManifestTransfers(const KVBlockManifest& manifest, const ArenaKVPool& source,
                                   const ArenaKVPool& destination, cache::TransferPlanner* planner,
                                   std::vector<cache::BoundTransfer>* transfers) {
  if (!planner || !transfers || !transfers->empty())
    return InvalidArgument("invalid semantic transfer binding arguments");
  const int32_t layers = source.pool.layer_num;
  if (layers != destination.pool.layer_num || static_cast<int32_t>(manifest.layer_mappings.size()) != layers)
    return InvalidArgument("semantic transfer layer coverage mismatch");
  std::vector<const KVBlockMapping*> by_layer(layers, nullptr);
  size_t pages = 0;
  for (const auto& m : manifest.layer_mappings) {
    if (m.layer_idx < 0 || m.layer_idx >= layers || by_layer[m.layer_idx] ||
        m.src_block_ids.size() != m.dst_block_ids.size())
      return InvalidArgument("semantic transfer mapping is incomplete or duplicate");
    if (pages && pages != m.src_block_ids.size())
      return InvalidArgument("semantic transfer page coverage mismatch");
    pages = m.src_block_ids.size();
    by_layer[m.layer_idx] = &m;
  }
  if (!pages) return InvalidArgument("semantic transfer has no pages");

  cache::PageSchema src_schema, dst_schema;
  auto schema_of = [](const KVPoolDescriptor& d, cache::PageSchema* out) {
    return cache::MakeKVPageSchema(1, d.layer_num, d.block_size, d.kv_head_num, d.head_size,
                                   base::MakeKVCacheStorageSpec(d.dtype, d.storage_mode), out);
  };
  base::Status status = schema_of(source.pool, &src_schema);
  if (!status) return status;
  status = schema_of(destination.pool, &dst_schema);
  if (!status) return status;
  std::shared_ptr<const cache::TransferPlan> plan;
  status = planner->compile(src_schema, dst_schema, cache::TransferPlacement::kExactDirect, &plan);
  if (!status) return status;
  std::vector<size_t> src_order(src_schema.components.size()), dst_order(dst_schema.components.size());
  std::iota(src_order.begin(), src_order.end(), 0);
  std::iota(dst_order.begin(), dst_order.end(), 0);
  cache::LayoutDescriptor src_layout, dst_layout;
  status = cache::MakePackedLayout(src_schema, "pd-source", 1, src_order, {}, &src_layout);
  if (!status) return status;
  status = cache::MakePackedLayout(dst_schema, "pd-destination", 1, dst_order, {}, &dst_layout);
  if (!status) return status;

  std::vector<cache::BoundTransfer> bound;
  bound.reserve(pages);
  for (size_t page = 0; page < pages; ++page) {
    cache::ConstComponentEndpoint src{{}, &src_layout};
    cache::MutableComponentEndpoint dst{{}, &dst_layout};
    src.components.reserve(src_schema.components.size());
    dst.components.reserve(dst_schema.components.size());
    for (const auto& c : src_schema.components) {
      uint8_t* a = nullptr;
      if (!component_address(source, c, by_layer[c.layer]->src_block_ids[page], &a))
        return InvalidArgument("source block outside its page-major arena");
      src.components.push_back({c, a, c.byte_size()});
    }
    for (const auto& c : dst_schema.components) {
      uint8_t* a = nullptr;
      if (!component_address(destination, c, by_layer[c.layer]->dst_block_ids[page], &a))
        return InvalidArgument("destination block outside its page-major arena");
      dst.components.push_back({c, a, c.byte_size()});
    }
    cache::BoundTransfer t;
    status = cache::BoundTransfer::BindComponents(*plan, src_schema, dst_schema, src, dst, &t);
    if (!status) return status;
    bound.push_back(std::move(t));
  }
  *transfers = std::move(bound);
  return base::error::Success();
}

InProcKVBlockCopyConnector::InProcKVBlockCopyConnector(ArenaKVPool source, ArenaKVPool destination,
                                                       int device, void* stream)
    : source_(source), destination_(destination), device_(device), stream_(stream) {
  if (!stream_) {
    if (pbe_stream_create(device_, &stream_) != PBE_OK)
      throw std::runtime_error(std::string("block copy connector stream: ") + pbe_last_error());
    owns_stream_ = true;
  }
}

InProcKVBlockCopyConnector::~InProcKVBlockCopyConnector() {
  if (pbe_stream_synchronize(device_, stream_) != PBE_OK) std::terminate();
  for (auto& r : records_)
    if (r.done) pbe_event_destroy(r.done);
  if (owns_stream_) pbe_stream_destroy(device_, stream_);
}

base::Status InProcKVBlockCopyConnector::submit(const KVBlockManifest& manifest, HandoffId* handle) {
  if (handle == nullptr) return InvalidArgument("pd block copy connector submit handle is null");
  base::Status status = manifest.validate();
  if (!status) return status;
  *handle = {next_handoff_id_++};
  std::vector<cache::BoundTransfer> transfers;
  status = BindManifestTransfers(manifest, source_, destination_, &planner_, &transfers);
  std::vector<pbe_copy_op> ops;
  uint64_t bytes = 0;
  if (status) {
    for (const auto& t : transfers)
      for (const auto& op : t.operations()) {
        ops.push_back({reinterpret_cast<uint64_t>(op.source), reinterpret_cast<uint64_t>(op.destination),
                       op.bytes});
        bytes += op.bytes;
      }
    const int rc = pbe_copy_ops(ops.data(), static_cast<int64_t>(ops.size()), device_, stream_);
    if (rc == PBE_ERR_INVALID) status = InvalidArgument(pbe_last_error());
    else if (rc != PBE_OK) status = base::error::InternalError(pbe_last_error());
  }
  if (!status) {
    records_.push_back({*handle, KVTransferStatus::Failed(status.get_err_msg()), nullptr, false, ""});
    return status;
  }
  last_ops_ = ops.size();
  copied_bytes_ += bytes;
  pbe_event* done = nullptr;
  if (pbe_event_create(device_, 0, &done) != PBE_OK || pbe_event_record(done, stream_) != PBE_OK) {
    if (done) pbe_event_destroy(done);
    if (pbe_stream_synchronize(device_, stream_) != PBE_OK) std::terminate();
    records_.push_back({*handle, KVTransferStatus::Completed(), nullptr, false, ""});
    return base::error::Success();
  }
  records_.push_back({*handle, KVTransferStatus::Pending(), done, false, ""});
  return base::error::Success();
}

InProcKVBlockCopyConnector::Record* InProcKVBlockCopyConnector::find(HandoffId handle) {
  for (auto& r : records_)
    if (r.handle.value == handle.value) return &r;
  return nullptr;
}

KVTransferStatus InProcKVBlockCopyConnector::settle(Record& r, bool wait) {
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

KVTransferStatus InProcKVBlockCopyConnector::poll(HandoffId handle) {
  Record* r = find(handle);
  if (!r) return KVTransferStatus::Failed("pd block copy connector unknown handoff id");
  return settle(*r, false);
}

void InProcKVBlockCopyConnector::cancel(HandoffId handle, const std::string& reason) {
  Record* r = find(handle);
  if (r && !r->status.done()) {
    r->cancel_requested = true;
    r->cancel_reason = reason;
  }
}

KVTransferStatus InProcKVBlockCopyConnector::drain(HandoffId handle) {
  Record* r = find(handle);
  if (!r) return KVTransferStatus::Failed("unknown handoff id");
  return settle(*r, true);
}

void InProcKVBlockCopyConnector::release(HandoffId handle) {
  auto it = std::find_if(records_.begin(), records_.end(),
                         [&](const Record& r) { return r.handle.value == handle.value; });
  if (it != records_.end() && it->status.done() && it->done == nullptr) records_.erase(it);
}

}  // namespace serving
