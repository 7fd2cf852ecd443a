// Generic plan form of the handoff over arena pools:
// bind_manifest_transfers (infMain/source/serving/pd_handoff_common.cpp:64-153)
// and InProcKVBlockCopyConnector (infMain/source/serving/pd_handoff.cpp:80-213),
// with the per-op memcpy loop replaced by one op-list kernel per handoff.
#include <algorithm>
#include <memory>
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

// Byte geometry of a page-major pool.
struct PoolGeometry {
  uint64_t half = 0;        // one K or V plane of one block
  uint64_t scale_rows = 0;  // fp32 scales per plane: block_size * kv_heads
  int64_t stride = 0;       // block ids per page: 2 * layers
};

PoolGeometry geometry_of(const ArenaKVPool& p) {
  const KVPoolDescriptor& d = p.pool;
  const auto storage = base::MakeKVCacheStorageSpec(d.dtype, d.storage_mode);
  PoolGeometry g;
  g.half = static_cast<uint64_t>(d.block_size) * d.kv_head_num * d.head_size *
           base::DataTypeSize(storage.storage_dtype);
  g.scale_rows = static_cast<uint64_t>(d.block_size) * d.kv_head_num;
  g.stride = 2ll * d.layer_num;
  return g;
}

// The block id a pool's lookups last saw and, when that id is a page id whose
// whole page span [id, id + stride) lies in one segment of the view, the
// span's base: the page's planes are then base + plane * half, with no
// segment division per component (every layer of a page-major manifest
// shares the id, so a page costs one lookup per pool).
struct PageMemo {
  int32_t id = -1;
  bool page_id = false;
  uint8_t* base = nullptr;
};

// Component address of (layer, kind) of block `id` in a page-major pool.
bool component_address(const ArenaKVPool& p, const PoolGeometry& g, const cache::ComponentDescriptor& c,
                       int32_t id, PageMemo* memo, uint8_t** out) {
  const uint64_t plane = 2ull * c.layer + (c.kind == cache::ComponentKind::kValue ||
                                            c.kind == cache::ComponentKind::kValueScale);
  if (id != memo->id) {
    memo->id = id;
    memo->page_id = id >= 0 && id % g.stride == 0;
    memo->base = nullptr;
    uint8_t* a = nullptr;
    if (memo->page_id &&
        address_of(p.view, static_cast<uint64_t>(id) * g.half, static_cast<uint64_t>(g.stride) * g.half, &a))
      memo->base = a;
  }
  if (!memo->page_id) return false;
  if (c.kind == cache::ComponentKind::kKey || c.kind == cache::ComponentKind::kValue) {
    // a plane of a page inside one segment is inside it too; otherwise the
    // plane is checked on its own (a page may cross a segment boundary
    // while each plane stays inside one)
    if (memo->base && plane < static_cast<uint64_t>(g.stride)) {
      *out = memo->base + plane * g.half;
      return true;
    }
    return address_of(p.view, (static_cast<uint64_t>(id) + plane) * g.half, g.half, out);
  }
  // scales: [page][layer][K|V][token][head] fp32
  if (!p.scales) return false;
  const uint64_t page = static_cast<uint64_t>(id) / static_cast<uint64_t>(g.stride);
  const uint64_t off = (page * static_cast<uint64_t>(g.stride) + plane) * g.scale_rows * 4u;
  if (off > p.scale_bytes || g.scale_rows * 4u > p.scale_bytes - off) return false;
  *out = static_cast<uint8_t*>(p.scales) + off;
  return true;
}
}  // namespace

namespace {

// What every page of a manifest shares: its layer mappings, both schemas,
// the compiled plan and both packed layouts.
struct ManifestBinding {
  PoolGeometry src_geo, dst_geo;
  std::vector<const KVBlockMapping*> by_layer;
  size_t pages = 0;
  cache::PageSchema src_schema, dst_schema;
  std::shared_ptr<const cache::TransferPlan> plan;
  cache::LayoutDescriptor src_layout, dst_layout;
  std::vector<size_t> src_bytes, dst_bytes;  // byte_size() of each schema component
};

// The manifest's mapping of each layer and its page count, checked against
// the pools' layer count.
base::Status map_layers(const KVBlockManifest& manifest, const ArenaKVPool& source,
                        const ArenaKVPool& destination, std::vector<const KVBlockMapping*>* by_layer,
                        size_t* pages) {
  const int32_t layers = source.pool.layer_num;
  if (layers != destination.pool.layer_num || static_cast<int32_t>(manifest.layer_mappings.size()) != layers)
    return InvalidArgument("semantic transfer layer coverage mismatch");
  by_layer->assign(layers, nullptr);
  *pages = 0;
  for (const auto& m : manifest.layer_mappings) {
    if (m.layer_idx < 0 || m.layer_idx >= layers || (*by_layer)[m.layer_idx] ||
        m.src_block_ids.size() != m.dst_block_ids.size())
      return InvalidArgument("semantic transfer mapping is incomplete or duplicate");
    if (*pages && *pages != m.src_block_ids.size())
      return InvalidArgument("semantic transfer page coverage mismatch");
    *pages = m.src_block_ids.size();
    (*by_layer)[m.layer_idx] = &m;
  }
  if (!*pages) return InvalidArgument("semantic transfer has no pages");
  return base::error::Success();
}

base::Status prepare(const KVBlockManifest& manifest, const ArenaKVPool& source,
                     const ArenaKVPool& destination, cache::TransferPlanner* planner, ManifestBinding* b) {
  base::Status status = map_layers(manifest, source, destination, &b->by_layer, &b->pages);
  if (!status) return status;
  b->src_geo = geometry_of(source);
  b->dst_geo = geometry_of(destination);

  auto schema_of = [](const KVPoolDescriptor& d, cache::PageSchema* out) {
    return cache::MakeKVPageSchema(1, d.layer_num, d.block_size, d.kv_head_num, d.head_size,
                                   base::MakeKVCacheStorageSpec(d.dtype, d.storage_mode), out);
  };
  status = schema_of(source.pool, &b->src_schema);
  if (!status) return status;
  status = schema_of(destination.pool, &b->dst_schema);
  if (!status) return status;
  status = planner->compile(b->src_schema, b->dst_schema, cache::TransferPlacement::kExactDirect, &b->plan);
  if (!status) return status;
  for (const auto& c : b->src_schema.components) b->src_bytes.push_back(c.byte_size());
  for (const auto& c : b->dst_schema.components) b->dst_bytes.push_back(c.byte_size());
  std::vector<size_t> src_order(b->src_schema.components.size()), dst_order(b->dst_schema.components.size());
  std::iota(src_order.begin(), src_order.end(), 0);
  std::iota(dst_order.begin(), dst_order.end(), 0);
  status = cache::MakePackedLayout(b->src_schema, "pd-source", 1, src_order, {}, &b->src_layout);
  if (!status) return status;
  return cache::MakePackedLayout(b->dst_schema, "pd-destination", 1, dst_order, {}, &b->dst_layout);
}

// Component endpoints of one page: its blocks' component addresses.
base::Status endpoints(const ManifestBinding& b, const ArenaKVPool& source, const ArenaKVPool& destination,
                       size_t page, cache::ConstComponentEndpoint* src, cache::MutableComponentEndpoint* dst) {
  src->layout = &b.src_layout;
  dst->layout = &b.dst_layout;
  src->components.clear();
  dst->components.clear();
  src->components.reserve(b.src_schema.components.size());
  dst->components.reserve(b.dst_schema.components.size());
  PageMemo src_memo, dst_memo;
  for (size_t i = 0; i < b.src_schema.components.size(); ++i) {
    const auto& c = b.src_schema.components[i];
    uint8_t* a = nullptr;
    if (!component_address(source, b.src_geo, c, b.by_layer[c.layer]->src_block_ids[page], &src_memo, &a))
      return InvalidArgument("source block outside its page-major arena");
    src->components.push_back({c, a, b.src_bytes[i]});
  }
  for (size_t i = 0; i < b.dst_schema.components.size(); ++i) {
    const auto& c = b.dst_schema.components[i];
    uint8_t* a = nullptr;
    if (!component_address(destination, b.dst_geo, c, b.by_layer[c.layer]->dst_block_ids[page], &dst_memo, &a))
      return InvalidArgument("destination block outside its page-major arena");
    dst->components.push_back({c, a, b.dst_bytes[i]});
  }
  return base::error::Success();
}

// Index of the span holding [p, p + bytes).
template <typename Span>
size_t span_holding(const std::vector<Span>& spans, const uint8_t* p, size_t bytes) {
  for (size_t i = 0; i < spans.size(); ++i) {
    const uint8_t* begin = spans[i].data;
    if (p >= begin && bytes <= spans[i].bytes && static_cast<size_t>(p - begin) <= spans[i].bytes - bytes)
      return i;
  }
  return spans.size();
}

}  // namespace

base::Status BindManifestTransfers(const KVBlockManifest& manifest, const ArenaKVPool& source,
                                   const ArenaKVPool& destination, cache::TransferPlanner* planner,
                                   std::vector<cache::BoundTransfer>* transfers) {
  if (!planner || !transfers || !transfers->empty())
    return InvalidArgument("invalid semantic transfer binding arguments");
  ManifestBinding b;
  base::Status status = prepare(manifest, source, destination, planner, &b);
  if (!status) return status;
  std::vector<cache::BoundTransfer> bound;
  bound.reserve(b.pages);
  cache::ConstComponentEndpoint src;
  cache::MutableComponentEndpoint dst;
  for (size_t page = 0; page < b.pages; ++page) {
    status = endpoints(b, source, destination, page, &src, &dst);
    if (!status) return status;
    cache::BoundTransfer t;
    status = cache::BoundTransfer::BindComponents(*b.plan, b.src_schema, b.dst_schema, src, dst, &t);
    if (!status) return status;
    bound.push_back(std::move(t));
  }
  *transfers = std::move(bound);
  return base::error::Success();
}

// What the copy ops of any manifest between two pools share: the pools'
// binding (schemas, plan, layouts; no layer mapping) and the first bound
// page's operations as (component span, offset) pieces. Every page follows
// the pieces at its own component addresses.
struct CopyOpTemplate {
  struct Piece {
    size_t src_span, dst_span;
    uint64_t src_off, dst_off, bytes;
  };
  ManifestBinding pools;  // by_layer cleared: the template outlives its manifest
  std::vector<Piece> pieces;
};

namespace {

// Binds page 0 of `b`'s manifest in full and keeps its operations as pieces.
base::Status make_template(ManifestBinding&& b, const ArenaKVPool& source, const ArenaKVPool& destination,
                           CopyOpTemplate* t) {
  cache::ConstComponentEndpoint src;
  cache::MutableComponentEndpoint dst;
  base::Status status = endpoints(b, source, destination, 0, &src, &dst);
  if (!status) return status;
  cache::BoundTransfer first;
  status = cache::BoundTransfer::BindComponents(*b.plan, b.src_schema, b.dst_schema, src, dst, &first);
  if (!status) return status;
  t->pieces.clear();
  t->pieces.reserve(first.operations().size());
  for (const auto& op : first.operations()) {
    const size_t si = span_holding(src.components, op.source, op.bytes);
    const size_t di = span_holding(dst.components, op.destination, op.bytes);
    if (si == src.components.size() || di == dst.components.size())
      return base::error::InternalError("bound operation outside its component span");
    t->pieces.push_back({si, di, static_cast<uint64_t>(op.source - src.components[si].data),
                         static_cast<uint64_t>(op.destination - dst.components[di].data), op.bytes});
  }
  b.by_layer.clear();
  b.pages = 0;
  t->pools = std::move(b);
  return base::error::Success();
}

// The ops of every page: its component addresses, each checked as
// endpoints() checks it, then the template's pieces at those addresses.
base::Status emit_ops(const CopyOpTemplate& t, const std::vector<const KVBlockMapping*>& by_layer,
                      size_t pages, const ArenaKVPool& source, const ArenaKVPool& destination,
                      std::vector<pbe_copy_op>* ops) {
  const ManifestBinding& b = t.pools;
  std::vector<uint64_t> src_at(b.src_schema.components.size()), dst_at(b.dst_schema.components.size());
  std::vector<pbe_copy_op> out(pages * t.pieces.size());
  pbe_copy_op* o = out.data();
  for (size_t page = 0; page < pages; ++page) {
    PageMemo src_memo, dst_memo;
    for (size_t i = 0; i < src_at.size(); ++i) {
      const auto& c = b.src_schema.components[i];
      uint8_t* a = nullptr;
      if (!component_address(source, b.src_geo, c, by_layer[c.layer]->src_block_ids[page], &src_memo, &a))
        return InvalidArgument("source block outside its page-major arena");
      src_at[i] = reinterpret_cast<uint64_t>(a);
    }
    for (size_t i = 0; i < dst_at.size(); ++i) {
      const auto& c = b.dst_schema.components[i];
      uint8_t* a = nullptr;
      if (!component_address(destination, b.dst_geo, c, by_layer[c.layer]->dst_block_ids[page], &dst_memo, &a))
        return InvalidArgument("destination block outside its page-major arena");
      dst_at[i] = reinterpret_cast<uint64_t>(a);
    }
    for (const auto& p : t.pieces) *o++ = {src_at[p.src_span] + p.src_off, dst_at[p.dst_span] + p.dst_off, p.bytes};
  }
  *ops = std::move(out);
  return base::error::Success();
}

}  // namespace

base::Status BindManifestCopyOps(const KVBlockManifest& manifest, const ArenaKVPool& source,
                                 const ArenaKVPool& destination, cache::TransferPlanner* planner,
                                 std::vector<pbe_copy_op>* ops) {
  if (!planner || !ops || !ops->empty()) return InvalidArgument("invalid semantic transfer binding arguments");
  ManifestBinding b;
  base::Status status = prepare(manifest, source, destination, planner, &b);
  if (!status) return status;
  const std::vector<const KVBlockMapping*> by_layer = b.by_layer;
  const size_t pages = b.pages;
  CopyOpTemplate t;
  status = make_template(std::move(b), source, destination, &t);
  if (!status) return status;
  return emit_ops(t, by_layer, pages, source, destination, ops);
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
  std::vector<pbe_copy_op> ops;
  // The pools are the connector's own, so their binding and the op template
  // are made once, from the first manifest that binds; each handoff then
  // only maps its layers and emits its pages' ops.
  if (template_) {
    std::vector<const KVBlockMapping*> by_layer;
    size_t pages = 0;
    status = map_layers(manifest, source_, destination_, &by_layer, &pages);
    if (status) status = emit_ops(*template_, by_layer, pages, source_, destination_, &ops);
  } else {
    ManifestBinding b;
    status = prepare(manifest, source_, destination_, &planner_, &b);
    if (status) {
      const std::vector<const KVBlockMapping*> by_layer = b.by_layer;
      const size_t pages = b.pages;
      auto t = std::make_shared<CopyOpTemplate>();
      status = make_template(std::move(b), source_, destination_, t.get());
      if (status) status = emit_ops(*t, by_layer, pages, source_, destination_, &ops);
      if (status) template_ = std::move(t);
    }
  }
  uint64_t bytes = 0;
  if (status) {
    for (const auto& op : ops) bytes += op.bytes;
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
