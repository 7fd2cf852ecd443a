// TEST INFRASTRUCTURE ONLY. A C-callable scenario driver over the
// GlobalChunkAllocator API (global_chunk_allocator.h:27-44). It is compiled
// twice: against the reference sources (oracle/_ref/libpbe_ref.so) and against
// this repository's drop-in implementation (tests), so both run the exact same
// operation sequence and their outcome logs can be compared entry by entry.
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "base/global_chunk_allocator.h"

namespace {
enum : int64_t {
  kOk = 0,
  kStaleOrDuplicate = 10,
  kIdentityMismatch = 11,
  kInvalidArgument = 12,
  kRuntimeError = 13,
  kNothingLive = 20,
};

int64_t classify_invalid(const std::invalid_argument& e) {
  const std::string what = e.what();
  if (what == "stale_or_duplicate_chunk_release") return kStaleOrDuplicate;
  if (what == "chunk_identity_mismatch") return kIdentityMismatch;
  return kInvalidArgument;
}
}  // namespace

extern "C" {

// Runs n_ops operations on a fresh allocator and writes 4 int64 per op to out:
//   [code, offset, generation, free_bytes]
// op kind 0: acquire(model[op_model], "layout" + op_layout, op_bytes, op_align)
// op kind 1: release(live[op_index]) and drop it from the live list
// op kind 2: release a copy of live[op_index] with field op_align mutated
//            (0 epoch,1 generation,2 offset,3 bytes,4 model,5 layout,6 id)
// op kind 3: release(live[op_index]) without dropping it (duplicate release)
// A release op with no live lease is recorded as code 20 and skipped.
// leased_bytes(model m) of every model is written to model_bytes_out.
// Returns 0, or -1 if the allocator could not be constructed.
int ref_alloc_run(uint64_t arena_bytes, uint64_t epoch, int32_t n_models, const uint64_t* limits,
                  int32_t n_ops, const int32_t* op_kind, const int32_t* op_model,
                  const int32_t* op_layout, const uint64_t* op_bytes, const uint64_t* op_align,
                  const int32_t* op_index, int64_t* out, int64_t* model_bytes_out) {
  try {
    base::GlobalChunkAllocator pool(arena_bytes, epoch);
    for (int32_t m = 0; m < n_models; ++m) pool.register_model("M" + std::to_string(m), limits[m]);
    std::vector<base::ChunkLease> live;
    for (int32_t i = 0; i < n_ops; ++i) {
      int64_t* o = out + 4 * i;
      o[0] = kOk;
      o[1] = o[2] = -1;
      try {
        if (op_kind[i] == 0) {
          auto lease = pool.acquire("M" + std::to_string(op_model[i]),
                                    "layout" + std::to_string(op_layout[i]), op_bytes[i], op_align[i]);
          o[1] = (int64_t)lease.offset;
          o[2] = (int64_t)lease.generation;
          live.push_back(lease);
        } else if (live.empty()) {
          o[0] = kNothingLive;
        } else {
          const size_t idx = (size_t)op_index[i] % live.size();
          base::ChunkLease lease = live[idx];
          if (op_kind[i] == 2) {
            switch (op_align[i]) {
              case 0: ++lease.epoch; break;
              case 1: ++lease.generation; break;
              case 2: ++lease.offset; break;
              case 3: ++lease.bytes; break;
              case 4: lease.model = "other"; break;
              case 5: lease.layout = "wrong"; break;
              default: ++lease.id; break;
            }
          }
          o[1] = (int64_t)lease.offset;
          pool.release(lease);
          if (op_kind[i] == 1) live.erase(live.begin() + (long)idx);
        }
      } catch (const base::ChunkAllocationError& e) {
        o[0] = static_cast<int64_t>(e.code());
      } catch (const std::invalid_argument& e) {
        o[0] = classify_invalid(e);
      } catch (const std::runtime_error&) {
        o[0] = kRuntimeError;
      }
      o[3] = (int64_t)pool.free_bytes();
    }
    for (int32_t m = 0; m < n_models; ++m)
      model_bytes_out[m] = (int64_t)pool.leased_bytes("M" + std::to_string(m));
    return 0;
  } catch (...) {
    return -1;
  }
}

}  // extern "C"

// ---------------------------------------------------------------------------
// TransferPlan scenario: builds a source and a destination schema (optionally
// head-sharded), packs each into a layout whose component order is a seeded
// permutation, compiles a plan, binds it over two byte buffers and executes it
// on the CPU. Writes a text log of every plan operation and bound copy
// (offsets relative to the buffers) followed by an FNV-1a hash of the
// destination buffer, so two builds can be compared byte for byte.
//   spec = [version, layers, page, heads, head_size, fp8, placement,
//           n_src_ranges, (begin, count)..., n_dst_ranges, (begin, count)...,
//           src_order_seed, dst_order_seed]
#include <cstdio>
#include <cstring>
#include <numeric>

#include "cache/layout_codec.h"
#include "cache/page_schema.h"
#include "cache/transfer_plan.h"

namespace {
std::vector<size_t> seeded_order(size_t n, uint32_t seed) {
  std::vector<size_t> o(n);
  std::iota(o.begin(), o.end(), 0);
  if (!seed) return o;
  uint32_t x = seed;
  for (size_t i = n; i > 1; --i) {
    x = x * 1664525u + 1013904223u;
    std::swap(o[i - 1], o[x % i]);
  }
  return o;
}

cache::PageSchema sharded(cache::PageSchema s, const std::vector<std::pair<int32_t, int32_t>>& r) {
  if (r.empty()) return s;
  std::vector<cache::ComponentDescriptor> parts;
  for (const auto& c : s.components)
    for (const auto& p : r) {
      auto d = c;
      d.head_begin = p.first;
      d.head_count = p.second;
      parts.push_back(d);
    }
  s.components = parts;
  return s;
}

void emit(std::string* log, const std::string& line) { *log += line + "\n"; }
}  // namespace

extern "C" int ref_plan_run(const int32_t* spec, int32_t n_spec, char* out, uint64_t cap) {
  std::string log;
  try {
    int32_t i = 0;
    auto next = [&]() { return i < n_spec ? spec[i++] : 0; };
    const int32_t version = next(), layers = next(), page = next(), heads = next(), hs = next();
    const bool fp8 = next() != 0;
    const auto placement = static_cast<cache::TransferPlacement>(next());
    std::vector<std::pair<int32_t, int32_t>> sr, dr;
    for (int32_t k = next(); k > 0; --k) { int32_t b = next(); sr.emplace_back(b, next()); }
    for (int32_t k = next(); k > 0; --k) { int32_t b = next(); dr.emplace_back(b, next()); }
    const uint32_t so = (uint32_t)next(), dso = (uint32_t)next();
    const auto storage = base::MakeKVCacheStorageSpec(
        base::DataType::kDataTypeBf16,
        fp8 ? base::BlockStorageMode::kFp8E4M3PerTokenHead : base::BlockStorageMode::kPlain);
    cache::PageSchema base_schema;
    auto st = cache::MakeKVPageSchema((uint32_t)version, layers, page, heads, hs, storage, &base_schema);
    if (!st) { emit(&log, "schema_error"); goto done; }
    {
      const auto src = sharded(base_schema, sr), dst = sharded(base_schema, dr);
      emit(&log, std::string("src_valid ") + (src.validate() ? "1" : "0"));
      emit(&log, std::string("dst_valid ") + (dst.validate() ? "1" : "0"));
      emit(&log, "src_fp " + src.fingerprint());
      cache::TransferPlanner planner;
      std::shared_ptr<const cache::TransferPlan> plan;
      st = planner.compile(src, dst, placement, &plan);
      if (!st) { emit(&log, "compile_error"); goto done; }
      for (const auto& op : plan->operations)
        emit(&log, "op " + op.component.semantic_key() + " <- " + op.source_component.semantic_key() +
                       " -> " + op.destination_component.semantic_key());
      cache::LayoutDescriptor sl, dl;
      if (!cache::MakePackedLayout(src, "src", 5, seeded_order(src.components.size(), so), {}, &sl) ||
          !cache::MakePackedLayout(dst, "dst", 6, seeded_order(dst.components.size(), dso), {}, &dl)) {
        emit(&log, "layout_error");
        goto done;
      }
      std::vector<uint8_t> sb(sl.total_bytes), db(dl.total_bytes, 0xa5);
      for (size_t k = 0; k < sb.size(); ++k) sb[k] = (uint8_t)(k * 131u + 7u);
      cache::BoundTransfer bound;
      st = cache::BoundTransfer::Bind(*plan, src, dst, {sb.data(), sb.size(), &sl},
                                      {db.data(), db.size(), &dl}, &bound);
      if (!st) { emit(&log, "bind_error"); goto done; }
      for (const auto& op : bound.operations()) {
        char line[256];
        std::snprintf(line, sizeof(line), "copy %s src+%zu dst+%zu bytes=%zu vid=%lld/%lld",
                      op.component.semantic_key().c_str(), (size_t)(op.source - sb.data()),
                      (size_t)(op.destination - db.data()), op.bytes,
                      (long long)op.source_virtual_block_id, (long long)op.destination_virtual_block_id);
        emit(&log, line);
      }
      emit(&log, "staging " + std::to_string(bound.staging_bytes()));
      if (placement == cache::TransferPlacement::kExactDirect) st = cache::ExecuteCpuTransfer(bound);
      else {
        std::vector<uint8_t> staging(bound.staging_bytes());
        st = cache::ExecuteCpuTransferStaged(bound, staging.data(), staging.size());
      }
      if (!st) { emit(&log, "execute_error"); goto done; }
      uint64_t h = 1469598103934665603ull;
      for (uint8_t b : db) { h ^= b; h *= 1099511628211ull; }
      emit(&log, "dst_hash " + std::to_string(h));
    }
  } catch (const std::exception& e) {
    emit(&log, std::string("exception ") + e.what());
  }
done:
  if (log.size() + 1 > cap) return -1;
  std::memcpy(out, log.c_str(), log.size() + 1);
  return (int)log.size();
}

// ---------------------------------------------------------------------------
// CPU handoff through the generic plan path, as the in-process block-copy
// connector runs it between two host pools (pd_handoff.cpp:192-213 with
// pd_handoff_common.cpp:64-140 binding the manifest): one KV page schema, one
// kExactDirect plan, then per page a BoundTransfer over that page's planes and
// ExecuteCpuTransfer (transfer_plan.cpp:392-403), i.e. one memcpy per (layer,
// K|V) component. Planes live in a page-major arena: plane 2l+kind of page id p
// starts at byte (p + 2l + kind) * half. Every binding and copy is repeated
// `repeats` times. Returns the bytes copied by one pass, or -1 on any error.
extern "C" int64_t ref_cpu_handoff(uint8_t* arena, uint64_t arena_bytes, const int32_t* src_ids,
                                   const int32_t* dst_ids, int64_t n, int32_t layers,
                                   int32_t kv_heads, int32_t head_size, int32_t page_tokens,
                                   int32_t repeats) {
  try {
    const auto storage =
        base::MakeKVCacheStorageSpec(base::DataType::kDataTypeBf16, base::BlockStorageMode::kPlain);
    cache::PageSchema schema;
    if (!cache::MakeKVPageSchema(1, layers, page_tokens, kv_heads, head_size, storage, &schema))
      return -1;
    cache::TransferPlanner planner;
    std::shared_ptr<const cache::TransferPlan> plan;
    if (!planner.compile(schema, schema, cache::TransferPlacement::kExactDirect, &plan)) return -1;
    std::vector<size_t> order(schema.components.size());
    std::iota(order.begin(), order.end(), 0);
    cache::LayoutDescriptor src_layout, dst_layout;
    if (!cache::MakePackedLayout(schema, "cpu-src", 1, order, {}, &src_layout) ||
        !cache::MakePackedLayout(schema, "cpu-dst", 1, order, {}, &dst_layout))
      return -1;
    const uint64_t half = (uint64_t)page_tokens * kv_heads * head_size * 2u;
    for (int64_t i = 0; i < n; ++i)
      if (src_ids[i] < 0 || dst_ids[i] < 0 ||
          ((uint64_t)src_ids[i] + 2ull * layers) * half > arena_bytes ||
          ((uint64_t)dst_ids[i] + 2ull * layers) * half > arena_bytes)
        return -1;
    int64_t copied = 0;
    for (int32_t rep = 0; rep < repeats; ++rep) {
      copied = 0;
      std::vector<cache::BoundTransfer> transfers(static_cast<size_t>(n));
      for (int64_t i = 0; i < n; ++i) {
        cache::ConstComponentEndpoint src;
        cache::MutableComponentEndpoint dst;
        src.layout = &src_layout;
        dst.layout = &dst_layout;
        for (const auto& c : schema.components) {
          const uint64_t plane = 2ull * c.layer + (c.kind == cache::ComponentKind::kValue ? 1 : 0);
          src.components.push_back({c, arena + (src_ids[i] + plane) * half, c.byte_size()});
          dst.components.push_back({c, arena + (dst_ids[i] + plane) * half, c.byte_size()});
        }
        if (!cache::BoundTransfer::BindComponents(*plan, schema, src, dst, &transfers[(size_t)i]))
          return -1;
      }
      for (const auto& t : transfers) {
        if (!cache::ExecuteCpuTransfer(t)) return -1;
        for (const auto& op : t.operations()) copied += (int64_t)op.bytes;
      }
    }
    return copied;
  } catch (const std::exception&) {
    return -1;
  }
}
