// CPU tests of the C++ drop-in API. The scenarios restate the reference's own
// tests as behaviour: test/test_global_chunk_allocator.cpp:8-97,
// test/test_cache_transfer_plan.cpp:130-467, test/test_page_migration.cpp:5-25,
// test/test_serving/test_pd_handoff.cpp:284-296.
#include <algorithm>
#include <array>
#include <map>
#include <cstring>
#include <memory>
#include <numeric>
#include <random>
#include <stdexcept>
#include <vector>

#include "base/global_chunk_allocator.h"
#include "base/kv_cache_format.h"
#include "cache/layout_codec.h"
#include "cache/page_migration.h"
#include "cache/page_schema.h"
#include "cache/transfer_plan.h"
#include "minitest.h"
#include "base/shared_kv_arena.h"
#include "serving/decode_kv_reservation.h"
#include "serving/pd_handoff.h"
#include "serving/kv_page_wire.h"
#include "serving/split_pd_handoff.h"
#include "serving/split_pd_admission.h"
#include "base/block_allocator.h"
#include "base/kv_cache_manager.h"
#include "base/page_index.h"
#include "kernels/xcd_order.h"

using namespace cache;

// ------------------------------------------------------------ chunk allocator

TEST_CASE("chunk allocator: freed bytes are reused across layouts") {
  base::GlobalChunkAllocator pool(12 << 10, 7);
  pool.register_model("A", 8 << 10);
  pool.register_model("B", 8 << 10);
  const auto a = pool.acquire("A", "24x64", 6 << 10, 512);
  const auto b = pool.acquire("B", "28x128", 4 << 10, 1024);
  CHECK_EQ(pool.free_bytes(), 2u << 10);
  CHECK_THROWS_AS(pool.acquire("B", "28x128", 4 << 10, 1024), std::runtime_error);
  pool.release(a);
  const auto again = pool.acquire("B", "28x128", 4 << 10, 1024);
  CHECK_EQ(again.offset, a.offset);           // best fit reuses the released range
  CHECK(again.generation != a.generation);
  CHECK_EQ(pool.leased_bytes("A"), 0u);
  CHECK_EQ(pool.leased_bytes("B"), 8u << 10);
  CHECK_THROWS_AS(pool.release(a), std::invalid_argument);
  pool.release(b);
  pool.release(again);
  CHECK_EQ(pool.free_bytes(), pool.bytes());
  CHECK_EQ(pool.lease_count(), 0u);
}

TEST_CASE("chunk allocator: every lease field is part of its identity") {
  base::GlobalChunkAllocator pool(16384, 42);
  pool.register_model("A", 8192);
  const auto live = pool.acquire("A", "layout", 4096, 256);
  for (int field = 0; field < 7; ++field) {
    auto forged = live;
    switch (field) {
      case 0: ++forged.epoch; break;
      case 1: ++forged.generation; break;
      case 2: ++forged.offset; break;
      case 3: ++forged.bytes; break;
      case 4: forged.model = "B"; break;
      case 5: forged.layout = "wrong"; break;
      default: ++forged.id; break;
    }
    CHECK_THROWS_AS(pool.release(forged), std::invalid_argument);
    CHECK_EQ(pool.leased_bytes("A"), 4096u);
  }
  pool.release(live);
  CHECK_THROWS_AS(pool.release(live), std::invalid_argument);
  CHECK_EQ(pool.free_bytes(), 16384u);
}

TEST_CASE("chunk allocator: alignment, fragmentation and quota fail atomically") {
  base::GlobalChunkAllocator pool(8192, 1);
  pool.register_model("A", 8192);
  pool.register_model("B", 2048);
  auto a = pool.acquire("A", "page3", 3072, 1536);
  auto b = pool.acquire("B", "page2", 2048, 2048);
  CHECK_EQ(a.offset % 1536, 0u);
  CHECK_EQ(b.offset % 2048, 0u);
  const auto free_before = pool.free_bytes();
  try {
    pool.acquire("B", "page2", 2048, 2048);
    CHECK(false);
  } catch (const base::ChunkAllocationError& e) {
    CHECK(e.code() == base::ChunkAllocationFailure::kQuota);
  }
  CHECK_EQ(pool.free_bytes(), free_before);
  try {
    pool.acquire("A", "page4", 4096, 4096);
    CHECK(false);
  } catch (const base::ChunkAllocationError& e) {
    // a at [0, 3072), b at [4096, 6144): only 3072 bytes are free.
    CHECK(e.code() == base::ChunkAllocationFailure::kExhausted);
  }
  CHECK_EQ(pool.free_bytes(), free_before);
  try {
    pool.acquire("A", "page2", 2048, 2048);  // 2048 free at 6144: fits
  } catch (...) {
    CHECK(false);
  }
  try {
    pool.acquire("A", "page1k", 1024, 1024);  // 1024 free at 3072: fits
  } catch (...) {
    CHECK(false);
  }
  CHECK_EQ(pool.free_bytes(), 0u);
  CHECK_THROWS_AS(pool.acquire("A", "bad", 100, 256), std::invalid_argument);
}

TEST_CASE("chunk allocator: fragmented when enough bytes are free but split") {
  base::GlobalChunkAllocator pool(8192, 1);
  pool.register_model("A", 8192);
  auto a = pool.acquire("A", "p", 2048, 2048);
  auto b = pool.acquire("A", "p", 2048, 2048);
  auto c = pool.acquire("A", "p", 2048, 2048);
  auto d = pool.acquire("A", "p", 2048, 2048);
  pool.release(a);
  pool.release(c);
  try {
    pool.acquire("A", "p", 4096, 2048);
    CHECK(false);
  } catch (const base::ChunkAllocationError& e) {
    CHECK(e.code() == base::ChunkAllocationFailure::kFragmented);
  }
  pool.release(b);  // coalesces [0, 6144)
  const auto big = pool.acquire("A", "p", 6144, 2048);
  CHECK_EQ(big.offset, 0u);
  pool.release(big);
  pool.release(d);
  const auto whole = pool.acquire("A", "whole", 8192, 256);
  CHECK_EQ(whole.offset, 0u);
}

TEST_CASE("chunk allocator: exhausted vs fragmented and invalid registration") {
  base::GlobalChunkAllocator pool(4096, 3);
  CHECK_THROWS_AS(base::GlobalChunkAllocator(0, 1), std::invalid_argument);
  CHECK_THROWS_AS(base::GlobalChunkAllocator(10, 0), std::invalid_argument);
  CHECK_THROWS_AS(pool.register_model("", 10), std::invalid_argument);
  CHECK_THROWS_AS(pool.register_model("A", 0), std::invalid_argument);
  CHECK_THROWS_AS(pool.register_model("A", 8192), std::invalid_argument);
  pool.register_model("A", 4096);
  CHECK_THROWS_AS(pool.register_model("A", 4096), std::invalid_argument);
  CHECK_THROWS_AS(pool.acquire("nobody", "x", 256, 256), std::invalid_argument);
  CHECK_THROWS_AS(pool.acquire("A", "", 256, 256), std::invalid_argument);
  CHECK_THROWS_AS(pool.acquire("A", "x", 0, 256), std::invalid_argument);
  CHECK_THROWS_AS(pool.acquire("A", "x", 256, 0), std::invalid_argument);
  auto a = pool.acquire("A", "x", 3072, 1024);
  try {
    pool.acquire("A", "x", 2048, 1024);
    CHECK(false);
  } catch (const base::ChunkAllocationError& e) {
    CHECK(e.code() == base::ChunkAllocationFailure::kQuota);
  }
  pool.release(a);
}

TEST_CASE("chunk allocator: randomized leases stay disjoint and accounted") {
  base::GlobalChunkAllocator pool(12u << 20, 77);
  pool.register_model("A", pool.bytes());
  pool.register_model("B", pool.bytes());
  std::mt19937 rng(42);
  std::vector<base::ChunkLease> leases;
  for (int step = 0; step < 4000; ++step) {
    if (!leases.empty() && rng() % 3 == 0) {
      const size_t idx = rng() % leases.size();
      pool.release(leases[idx]);
      leases.erase(leases.begin() + static_cast<long>(idx));
    } else {
      const uint64_t page = (rng() % 2 ? 24 : 28) * 8192ull;
      const bool model_a = rng() % 2;
      const uint64_t bytes = page * (1 + rng() % 4);
      try {
        leases.push_back(pool.acquire(model_a ? "A" : "B", "gqa", bytes, page));
      } catch (const std::runtime_error&) {
      }
    }
    std::sort(leases.begin(), leases.end(),
              [](const base::ChunkLease& x, const base::ChunkLease& y) { return x.offset < y.offset; });
    uint64_t total = 0, a_bytes = 0, b_bytes = 0;
    for (size_t i = 0; i < leases.size(); ++i) {
      CHECK(leases[i].offset + leases[i].bytes <= pool.bytes());
      if (i) CHECK(leases[i - 1].offset + leases[i - 1].bytes <= leases[i].offset);
      total += leases[i].bytes;
      (leases[i].model == "A" ? a_bytes : b_bytes) += leases[i].bytes;
    }
    CHECK_EQ(total + pool.free_bytes(), pool.bytes());
    CHECK_EQ(a_bytes, pool.leased_bytes("A"));
    CHECK_EQ(b_bytes, pool.leased_bytes("B"));
  }
  for (const auto& l : leases) pool.release(l);
  CHECK_EQ(pool.free_bytes(), pool.bytes());
}

// ------------------------------------------------------------ schema / plans

namespace {

PageSchema plain_schema() {
  PageSchema s;
  CHECK(MakeKVPageSchema(1, 3, 4, 2, 8,
                         base::MakeKVCacheStorageSpec(base::DataType::kDataTypeBf16,
                                                      base::BlockStorageMode::kPlain),
                         &s));
  return s;
}

PageSchema fp8_schema() {
  PageSchema s;
  CHECK(MakeKVPageSchema(1, 2, 4, 2, 8,
                         base::MakeKVCacheStorageSpec(base::DataType::kDataTypeBf16,
                                                      base::BlockStorageMode::kFp8E4M3PerTokenHead),
                         &s));
  return s;
}

PageSchema headed_schema(bool fp8, int32_t heads = 4, uint32_t version = 1) {
  PageSchema s;
  CHECK(MakeKVPageSchema(version, 2, 4, heads, 3,
                         base::MakeKVCacheStorageSpec(base::DataType::kDataTypeBf16,
                                                      fp8 ? base::BlockStorageMode::kFp8E4M3PerTokenHead
                                                          : base::BlockStorageMode::kPlain),
                         &s));
  return s;
}

// Splits every component into the given head ranges (tensor-parallel shards).
PageSchema shard(PageSchema s, const std::vector<std::pair<int32_t, int32_t>>& ranges) {
  std::vector<ComponentDescriptor> parts;
  for (const auto& c : s.components)
    for (const auto& r : ranges) {
      auto p = c;
      p.head_begin = r.first;
      p.head_count = r.second;
      parts.push_back(p);
    }
  s.components = parts;
  CHECK(s.validate());
  return s;
}

std::vector<size_t> iota_order(size_t n) {
  std::vector<size_t> o(n);
  std::iota(o.begin(), o.end(), 0);
  return o;
}

const ComponentLayout& entry_of(const LayoutDescriptor& l, const ComponentDescriptor& c) {
  for (const auto& e : l.components)
    if (e.component.semantic_key() == c.semantic_key()) return e;
  static ComponentLayout none;
  CHECK(false);
  return none;
}

// One byte value per (layer, kind) component.
void fill_by_component(const LayoutDescriptor& l, std::vector<uint8_t>* bytes) {
  for (const auto& e : l.components) {
    const uint8_t v = static_cast<uint8_t>(1 + e.component.layer * 17 + static_cast<int>(e.component.kind) * 3);
    std::fill(bytes->begin() + e.offset_bytes, bytes->begin() + e.offset_bytes + e.size_bytes, v);
  }
}

// A byte value that depends on (layer, kind, token, absolute head, element, byte),
// so any slice landing in the wrong place shows up.
void fill_by_element(const LayoutDescriptor& l, std::vector<uint8_t>* bytes) {
  for (const auto& e : l.components) {
    const auto& c = e.component;
    const size_t width = base::DataTypeSize(c.dtype);
    size_t at = e.offset_bytes;
    for (int32_t t = 0; t < c.token_count; ++t)
      for (int32_t h = 0; h < c.head_count; ++h)
        for (int32_t x = 0; x < c.elements_per_head; ++x)
          for (size_t b = 0; b < width; ++b)
            (*bytes)[at++] = static_cast<uint8_t>(1 + c.layer * 71 + static_cast<int>(c.kind) * 31 +
                                                  t * 13 + (c.head_begin + h) * 7 + x * 3 +
                                                  static_cast<int>(b));
  }
}

}  // namespace

TEST_CASE("page schema: K, V and scale coverage is required") {
  auto plain = plain_schema();
  CHECK(plain.validate());
  plain.components.pop_back();
  CHECK(!plain.validate());
  auto fp8 = fp8_schema();
  CHECK(fp8.validate());
  fp8.components.erase(std::find_if(fp8.components.begin(), fp8.components.end(), [](const auto& c) {
    return c.kind == ComponentKind::kValueScale;
  }));
  CHECK(!fp8.validate());
  auto bad = plain_schema();
  bad.storage.scale_dtype = base::DataType::kDataTypeFp32;
  CHECK(!bad.validate());
  auto overlap = headed_schema(false);
  overlap.components.push_back(overlap.components.front());
  overlap.components.back().head_count = 1;
  CHECK(!overlap.validate());
}

TEST_CASE("transfer plan: shuffled layouts and virtual block ids round trip") {
  const auto schema = fp8_schema();
  const auto src_order = iota_order(schema.components.size());
  auto host_order = src_order;
  std::reverse(host_order.begin(), host_order.end());
  const std::vector<size_t> back_order = {2, 5, 0, 7, 1, 6, 3, 4};
  LayoutDescriptor src_l, host_l, back_l;
  REQUIRE(MakePackedLayout(schema, "gpu-layer-first", 11, src_order,
                           {101, 203, 307, 409, 503, 601, 709, 809}, &src_l));
  REQUIRE(MakePackedLayout(schema, "host-page-first", 12, host_order,
                           {9001, 9002, 9003, 9004, 9005, 9006, 9007, 9008}, &host_l));
  REQUIRE(MakePackedLayout(schema, "gpu-restored", 13, back_order, {41, 37, 31, 29, 23, 19, 17, 13},
                           &back_l));
  std::vector<uint8_t> src(src_l.total_bytes), host(host_l.total_bytes, 0), back(back_l.total_bytes, 0);
  fill_by_component(src_l, &src);
  TransferPlanner planner;
  TransferPlan plan;
  REQUIRE(planner.plan(schema, schema, &plan));
  BoundTransfer pack;
  REQUIRE(BoundTransfer::Bind(plan, schema, {src.data(), src.size(), &src_l},
                              {host.data(), host.size(), &host_l}, &pack));
  REQUIRE(ExecuteCpuTransfer(pack));
  CHECK_EQ(pack.source_epoch(), 11u);
  CHECK_EQ(pack.destination_epoch(), 12u);
  for (const auto& op : pack.operations()) {
    CHECK_EQ(op.source_virtual_block_id, entry_of(src_l, op.component).virtual_block_id);
    CHECK_EQ(op.destination_virtual_block_id, entry_of(host_l, op.component).virtual_block_id);
  }
  BoundTransfer unpack;
  REQUIRE(BoundTransfer::Bind(plan, schema, {host.data(), host.size(), &host_l},
                              {back.data(), back.size(), &back_l}, &unpack));
  REQUIRE(ExecuteCpuTransfer(unpack));
  for (const auto& e : src_l.components) {
    const auto& o = entry_of(back_l, e.component);
    CHECK(std::equal(src.begin() + e.offset_bytes, src.begin() + e.offset_bytes + e.size_bytes,
                     back.begin() + o.offset_bytes));
  }
  TransferPlan again;
  REQUIRE(planner.plan(schema, schema, &again));
  CHECK_EQ(planner.cache_hits(), 1u);
  CHECK_EQ(planner.cache_entries(), 1u);
}

TEST_CASE("transfer plan: a missing or corrupt component fails before any write") {
  const auto schema = fp8_schema();
  const auto order = iota_order(schema.components.size());
  LayoutDescriptor src_l, dst_l;
  REQUIRE(MakePackedLayout(schema, "source", 1, order, {}, &src_l));
  REQUIRE(MakePackedLayout(schema, "destination", 2, order, {}, &dst_l));
  src_l.components.pop_back();
  std::vector<uint8_t> src(src_l.total_bytes, 0x27), dst(dst_l.total_bytes, 0xa5);
  const auto original = dst;
  TransferPlanner planner;
  TransferPlan plan;
  REQUIRE(planner.plan(schema, schema, &plan));
  BoundTransfer bound;
  CHECK(!BoundTransfer::Bind(plan, schema, {src.data(), src.size(), &src_l},
                             {dst.data(), dst.size(), &dst_l}, &bound));
  CHECK(dst == original);
  src_l.components.push_back(dst_l.components.back());
  plan.operations.back() = plan.operations.front();
  CHECK(!BoundTransfer::Bind(plan, schema, {src.data(), src.size(), &src_l},
                             {dst.data(), dst.size(), &dst_l}, &bound));
  CHECK(dst == original);
}

TEST_CASE("transfer plan: a schema or layout changed in place is checked again") {
  // Binding keeps the facts of recently seen schemas and layouts; a change to
  // the same object must give what a first binding of the new contents gives.
  auto schema = fp8_schema();
  const auto order = iota_order(schema.components.size());
  LayoutDescriptor src_l, dst_l;
  REQUIRE(MakePackedLayout(schema, "source", 1, order, {}, &src_l));
  REQUIRE(MakePackedLayout(schema, "destination", 2, order, {}, &dst_l));
  std::vector<uint8_t> src(src_l.total_bytes, 0x27), dst(dst_l.total_bytes, 0xa5);
  TransferPlanner planner;
  TransferPlan plan;
  REQUIRE(planner.plan(schema, schema, &plan));
  auto bind = [&](const PageSchema& s) {
    BoundTransfer b;
    return static_cast<bool>(BoundTransfer::Bind(plan, s, {src.data(), src.size(), &src_l},
                                                 {dst.data(), dst.size(), &dst_l}, &b));
  };
  CHECK(bind(schema));
  schema.components[0].head_count += 1;  // beyond the schema's heads: invalid
  CHECK(!schema.validate());
  CHECK(!bind(schema));
  schema.components[0].head_count -= 1;
  CHECK(bind(schema));
  const size_t offset = dst_l.components[1].offset_bytes;
  dst_l.components[1].offset_bytes = dst_l.components[0].offset_bytes;  // overlapping entries
  CHECK(!dst_l.validate(schema));
  CHECK(!bind(schema));
  dst_l.components[1].offset_bytes = offset;
  CHECK(bind(schema));
  auto other = schema;
  other.version = 2;  // same components, another plan: the fingerprints differ
  CHECK(!bind(other));
  // more distinct schemas than are remembered, each bound twice in turn
  for (int round = 0; round < 2; ++round)
    for (int layers = 1; layers <= 7; ++layers) {
      PageSchema s;
      REQUIRE(MakeKVPageSchema(1, layers, 16, 2, 64,
                               base::MakeKVCacheStorageSpec(base::DataType::kDataTypeBf16,
                                                            base::BlockStorageMode::kPlain),
                               &s));
      LayoutDescriptor a, b;
      REQUIRE(MakePackedLayout(s, "a", 1, iota_order(s.components.size()), {}, &a));
      REQUIRE(MakePackedLayout(s, "b", 2, iota_order(s.components.size()), {}, &b));
      std::vector<uint8_t> x(a.total_bytes, 1), y(b.total_bytes, 2);
      TransferPlan p;
      REQUIRE(planner.plan(s, s, &p));
      BoundTransfer t;
      REQUIRE(BoundTransfer::Bind(p, s, {x.data(), x.size(), &a}, {y.data(), y.size(), &b}, &t));
      CHECK_EQ(t.operations().size(), static_cast<size_t>(2 * layers));
      REQUIRE(ExecuteCpuTransfer(t));
      CHECK(x == y);
    }
}

TEST_CASE("transfer plan: shape and dtype mismatches fail before any write") {
  const auto schema = plain_schema();
  const auto order = iota_order(schema.components.size());
  LayoutDescriptor src_l, dst_l;
  REQUIRE(MakePackedLayout(schema, "source", 1, order, {}, &src_l));
  REQUIRE(MakePackedLayout(schema, "destination", 2, order, {}, &dst_l));
  std::vector<uint8_t> src(src_l.total_bytes, 0x33), dst(dst_l.total_bytes, 0x5a);
  const auto original = dst;
  dst_l.components.front().component.dtype = base::DataType::kDataTypeFp32;
  TransferPlanner planner;
  TransferPlan plan;
  REQUIRE(planner.plan(schema, schema, &plan));
  BoundTransfer bound;
  CHECK(!BoundTransfer::Bind(plan, schema, {src.data(), src.size(), &src_l},
                             {dst.data(), dst.size(), &dst_l}, &bound));
  CHECK(dst == original);
  auto wider = schema;
  wider.head_size += 1;
  for (auto& c : wider.components) c.elements_per_head += 1;
  CHECK(!planner.plan(schema, wider, &plan));
}

TEST_CASE("transfer plan: independent allocations pack and restore (plain and FP8)") {
  for (const auto& schema : {plain_schema(), fp8_schema()}) {
    auto order = iota_order(schema.components.size());
    LayoutDescriptor gpu_l, host_l, back_l;
    REQUIRE(MakePackedLayout(schema, "scatter-gpu", 31, order, {}, &gpu_l));
    std::reverse(order.begin(), order.end());
    REQUIRE(MakePackedLayout(schema, "packed-host", 32, order, {}, &host_l));
    REQUIRE(MakePackedLayout(schema, "restored-gpu", 33, order, {}, &back_l));
    std::vector<std::vector<uint8_t>> originals, restored;
    for (size_t i = 0; i < schema.components.size(); ++i) {
      originals.emplace_back(schema.components[i].byte_size(), static_cast<uint8_t>(i + 71));
      restored.emplace_back(schema.components[i].byte_size(), 0);
    }
    std::vector<uint8_t> host(host_l.total_bytes, 0);
    ConstComponentEndpoint source{{}, &gpu_l}, packed_source{{}, &host_l};
    MutableComponentEndpoint packed{{}, &host_l}, target{{}, &back_l};
    for (size_t i = 0; i < schema.components.size(); ++i) {
      const auto& c = schema.components[i];
      source.components.push_back({c, originals[i].data(), originals[i].size()});
      target.components.push_back({c, restored[i].data(), restored[i].size()});
      const auto& e = entry_of(host_l, c);
      packed.components.push_back({c, host.data() + e.offset_bytes, e.size_bytes});
      packed_source.components.push_back({c, host.data() + e.offset_bytes, e.size_bytes});
    }
    std::reverse(source.components.begin(), source.components.end());
    TransferPlanner planner;
    TransferPlan plan;
    REQUIRE(planner.plan(schema, schema, &plan));
    BoundTransfer pack, unpack;
    REQUIRE(BoundTransfer::BindComponents(plan, schema, source, packed, &pack));
    REQUIRE(ExecuteCpuTransfer(pack));
    REQUIRE(BoundTransfer::BindComponents(plan, schema, packed_source, target, &unpack));
    REQUIRE(ExecuteCpuTransfer(unpack));
    CHECK(originals == restored);
    CHECK_EQ(pack.source_epoch(), 31u);
    CHECK_EQ(unpack.destination_epoch(), 33u);

    // Failed bindings leave the destination bytes and the earlier binding intact.
    const auto host_before = host;
    const auto ops_before = pack.operations().size();
    const auto kept = source;
    source.components.pop_back();
    CHECK(!BoundTransfer::BindComponents(plan, schema, source, packed, &pack));
    source = kept;
    source.components.back() = source.components.front();
    CHECK(!BoundTransfer::BindComponents(plan, schema, source, packed, &pack));
    source = kept;
    source.components.back().bytes = 1;
    CHECK(!BoundTransfer::BindComponents(plan, schema, source, packed, &pack));
    source = kept;
    source.components.back().component.dtype = base::DataType::kDataTypeFp32;
    CHECK(!BoundTransfer::BindComponents(plan, schema, source, packed, &pack));
    source = kept;
    auto aliased = packed;
    aliased.components.back().data = aliased.components.front().data;
    CHECK(!BoundTransfer::BindComponents(plan, schema, source, aliased, &pack));
    plan.operations.back() = plan.operations.front();
    CHECK(!BoundTransfer::BindComponents(plan, schema, source, packed, &pack));
    CHECK(host == host_before);
    CHECK_EQ(pack.operations().size(), ops_before);
    CHECK_EQ(pack.source_epoch(), 31u);
  }
}

TEST_CASE("transfer plan: head split/merge keeps every element in place") {
  for (bool fp8 : {false, true}) {
    const auto src_schema = shard(headed_schema(fp8), {{0, 1}, {1, 3}});
    const auto dst_schema = shard(headed_schema(fp8), {{0, 2}, {2, 2}});
    auto src_order = iota_order(src_schema.components.size());
    auto dst_order = iota_order(dst_schema.components.size());
    std::reverse(src_order.begin(), src_order.end());
    std::rotate(dst_order.begin(), dst_order.begin() + 3, dst_order.end());
    LayoutDescriptor src_l, dst_l;
    REQUIRE(MakePackedLayout(src_schema, "tp-source", 41, src_order, {}, &src_l));
    REQUIRE(MakePackedLayout(dst_schema, "tp-destination", 42, dst_order, {}, &dst_l));
    std::vector<uint8_t> src(src_l.total_bytes), expected(dst_l.total_bytes);
    fill_by_element(src_l, &src);
    fill_by_element(dst_l, &expected);
    for (auto placement : {TransferPlacement::kExactDirect, TransferPlacement::kSenderPack,
                           TransferPlacement::kReceiverUnpack}) {
      TransferPlanner planner;
      std::shared_ptr<const TransferPlan> plan;
      REQUIRE(planner.compile(src_schema, dst_schema, placement, &plan));
      std::vector<uint8_t> dst(dst_l.total_bytes, 0xa5);
      BoundTransfer bound;
      REQUIRE(BoundTransfer::Bind(*plan, src_schema, dst_schema, {src.data(), src.size(), &src_l},
                                  {dst.data(), dst.size(), &dst_l}, &bound));
      if (placement == TransferPlacement::kExactDirect) {
        REQUIRE(ExecuteCpuTransfer(bound));
      } else {
        std::vector<uint8_t> staging(bound.staging_bytes());
        REQUIRE(ExecuteCpuTransferStaged(bound, staging.data(), staging.size()));
        CHECK(!ExecuteCpuTransferStaged(bound, staging.data(), staging.size() - 1));
      }
      CHECK(dst == expected);
      CHECK_EQ(bound.source_epoch(), 41u);
      CHECK_EQ(bound.destination_epoch(), 42u);
      CHECK(bound.placement() == placement);
    }
  }
}

TEST_CASE("transfer plan: invalid coverage or conversions fail before any write") {
  auto src_schema = shard(headed_schema(false), {{0, 2}, {2, 2}});
  auto dst_schema = shard(headed_schema(false), {{0, 1}, {1, 3}});
  TransferPlanner planner;
  std::shared_ptr<const TransferPlan> plan;
  REQUIRE(planner.compile(src_schema, dst_schema, TransferPlacement::kExactDirect, &plan));
  LayoutDescriptor src_l, dst_l;
  REQUIRE(MakePackedLayout(src_schema, "source", 1, iota_order(src_schema.components.size()), {}, &src_l));
  REQUIRE(MakePackedLayout(dst_schema, "destination", 2, iota_order(dst_schema.components.size()), {},
                           &dst_l));
  std::vector<uint8_t> src(src_l.total_bytes, 0x37), dst(dst_l.total_bytes, 0xa5);
  const auto original = dst;
  auto stale = src_schema;
  stale.version++;
  BoundTransfer bound;
  CHECK(!BoundTransfer::Bind(*plan, stale, dst_schema, {src.data(), src.size(), &src_l},
                             {dst.data(), dst.size(), &dst_l}, &bound));
  CHECK(dst == original);
  auto missing = src_schema;
  missing.components.pop_back();
  CHECK(!planner.compile(missing, dst_schema, TransferPlacement::kExactDirect, &plan));
  auto duplicate = dst_schema;
  duplicate.components.push_back(duplicate.components.back());
  CHECK(!planner.compile(src_schema, duplicate, TransferPlacement::kExactDirect, &plan));
  auto converted = dst_schema;
  converted.storage = base::MakeKVCacheStorageSpec(base::DataType::kDataTypeBf16,
                                                   base::BlockStorageMode::kFp8E4M3PerTokenHead);
  CHECK(!planner.compile(src_schema, converted, TransferPlacement::kExactDirect, &plan));
  CHECK(dst == original);
}

TEST_CASE("transfer plan: template cache ignores addresses and stays bounded") {
  const auto src = shard(headed_schema(false), {{0, 2}, {2, 2}});
  const auto dst = shard(headed_schema(false), {{0, 1}, {1, 3}});
  TransferPlanner planner(2, 1u << 20);
  std::shared_ptr<const TransferPlan> first;
  REQUIRE(planner.compile(src, dst, TransferPlacement::kSenderPack, &first));
  for (int i = 0; i < 1000; ++i) {
    std::shared_ptr<const TransferPlan> again;
    REQUIRE(planner.compile(src, dst, TransferPlacement::kSenderPack, &again));
    CHECK(again.get() == first.get());
  }
  CHECK_EQ(planner.cache_entries(), 1u);
  CHECK_EQ(planner.cache_hits(), 1000u);
  CHECK(planner.cache_bytes() > 0u);
  std::shared_ptr<const TransferPlan> m2, m3;
  REQUIRE(planner.compile(src, dst, TransferPlacement::kReceiverUnpack, &m2));
  REQUIRE(planner.compile(src, dst, TransferPlacement::kExactDirect, &m3));
  CHECK_EQ(planner.cache_entries(), 2u);
  CHECK(planner.cache_evictions() >= 1u);
  CHECK(planner.cache_bytes() <= (1u << 20));
  CHECK(first.get() != m2.get());
  CHECK_THROWS_AS(TransferPlanner(0, 1), std::invalid_argument);
}

TEST_CASE("transfer plan: the cache evicts the least recently used plan") {
  const auto src = shard(headed_schema(false), {{0, 2}, {2, 2}});
  const auto dst = shard(headed_schema(false), {{0, 1}, {1, 3}});
  auto get = [&](TransferPlanner& p, TransferPlacement where) -> const TransferPlan* {
    std::shared_ptr<const TransferPlan> out;
    CHECK(p.compile(src, dst, where, &out));
    return out.get();  // the cache, or nothing, keeps it alive
  };
  const auto A = TransferPlacement::kSenderPack, B = TransferPlacement::kReceiverUnpack,
             C = TransferPlacement::kExactDirect;
  TransferPlanner lru(2, 1u << 20);
  const TransferPlan* a = get(lru, A);
  const TransferPlan* b = get(lru, B);
  CHECK(get(lru, A) == a);  // A is now the most recent
  get(lru, C);              // evicts B, not A
  CHECK_EQ(lru.cache_evictions(), 1u);
  CHECK(get(lru, A) == a);
  const size_t hits = lru.cache_hits();
  CHECK(get(lru, B) != nullptr);  // B was gone: compiled again, evicting C
  CHECK_EQ(lru.cache_hits(), hits);
  CHECK_EQ(lru.cache_evictions(), 2u);
  (void)b;

  // Byte budget of one plan: every new plan replaces the previous one; a
  // budget below one plan caches nothing and still returns plans.
  std::shared_ptr<const TransferPlan> probe;
  REQUIRE(lru.compile(src, dst, A, &probe));
  const size_t one = probe->template_bytes;
  TransferPlanner tight(16, one + one / 2);
  get(tight, A);
  get(tight, B);
  CHECK_EQ(tight.cache_entries(), 1u);
  CHECK_EQ(tight.cache_bytes(), one);
  get(tight, A);  // A was replaced by B: a miss
  CHECK_EQ(tight.cache_hits(), 0u);
  CHECK_EQ(tight.cache_evictions(), 2u);
  TransferPlanner none(16, one - 1);
  std::shared_ptr<const TransferPlan> p1, p2;
  REQUIRE(none.compile(src, dst, A, &p1));
  REQUIRE(none.compile(src, dst, A, &p2));
  CHECK(p1 && p2 && p1.get() != p2.get());
  CHECK_EQ(none.cache_entries(), 0u);
  CHECK_EQ(none.cache_bytes(), 0u);
  CHECK(p1->operations.size() == p2->operations.size());
}

TEST_CASE("layout codec: overlapping or non-permutation layouts are rejected") {
  const auto schema = plain_schema();
  auto order = iota_order(schema.components.size());
  order.back() = order.front();
  LayoutDescriptor l;
  CHECK(!MakePackedLayout(schema, "duplicate", 1, order, {}, &l));
  REQUIRE(MakePackedLayout(schema, "overlap", 1, iota_order(schema.components.size()), {}, &l));
  l.components.back().offset_bytes = l.components.front().offset_bytes;
  CHECK(!l.validate(schema));
}

// ------------------------------------------------------------ backends

namespace {
// A backend that reports Pending until told otherwise and copies on success
// (test/test_page_migration.cpp:5-25 uses the same fake).
class DelayedBackend final : public TransferBackend {
 public:
  BoundTransfer bound;
  BackendResult next = BackendResult::kPending;
  bool copied = false;
  int submitted = 0, released = 0;
  bool supports(base::DeviceType d) const override { return d == base::DeviceType::kDeviceCPU; }
  BackendResult submit(MigrationId, TransferDirection, const BoundTransfer& t) noexcept override {
    bound = t;
    ++submitted;
    copied = false;
    return next;
  }
  BackendResult poll(MigrationId) noexcept override {
    if (next == BackendResult::kSucceeded && !copied) {
      if (!ExecuteCpuTransfer(bound)) return BackendResult::kFailedSafe;
      copied = true;
    }
    return next;
  }
  BackendResult drain(MigrationId id) noexcept override { return poll(id); }
  void release(MigrationId) noexcept override {
    ++released;
    bound = {};
  }
};
}  // namespace

TEST_CASE("backends: CPU backend copies synchronously; a fake shows pending states") {
  const auto schema = plain_schema();
  LayoutDescriptor l;
  REQUIRE(MakePackedLayout(schema, "p", 1, iota_order(schema.components.size()), {}, &l));
  std::vector<uint8_t> src(l.total_bytes, 0x38), dst(l.total_bytes, 0);
  TransferPlanner planner;
  TransferPlan plan;
  REQUIRE(planner.plan(schema, schema, &plan));
  BoundTransfer bound;
  REQUIRE(BoundTransfer::Bind(plan, schema, {src.data(), src.size(), &l}, {dst.data(), dst.size(), &l},
                              &bound));
  auto cpu = MakeCpuTransferBackend();
  CHECK(cpu->supports(base::DeviceType::kDeviceCPU));
  CHECK(!cpu->supports(base::DeviceType::kDeviceHIP));
  CHECK(cpu->submit(1, TransferDirection::kToHost, bound) == BackendResult::kSucceeded);
  CHECK(dst == src);
  CHECK(cpu->poll(1) == BackendResult::kSucceeded);
  CHECK(cpu->submit(2, TransferDirection::kToHost, BoundTransfer{}) == BackendResult::kSucceeded);

  std::fill(dst.begin(), dst.end(), 0);
  DelayedBackend fake;
  CHECK(fake.submit(3, TransferDirection::kToGpu, bound) == BackendResult::kPending);
  CHECK(fake.poll(3) == BackendResult::kPending);
  CHECK(dst != src);
  fake.next = BackendResult::kSucceeded;
  CHECK(fake.drain(3) == BackendResult::kSucceeded);
  CHECK(dst == src);
  fake.release(3);
  CHECK_EQ(fake.released, 1);
}

// ------------------------------------------------------------ handoff manifest

namespace {
serving::KVBlockManifest good_manifest() {
  serving::KVBlockManifest m;
  m.client_request_id.value = "req-1";
  m.handoff_id.value = 9;
  m.prompt_tokens = 41;
  m.computed_tokens = 41;
  m.src_pool = {0, 2, 16, 2, 64, base::DataType::kDataTypeBf16, base::BlockStorageMode::kPlain};
  m.dst_pool = m.src_pool;
  for (int l = 0; l < 2; ++l) m.layer_mappings.push_back({l, {0, 4, 8}, {12, 16, 20}});
  return m;
}
}  // namespace

TEST_CASE("manifest: validation mirrors the reference") {
  CHECK(good_manifest().validate());
  auto m = good_manifest();
  m.client_request_id.value.clear();
  CHECK(!m.validate());
  m = good_manifest();
  m.handoff_id.value = 0;
  CHECK(!m.validate());
  m = good_manifest();
  m.computed_tokens = 42;
  CHECK(!m.validate());
  m = good_manifest();
  m.dst_pool.head_size = 128;
  CHECK(!m.validate());
  m = good_manifest();
  m.layer_mappings.pop_back();
  CHECK(!m.validate());
  m = good_manifest();
  m.layer_mappings[1].dst_block_ids.pop_back();
  CHECK(!m.validate());
  m = good_manifest();
  m.layer_mappings[0].src_block_ids.clear();
  m.layer_mappings[0].dst_block_ids.clear();
  CHECK(!m.validate());
  serving::KVPoolDescriptor d = good_manifest().src_pool;
  CHECK_EQ(d.bytes_per_block_per_layer(), 2 * 16 * 2 * 64 * 2);
  d.storage_mode = base::BlockStorageMode::kFp8E4M3PerTokenHead;
  CHECK_EQ(d.bytes_per_block_per_layer(), 2 * 16 * 2 * 64 + 2 * 16 * 2 * 4);
}

TEST_CASE("storage spec: plain and FP8 specs and per-token bytes") {
  const auto plain = base::MakeKVCacheStorageSpec(base::DataType::kDataTypeBf16, base::BlockStorageMode::kPlain);
  CHECK(!plain.has_scales());
  CHECK(base::ValidateKVCacheStorageSpec(plain, base::DeviceType::kDeviceHIP, base::DataType::kDataTypeBf16));
  // Qwen2.5-1.5B: 28 layers, 2 KV heads x 128, BF16 -> 28 KiB per token.
  CHECK_EQ(base::KVCacheBytesPerToken(plain, 28, 2, 128), 28u * 1024u);
  const auto fp8 = base::MakeKVCacheStorageSpec(base::DataType::kDataTypeBf16,
                                                base::BlockStorageMode::kFp8E4M3PerTokenHead);
  CHECK(fp8.has_scales());
  CHECK(base::ValidateKVCacheStorageSpec(fp8, base::DeviceType::kDeviceHIP, base::DataType::kDataTypeBf16));
  CHECK(!base::ValidateKVCacheStorageSpec(fp8, base::DeviceType::kDeviceCPU, base::DataType::kDataTypeBf16));
  CHECK_EQ(base::KVCacheBytesPerToken(fp8, 28, 2, 128), 28u * 2 * 2 * 128 + 28u * 2 * 2 * 4);
}

// ------------------------------------------------------------ page group

namespace {
// Metadata-only arena mapping (device -1: nothing is ever launched on it).
pbe_arena_view fake_view(uint64_t bytes, uint64_t segment = 0) {
  pbe_arena_view v{};
  v.bytes = bytes;
  v.segment_bytes = segment ? segment : bytes;
  v.nseg = static_cast<uint32_t>((bytes + v.segment_bytes - 1) / v.segment_bytes);
  for (uint32_t i = 0; i < v.nseg; ++i) v.base[i] = reinterpret_cast<void*>(0x100000ull * (i + 1));
  return v;
}

struct Group {
  // 3 layers, half 4 KiB -> page 24 KiB; Chunk target 3 pages.
  static constexpr uint64_t kHalf = 4096, kPage = 6 * 4096;
  std::shared_ptr<base::LocalChunkOwner> owner;
  std::shared_ptr<base::SharedKVArenaClient> client;
  std::shared_ptr<base::SharedKVPageGroup> group;
  Group(uint64_t arena_pages, uint64_t limit_bytes, uint64_t target = 3 * kPage) {
    owner = std::make_shared<base::LocalChunkOwner>(arena_pages * kPage, 9);
    owner->register_model("d", limit_bytes);
    client = std::make_shared<base::SharedKVArenaClient>(owner, fake_view(arena_pages * kPage), "d",
                                                         limit_bytes, -1);
    group = std::make_shared<base::SharedKVPageGroup>(client, 3, kHalf, target, nullptr);
  }
  int page_id(int n) const { return n * 6; }  // block id of the n-th page
};
}  // namespace

TEST_CASE("page group: layer 0 picks pages, later layers take the same ids in order") {
  Group g(12, 12 * Group::kPage);
  CHECK_EQ(g.group->capacity(), 12);
  CHECK_EQ(g.group->addressable_blocks(), static_cast<int>(12 * 6 - 6 + 1));
  const int a = g.group->allocate(0);
  CHECK_EQ(a, g.page_id(0));
  CHECK_EQ(g.group->leased_bytes(), 3 * Group::kPage);  // one Chunk of 3 pages
  const int b = g.group->allocate(0);
  CHECK_EQ(b, g.page_id(1));
  CHECK_EQ(g.group->allocate(1), a);
  CHECK_EQ(g.group->allocate(1), b);
  CHECK_EQ(g.group->allocate(2), a);
  CHECK_EQ(g.group->allocate(2), b);
  CHECK_THROWS_AS(g.group->allocate(1), std::logic_error);
  CHECK_THROWS_AS(g.group->allocate(3), std::invalid_argument);
  // 9 unleased pages + 1 free page in the Chunk
  CHECK_EQ(g.group->free_blocks(0), 10);
  CHECK(g.group->key_base(1) == reinterpret_cast<char*>(0x100000) + 2 * Group::kHalf);
  CHECK(g.group->value_base(1) == reinterpret_cast<char*>(0x100000) + 3 * Group::kHalf);
}

TEST_CASE("page group: retire returns pages, Chunks go back to the owner when empty") {
  Group g(12, 12 * Group::kPage);
  std::vector<int> ids;
  for (int i = 0; i < 4; ++i) ids.push_back(g.group->allocate(0));  // spans two Chunks
  for (int l = 1; l < 3; ++l)
    for (int i = 0; i < 4; ++i) CHECK_EQ(g.group->allocate(l), ids[i]);
  CHECK_EQ(g.group->leased_bytes(), 6 * Group::kPage);
  CHECK_EQ(g.owner->lease_count(), 2u);
  for (int l = 0; l < 3; ++l) g.group->retire(l, ids[3]);
  CHECK_THROWS_AS(g.group->retire(0, ids[3]), std::logic_error);  // double retire
  CHECK_THROWS_AS(g.group->retire(0, 999), std::logic_error);     // not a page of this group
  // the second Chunk held only page 3: it is empty now and was released
  CHECK_EQ(g.owner->lease_count(), 1u);
  CHECK_EQ(g.group->leased_bytes(), 3 * Group::kPage);
  for (int i = 0; i < 3; ++i)
    for (int l = 0; l < 3; ++l) g.group->retire(l, ids[i]);
  CHECK_EQ(g.owner->lease_count(), 0u);
  CHECK_EQ(g.owner->free_bytes(), 12 * Group::kPage);
  // the lowest free id is reused first
  CHECK_EQ(g.group->allocate(0), g.page_id(0));
}

TEST_CASE("page group: retiring layer 0 first rolls back unconsumed reservations") {
  Group g(6, 6 * Group::kPage);
  const int id = g.group->allocate(0);
  CHECK_EQ(g.group->allocate(1), id);  // layer 2 never allocated
  g.group->retire(1, id);
  g.group->retire(0, id);               // drops the layer-2 reservation, page retires
  CHECK_THROWS_AS(g.group->allocate(2), std::logic_error);
  CHECK_EQ(g.owner->lease_count(), 0u);
}

TEST_CASE("page group: randomized reservations, rollbacks and retires against a model (long log)") {
  // 3 layers, 3000 pages: layer 0 may run far ahead of layers 1 and 2, so
  // the reservation log grows past its trimming threshold; layer-0 retires
  // roll back pages the later layers never took, in any position of the log.
  // The model: per layer, the FIFO of page ids layer 0 reserved and that
  // layer has not taken; per page, which layers hold it.
  Group g(3000, 3000 * Group::kPage);
  std::mt19937 rng(2024);
  std::vector<std::vector<int>> pending(3);  // layers 1, 2
  std::map<int, std::array<bool, 3>> held;   // page id -> layers holding it
  auto live_in = [&](int layer) {
    std::vector<int> ids;
    for (const auto& e : held)
      if (e.second[layer]) ids.push_back(e.first);
    return ids;
  };
  auto erase_pending = [&](int layer, int id) {
    auto& q = pending[layer];
    auto it = std::find(q.begin(), q.end(), id);
    if (it == q.end()) return false;
    q.erase(it);
    return true;
  };
  int max_log = 0;
  for (int step = 0; step < 12000; ++step) {
    const int phase = step < 4000 ? 0 : 1;  // first let layer 0 run ahead
    const int op = static_cast<int>(rng() % 10);
    if (op < (phase == 0 ? 6 : 3)) {
      // layer 0 takes 1..8 pages
      const int n = 1 + static_cast<int>(rng() % 8);
      std::vector<int32_t> got;
      // arena full part-way: the pages handed out before stay reserved
      if (!g.group->allocate_many(0, n, &got)) CHECK(got.size() < static_cast<size_t>(n));
      else REQUIRE(got.size() == static_cast<size_t>(n));
      for (int id : got) {
        CHECK(!held.count(id));  // never a page some layer still holds
        held[id] = {true, true, true};
        pending[1].push_back(id);
        pending[2].push_back(id);
      }
      max_log = std::max<int>(max_log, static_cast<int>(pending[2].size()));
    } else if (op < (phase == 0 ? 8 : 6)) {
      // a later layer takes the next k of layer 0's reservations, in order
      const int layer = 1 + static_cast<int>(rng() % 2);
      const int k = static_cast<int>(rng() % (phase == 0 ? 3 : 12));
      auto& q = pending[layer];
      if (static_cast<size_t>(k) > q.size()) {
        std::vector<int32_t> got;
        CHECK_THROWS_AS(g.group->allocate_many(layer, k, &got), std::logic_error);
        continue;
      }
      std::vector<int32_t> got;
      if (k == 1) got.push_back(g.group->allocate(layer));
      else CHECK(g.group->allocate_many(layer, k, &got));
      REQUIRE(got.size() == static_cast<size_t>(k));
      for (int i = 0; i < k; ++i) CHECK_EQ(got[i], q[i]);
      q.erase(q.begin(), q.begin() + k);
    } else {
      // retire one page from one layer that holds it (taken, not pending)
      const int layer = static_cast<int>(rng() % 3);
      std::vector<int> ids = live_in(layer);
      std::vector<int> taken;
      for (int id : ids)
        if (layer == 0 || std::find(pending[layer].begin(), pending[layer].end(), id) == pending[layer].end())
          taken.push_back(id);
      if (taken.empty()) continue;
      const int id = taken[rng() % taken.size()];
      g.group->retire(layer, id);
      held[id][layer] = false;
      if (layer == 0)  // reservations the later layers never took go with it
        for (int l = 1; l < 3; ++l)
          if (erase_pending(l, id)) held[id][l] = false;
      if (!held[id][0] && !held[id][1] && !held[id][2]) held.erase(id);
      CHECK_THROWS_AS(g.group->retire(layer, id), std::logic_error);  // no double retire
    }
    // free counts follow the model: later layers can take exactly their pending pages
    for (int l = 1; l < 3; ++l) {
      const int room = g.group->free_blocks(l) - g.group->free_blocks(0);
      CHECK_EQ(room, static_cast<int>(pending[l].size()));
    }
  }
  CHECK(max_log > 1024);  // the log's trimming ran
  // drain: later layers take what is pending, then every layer retires
  for (int l = 1; l < 3; ++l) {
    std::vector<int32_t> got;
    CHECK(g.group->allocate_many(l, static_cast<int>(pending[l].size()), &got));
    CHECK(got == std::vector<int32_t>(pending[l].begin(), pending[l].end()));
  }
  for (const auto& e : held)
    for (int l = 2; l >= 0; --l)
      if (e.second[l]) g.group->retire(l, e.first);
  CHECK_EQ(g.group->leased_bytes(), 0u);
  CHECK_EQ(g.owner->lease_count(), 0u);
}

TEST_CASE("page group: quota, single-page fallback and exhaustion") {
  // limit = one Chunk + one page: the second lease falls back to one page
  Group g(12, 4 * Group::kPage);
  for (int i = 0; i < 3; ++i) g.group->allocate(0);
  const int fourth = g.group->allocate(0);
  CHECK_EQ(fourth, g.page_id(3));
  CHECK_EQ(g.group->leased_bytes(), 4 * Group::kPage);
  CHECK_EQ(g.group->allocate(0), -1);  // hard limit reached
  // fragmented arena: no 3-page range left, one page still fits
  Group f(5, 5 * Group::kPage);
  auto blocker = f.owner->acquire("d", "other", Group::kPage, Group::kPage);  // page 0
  (void)blocker;
  const int x = f.group->allocate(0);  // Chunk at pages 1..3
  CHECK_EQ(x, f.page_id(1));
  f.group->allocate(0);
  f.group->allocate(0);
  const int y = f.group->allocate(0);  // only page 4 remains: single-page lease
  CHECK_EQ(y, f.page_id(4));
  CHECK_EQ(f.group->allocate(0), -1);
  CHECK_THROWS_AS(base::SharedKVPageGroup(f.client, 3, 100, 1, nullptr), std::invalid_argument);
  CHECK_THROWS_AS(base::SharedKVPageGroup(f.client, 0, 4096, 1, nullptr), std::invalid_argument);
}

TEST_CASE("page group: segmented mappings have no flat plane bases") {
  auto owner = std::make_shared<base::LocalChunkOwner>(12 * Group::kPage, 3);
  owner->register_model("d", 12 * Group::kPage);
  auto client = std::make_shared<base::SharedKVArenaClient>(
      owner, fake_view(12 * Group::kPage, 4 * Group::kPage), "d", 12 * Group::kPage, -1);
  base::SharedKVPageGroup group(client, 3, Group::kHalf, Group::kPage, nullptr);
  CHECK(group.key_base(0) == nullptr);
  CHECK(client->data() == nullptr);
  CHECK_THROWS_AS(base::SharedKVPageGroup(client, 3, 12288, 1, nullptr), std::invalid_argument);
  CHECK_THROWS_AS(base::SharedKVArenaClient(owner, fake_view(8 * Group::kPage), "d", 1, -1),
                  std::runtime_error);
}

// ------------------------------------------------------------ decode reservation

namespace {
serving::KVPoolDescriptor pool3() {
  // 3 layers, 16 tokens x 2 heads x 64 dims BF16: half = 4 KiB
  return {0, 3, 16, 2, 64, base::DataType::kDataTypeBf16, base::BlockStorageMode::kPlain};
}

// One shared-arena allocator per layer over the group, 16-token blocks of
// 2 heads x 64 dims (half = 4 KiB), as the decode runtime builds them.
std::unique_ptr<base::KVCacheManager> manager_over(const std::shared_ptr<base::SharedKVPageGroup>& g) {
  std::vector<std::unique_ptr<base::BlockAllocator>> layers;
  for (int l = 0; l < g->layers(); ++l)
    layers.push_back(std::make_unique<base::BlockAllocator>(16, 2, 64, g, l));
  return std::make_unique<base::KVCacheManager>(16, g->layers(), std::move(layers));
}

serving::DecodeKVReservationRequest request_for(int32_t computed, int32_t prompt, int32_t pages) {
  serving::DecodeKVReservationRequest r;
  r.client_request_id.value = "r";
  r.handoff_id.value = 5;
  r.prompt_tokens = prompt;
  r.computed_tokens = computed;
  r.first_token = 17;
  r.src_pool = pool3();
  std::vector<int32_t> ids;
  for (int32_t i = 0; i < pages; ++i) ids.push_back(600 + 6 * i);
  r.src_block_ids_per_layer.assign(3, ids);
  return r;
}
}  // namespace

TEST_CASE("kv cache manager: an allocator that throws part-way leaves every layer's table unchanged") {
  // Layers 0 and 2 over group a, layer 1 over group b: layer 1's allocate
  // throws (group b holds no layer-0 reservations), after layer 0 has taken
  // its pages. append_slots must give those pages back and rethrow.
  Group a(12, 12 * Group::kPage), b(12, 12 * Group::kPage);
  std::vector<std::unique_ptr<base::BlockAllocator>> layers;
  layers.push_back(std::make_unique<base::BlockAllocator>(16, 2, 64, a.group, 0));
  layers.push_back(std::make_unique<base::BlockAllocator>(16, 2, 64, b.group, 1));
  layers.push_back(std::make_unique<base::BlockAllocator>(16, 2, 64, a.group, 2));
  base::KVCacheManager kv(16, 3, std::move(layers));
  const base::RequestId id = kv.register_request();
  const int32_t free0 = kv.num_free_blocks(0);
  CHECK_THROWS_AS(kv.append_slots(id, 40), std::logic_error);
  for (int l = 0; l < 3; ++l) CHECK(kv.get_block_ids(id, l).empty());
  CHECK_EQ(kv.get_context_len(id), 0);
  CHECK_EQ(kv.num_free_blocks(0), free0);
  CHECK_EQ(a.group->leased_bytes(), 0u);  // layer 0's pages went back, Chunk released
  CHECK_EQ(a.owner->lease_count(), 0u);
  kv.free_request(id);
  CHECK_EQ(kv.num_active_requests(), 0);
}

TEST_CASE("decode reservation: ceil(tokens/16) page-major pages and a valid manifest") {
  Group g(24, 24 * Group::kPage);
  auto kv = manager_over(g.group);
  serving::DecodeKVReservationManager mgr(kv.get(), pool3());
  serving::DecodeKVReservation res;
  serving::KVBlockManifest man;
  REQUIRE(mgr.reserve(request_for(41, 50, 4), &res, &man));
  CHECK(res.valid());
  CHECK_EQ(res.reserved_tokens, 41);
  CHECK_EQ(res.first_token, 17);
  REQUIRE(man.layer_mappings.size() == 3u);
  for (int l = 0; l < 3; ++l) {
    CHECK_EQ(man.layer_mappings[l].layer_idx, l);
    CHECK_EQ(man.layer_mappings[l].src_block_ids.size(), 3u);  // truncated to 3 pages
    CHECK(man.layer_mappings[l].dst_block_ids == man.layer_mappings[0].dst_block_ids);
  }
  CHECK(man.layer_mappings[0].dst_block_ids == (std::vector<int32_t>{0, 6, 12}));
  CHECK(man.validate());
  const auto leased = g.group->leased_bytes();
  mgr.release(&res);
  CHECK(!res.valid());
  CHECK_EQ(g.owner->lease_count(), 0u);
  (void)leased;
}

TEST_CASE("decode reservation: invalid requests and exhaustion reserve nothing") {
  Group g(6, 3 * Group::kPage);
  auto kv = manager_over(g.group);
  serving::DecodeKVReservationManager mgr(kv.get(), pool3());
  serving::DecodeKVReservation res;
  serving::KVBlockManifest man;
  auto r = request_for(41, 50, 4);
  r.client_request_id.value.clear();
  CHECK(!mgr.reserve(r, &res, &man));
  r = request_for(41, 40, 4);
  CHECK(!mgr.reserve(r, &res, &man));  // computed > prompt
  r = request_for(41, 50, 2);
  CHECK(!mgr.reserve(r, &res, &man));  // too few source pages
  r = request_for(41, 50, 4);
  r.src_pool.head_size = 128;
  CHECK(!mgr.reserve(r, &res, &man));  // incompatible pools
  r = request_for(41, 50, 4);
  r.src_block_ids_per_layer.pop_back();
  CHECK(!mgr.reserve(r, &res, &man));
  CHECK(!res.valid());
  // 4 pages needed, the limit allows 3: fails and rolls back
  r = request_for(64, 64, 4);
  CHECK(!mgr.reserve(r, &res, &man));
  CHECK_EQ(g.owner->lease_count(), 0u);
  CHECK(man.layer_mappings.empty());
  CHECK(mgr.reserve(request_for(48, 48, 3), &res, &man));
  mgr.release(&res);
}

// ------------------------------------------------------------ generic plan form

TEST_CASE("bind manifest transfers: 2L component ops per page at page-major addresses") {
  serving::ArenaKVPool pool;
  pool.pool = pool3();  // 3 layers, half 4 KiB
  pool.view = fake_view(40 * Group::kPage);
  auto m = good_manifest();
  m.src_pool = m.dst_pool = pool3();
  m.layer_mappings.clear();
  for (int l = 0; l < 3; ++l) m.layer_mappings.push_back({l, {0, 6, 30}, {60, 66, 120}});
  cache::TransferPlanner planner;
  std::vector<cache::BoundTransfer> t;
  REQUIRE(serving::BindManifestTransfers(m, pool, pool, &planner, &t));
  REQUIRE(t.size() == 3u);
  const uint64_t half = Group::kHalf;
  const uint8_t* base = static_cast<const uint8_t*>(pool.view.base[0]);
  for (size_t page = 0; page < 3; ++page) {
    CHECK_EQ(t[page].operations().size(), 6u);
    for (const auto& op : t[page].operations()) {
      const uint64_t plane = 2 * op.component.layer + (op.component.kind == cache::ComponentKind::kValue);
      const uint64_t s_id = m.layer_mappings[0].src_block_ids[page];
      const uint64_t d_id = m.layer_mappings[0].dst_block_ids[page];
      CHECK(op.source == base + (s_id + plane) * half);
      CHECK(op.destination == base + (d_id + plane) * half);
      CHECK_EQ(op.bytes, half);
    }
  }
  // the plan template was compiled once
  std::vector<cache::BoundTransfer> again;
  REQUIRE(serving::BindManifestTransfers(m, pool, pool, &planner, &again));
  CHECK_EQ(planner.cache_hits(), 1u);
  // errors bind nothing
  auto bad = m;
  bad.layer_mappings[1].dst_block_ids[0] = 40 * 6;  // past the arena
  std::vector<cache::BoundTransfer> none;
  CHECK(!serving::BindManifestTransfers(bad, pool, pool, &planner, &none));
  CHECK(none.empty());
  bad = m;
  bad.layer_mappings[2].layer_idx = 1;  // duplicate layer
  CHECK(!serving::BindManifestTransfers(bad, pool, pool, &planner, &none));
  bad = m;
  bad.layer_mappings[0].src_block_ids[1] = 7;  // not a page id
  CHECK(!serving::BindManifestTransfers(bad, pool, pool, &planner, &none));
  auto fp8 = pool;
  fp8.pool.storage_mode = base::BlockStorageMode::kFp8E4M3PerTokenHead;
  CHECK(!serving::BindManifestTransfers(m, pool, fp8, &planner, &none));  // conversion: no plan
}

TEST_CASE("bind manifest copy ops: the flattened transfers, page after page, with the same errors") {
  std::mt19937 rng(31);
  for (bool fp8 : {false, true})
    for (uint64_t segment : {uint64_t{0}, uint64_t{4 * Group::kPage}}) {
      serving::ArenaKVPool pool;
      pool.pool = pool3();
      if (fp8) pool.pool.storage_mode = base::BlockStorageMode::kFp8E4M3PerTokenHead;
      const uint64_t page = fp8 ? Group::kPage / 2 : Group::kPage;
      pool.view = fake_view(40 * page, segment ? segment / (fp8 ? 2 : 1) : 0);
      std::vector<uint8_t> scales(40 * 2 * 3 * 16 * 2 * 4);
      if (fp8) {
        pool.scales = scales.data();
        pool.scale_bytes = scales.size();
      }
      std::vector<int32_t> ids(40);
      std::iota(ids.begin(), ids.end(), 0);
      std::shuffle(ids.begin(), ids.end(), rng);
      std::vector<int32_t> src, dst;
      for (int i = 0; i < 13; ++i) {
        src.push_back(ids[i] * 6);
        dst.push_back(ids[20 + i] * 6);
      }
      auto m = good_manifest();
      m.src_pool = m.dst_pool = pool.pool;
      m.layer_mappings.clear();
      for (int l = 0; l < 3; ++l) m.layer_mappings.push_back({l, src, dst});
      cache::TransferPlanner planner;
      std::vector<cache::BoundTransfer> t;
      REQUIRE(serving::BindManifestTransfers(m, pool, pool, &planner, &t));
      std::vector<pbe_copy_op> want;
      for (const auto& x : t)
        for (const auto& op : x.operations())
          want.push_back({reinterpret_cast<uint64_t>(op.source), reinterpret_cast<uint64_t>(op.destination), op.bytes});
      std::vector<pbe_copy_op> got;
      REQUIRE(serving::BindManifestCopyOps(m, pool, pool, &planner, &got));
      REQUIRE(got.size() == want.size());
      CHECK_EQ(got.size(), 13u * 6u * (fp8 ? 2u : 1u));
      for (size_t i = 0; i < got.size(); ++i) {
        CHECK_EQ(got[i].src, want[i].src);
        CHECK_EQ(got[i].dst, want[i].dst);
        CHECK_EQ(got[i].bytes, want[i].bytes);
      }
      // a bad id on the first or a later page fails both forms with one message
      for (size_t bad_page : {size_t{0}, size_t{7}}) {
        for (bool on_dst : {false, true}) {
          auto b = m;
          for (auto& lm : b.layer_mappings) (on_dst ? lm.dst_block_ids : lm.src_block_ids)[bad_page] = 40 * 6;
          std::vector<cache::BoundTransfer> none;
          std::vector<pbe_copy_op> no_ops;
          const auto e1 = serving::BindManifestTransfers(b, pool, pool, &planner, &none);
          const auto e2 = serving::BindManifestCopyOps(b, pool, pool, &planner, &no_ops);
          CHECK(!e1);
          CHECK(!e2);
          CHECK(e1.get_err_msg() == e2.get_err_msg());
          CHECK(no_ops.empty());
        }
      }
    }
}

TEST_CASE("bind manifest transfers: FP8 pools add scale components") {
  serving::ArenaKVPool pool;
  pool.pool = pool3();
  pool.pool.storage_mode = base::BlockStorageMode::kFp8E4M3PerTokenHead;
  pool.view = fake_view(20 * Group::kPage / 2);  // FP8 half = 2 KiB
  std::vector<uint8_t> scales(20 * 2 * 3 * 16 * 2 * 4);
  pool.scales = scales.data();
  pool.scale_bytes = scales.size();
  auto m = good_manifest();
  m.src_pool = m.dst_pool = pool.pool;
  m.layer_mappings.clear();
  for (int l = 0; l < 3; ++l) m.layer_mappings.push_back({l, {0, 6}, {12, 18}});
  cache::TransferPlanner planner;
  std::vector<cache::BoundTransfer> t;
  REQUIRE(serving::BindManifestTransfers(m, pool, pool, &planner, &t));
  REQUIRE(t.size() == 2u);
  CHECK_EQ(t[0].operations().size(), 12u);  // K, V, K-scale, V-scale per layer
  size_t scale_ops = 0;
  for (const auto& op : t[1].operations())
    if (op.component.kind == cache::ComponentKind::kKeyScale) {
      ++scale_ops;
      // page 3 (id 18) -> scale page 3, plane 2*layer
      CHECK(op.destination == scales.data() + (3 * 6 + 2 * op.component.layer) * 32 * 4);
      CHECK_EQ(op.bytes, 32u * 4u);
    }
  CHECK_EQ(scale_ops, 3u);
  pool.scales = nullptr;
  std::vector<cache::BoundTransfer> none;
  CHECK(!serving::BindManifestTransfers(m, pool, pool, &planner, &none));
}

TEST_CASE("kv page wire: per-layer id lists round trip through the compact form") {
  const int L = 4;
  std::vector<int32_t> ids = {0, 8, 16, 64, 72, 24, 200, 208, 216, 224};
  std::vector<serving::RemoteKVLayerPayload> layers;
  for (int l = 0; l < L; ++l) layers.push_back({l, ids});
  std::string wire;
  REQUIRE(serving::EncodeKVPageList(77, layers, &wire));
  CHECK_EQ(wire.size(), 32u + 4u * 8u);  // spans {0,3} {64,2} {24,1} {200,4}
  uint64_t epoch = 0;
  std::vector<serving::RemoteKVLayerPayload> back;
  REQUIRE(serving::DecodeKVPageList(wire, &epoch, &back));
  CHECK_EQ(epoch, 77u);
  REQUIRE(back.size() == layers.size());
  for (int l = 0; l < L; ++l) {
    CHECK_EQ(back[l].layer_idx, l);
    CHECK(back[l].src_block_ids == ids);
  }
  int32_t n_layers = 0;
  std::vector<int32_t> flat;
  REQUIRE(serving::DecodeKVPageIds(wire, &epoch, &n_layers, &flat));
  CHECK_EQ(n_layers, L);
  CHECK(flat == ids);
  // a bound on the page count (the arena's capacity) is enforced before allocating
  CHECK(!serving::DecodeKVPageIds(wire, &epoch, &n_layers, &flat, 9));
  CHECK(!serving::DecodeKVPageList(wire, &epoch, &back, 9));
  REQUIRE(serving::DecodeKVPageIds(wire, &epoch, &n_layers, &flat, 10));
  CHECK(flat == ids);
  // empty prefix: header only
  std::vector<serving::RemoteKVLayerPayload> empty{{0, {}}, {1, {}}};
  REQUIRE(serving::EncodeKVPageList(5, empty, &wire));
  CHECK_EQ(wire.size(), 32u);
  REQUIRE(serving::DecodeKVPageList(wire, &epoch, &back));
  CHECK_EQ(back.size(), 2u);
  CHECK(back[1].src_block_ids.empty());
}

TEST_CASE("kv page wire: copy_shared_kv's layer checks and corrupt input are rejected") {
  std::vector<int32_t> ids = {0, 4, 8};
  std::vector<serving::RemoteKVLayerPayload> layers{{0, ids}, {1, ids}};
  std::string wire;
  auto bad = layers;
  bad[1].src_block_ids[2] = 12;
  CHECK(!serving::EncodeKVPageList(1, bad, &wire));  // layers disagree
  CHECK(wire.empty());
  bad = layers;
  bad[1].layer_idx = 0;
  CHECK(!serving::EncodeKVPageList(1, bad, &wire));  // layer order
  bad = layers;
  bad[0].src_block_ids[1] = bad[1].src_block_ids[1] = 6;  // not a multiple of 2L = 4
  CHECK(!serving::EncodeKVPageList(1, bad, &wire));
  CHECK(!serving::EncodeKVPageList(1, {}, &wire));
  REQUIRE(serving::EncodeKVPageList(9, layers, &wire));
  uint64_t epoch = 0;
  std::vector<serving::RemoteKVLayerPayload> back;
  for (size_t i = 0; i < wire.size(); ++i) {
    std::string w = wire;
    w[i] = static_cast<char>(w[i] ^ 0x10);
    CHECK(!serving::DecodeKVPageList(w, &epoch, &back));
    CHECK(back.empty());
  }
  CHECK(!serving::DecodeKVPageList(wire.substr(0, wire.size() - 1), &epoch, &back));
  CHECK(!serving::DecodeKVPageList(wire + std::string(8, '\0'), &epoch, &back));
  CHECK(!serving::DecodeKVPageList(std::string(), &epoch, &back));
}

namespace {
// Prefill ("p") and decode ("d") page groups over one owner; 3 layers, page
// 24 KiB, Chunks of 3 pages.
struct TwoGroups {
  static constexpr uint64_t kHalf = 4096, kPage = 6 * 4096;
  std::shared_ptr<base::LocalChunkOwner> owner;
  std::shared_ptr<base::SharedKVArenaClient> pc, dc;
  std::unique_ptr<base::SharedKVPageGroup> p, d;
  TwoGroups(uint64_t arena_pages, uint64_t p_limit, uint64_t d_limit) {
    owner = std::make_shared<base::LocalChunkOwner>(arena_pages * kPage, 11);
    owner->register_model("p", p_limit * kPage);
    owner->register_model("d", d_limit * kPage);
    pc = std::make_shared<base::SharedKVArenaClient>(owner, fake_view(arena_pages * kPage), "p",
                                                     p_limit * kPage, -1);
    dc = std::make_shared<base::SharedKVArenaClient>(owner, fake_view(arena_pages * kPage), "d",
                                                     d_limit * kPage, -1);
    p = std::make_unique<base::SharedKVPageGroup>(pc, 3, kHalf, 3 * kPage, nullptr);
    d = std::make_unique<base::SharedKVPageGroup>(dc, 3, kHalf, 3 * kPage, nullptr);
  }
  // Allocates n pages in every layer of group g, as a model does.
  static std::vector<int32_t> alloc(base::SharedKVPageGroup& g, int n) {
    std::vector<int32_t> ids;
    for (int i = 0; i < n; ++i) ids.push_back(g.allocate(0));
    for (int l = 1; l < 3; ++l)
      for (int i = 0; i < n; ++i) CHECK_EQ(g.allocate(l), ids[i]);
    return ids;
  }
  static void retire_all(base::SharedKVPageGroup& g, const std::vector<int32_t>& ids) {
    for (int32_t id : ids)
      for (int l = 0; l < 3; ++l) g.retire(l, id);
  }
};
}  // namespace

TEST_CASE("chunk allocator: transfer moves quota and identity, all or nothing") {
  base::GlobalChunkAllocator a(100, 5);
  a.register_model("p", 60);
  a.register_model("d", 40);
  auto x = a.acquire("p", "L", 20, 10);
  auto y = a.acquire("p", "L", 30, 10);
  CHECK_THROWS_AS(a.transfer({x, y}, "d"), base::ChunkAllocationError);  // 50 > 40
  CHECK_EQ(a.leased_bytes("p"), 50u);
  CHECK_EQ(a.leased_bytes("d"), 0u);
  CHECK_THROWS_AS(a.transfer({y, y}, "d"), std::invalid_argument);
  CHECK_THROWS_AS(a.transfer({y}, "p"), std::invalid_argument);
  CHECK_THROWS_AS(a.transfer({y}, "nobody"), std::invalid_argument);
  auto moved = a.transfer({x}, "d");
  REQUIRE(moved.size() == 1u);
  CHECK_EQ(moved[0].id, x.id);
  CHECK_EQ(moved[0].offset, x.offset);
  CHECK_EQ(moved[0].bytes, x.bytes);
  CHECK(moved[0].generation != x.generation);
  CHECK_EQ(moved[0].model, std::string("d"));
  CHECK_EQ(a.leased_bytes("p"), 30u);
  CHECK_EQ(a.leased_bytes("d"), 20u);
  CHECK_EQ(a.lease_count(), 2u);
  CHECK_THROWS_AS(a.release(x), std::invalid_argument);  // the old holder's identity is stale
  auto z = a.acquire("d", "L", 10, 10);
  CHECK(z.id != x.id && z.id != y.id && z.id != moved[0].id);
  a.release(moved[0]);
  a.release(y);
  a.release(z);
  CHECK_EQ(a.free_bytes(), 100u);
}

TEST_CASE("page takeover: exclusive Chunks move whole, shared ones are copied") {
  TwoGroups t(30, 15, 15);
  // request A: 4 pages (Chunks {0,1,2} and {3,4,5}); request B: 1 page, sharing Chunk 2
  auto a = TwoGroups::alloc(*t.p, 4);
  auto b = TwoGroups::alloc(*t.p, 1);
  CHECK_EQ(a[0], 0);
  CHECK_EQ(b[0], 4 * 6);
  CHECK_EQ(t.owner->leased_bytes("p"), 6 * TwoGroups::kPage);
  base::SharedKVPageGroup::PageTakeover tk;
  t.p->detach_for_takeover(a, &tk);
  REQUIRE(tk.chunks.size() == 1u);                 // Chunk {0,1,2}; page 3 shares a Chunk with B
  CHECK(tk.moved_ids == std::vector<int32_t>({0, 6, 12}));
  CHECK(tk.copy_ids == std::vector<int32_t>({18}));
  CHECK_EQ(t.p->leased_bytes(), 3 * TwoGroups::kPage);
  CHECK_THROWS_AS(t.p->retire(0, 0), std::logic_error);  // no longer the source's page
  CHECK_EQ(t.d->adopt(tk), 3u);
  t.p->finish_takeover(tk);
  CHECK_EQ(t.owner->leased_bytes("p"), 3 * TwoGroups::kPage);
  CHECK_EQ(t.owner->leased_bytes("d"), 3 * TwoGroups::kPage);
  CHECK_EQ(t.d->leased_bytes(), 3 * TwoGroups::kPage);
  // the receiver uses and retires the pages like its own
  auto more = TwoGroups::alloc(*t.d, 1);             // a fresh Chunk of its own
  CHECK(std::find(tk.moved_ids.begin(), tk.moved_ids.end(), more[0]) == tk.moved_ids.end());
  const size_t leases = t.owner->lease_count();
  TwoGroups::retire_all(*t.d, tk.moved_ids);
  t.d->collect();
  CHECK_EQ(t.owner->lease_count(), leases - 1);      // the adopted Chunk went back to the owner
  CHECK_EQ(t.owner->leased_bytes("d"), 3 * TwoGroups::kPage);
  // the source still retires the copied page and B normally
  TwoGroups::retire_all(*t.p, {18});
  TwoGroups::retire_all(*t.p, b);
  t.p->collect();
  CHECK_EQ(t.owner->leased_bytes("p"), 0u);
}

TEST_CASE("page takeover: refused adoption leaves both sides as they were") {
  TwoGroups t(30, 15, 2);                            // receiver limit: 2 pages
  auto a = TwoGroups::alloc(*t.p, 3);
  base::SharedKVPageGroup::PageTakeover tk;
  t.p->detach_for_takeover(a, &tk);
  REQUIRE(tk.chunks.size() == 1u);
  CHECK_THROWS_AS(t.d->adopt(tk), base::ChunkAllocationError);
  CHECK_EQ(t.owner->leased_bytes("d"), 0u);
  CHECK_EQ(t.d->leased_bytes(), 0u);
  t.p->reattach(tk);
  CHECK_EQ(t.p->leased_bytes(), 3 * TwoGroups::kPage);
  TwoGroups::retire_all(*t.p, a);                    // the source owns them again
  t.p->collect();
  CHECK_EQ(t.owner->leased_bytes("p"), 0u);
  CHECK_EQ(t.owner->lease_count(), 0u);
}

TEST_CASE("page takeover: stale identities, bad inputs and geometry mismatches are rejected") {
  TwoGroups t(30, 15, 15);
  auto a = TwoGroups::alloc(*t.p, 3);
  base::SharedKVPageGroup::PageTakeover tk;
  CHECK_THROWS_AS(t.p->detach_for_takeover({a[0], a[0]}, &tk), std::logic_error);
  CHECK_THROWS_AS(t.p->detach_for_takeover({7}, &tk), std::logic_error);
  const int half = t.p->allocate(0);                 // layer 0 only: not a finished page
  CHECK_THROWS_AS(t.p->detach_for_takeover({half}, &tk), std::logic_error);
  t.p->retire(0, half);
  t.p->detach_for_takeover(a, &tk);
  auto old = tk.chunks;
  REQUIRE(t.d->adopt(tk) == 3u);
  CHECK_THROWS_AS(t.owner->release(old[0]), std::invalid_argument);  // the source's identity is stale
  CHECK_THROWS_AS(t.d->adopt(tk), std::logic_error);                 // already held
  auto wrong = tk;
  wrong.epoch = 99;
  CHECK_THROWS_AS(t.d->adopt(wrong), std::invalid_argument);
  // a receiver with another geometry refuses the Chunk before asking the owner
  base::SharedKVPageGroup other(t.dc, 2, TwoGroups::kHalf, 3 * TwoGroups::kPage, nullptr);
  base::SharedKVPageGroup::PageTakeover tk2;
  auto b = TwoGroups::alloc(*t.p, 3);
  t.p->detach_for_takeover(b, &tk2);
  CHECK_THROWS_AS(other.adopt(tk2), std::invalid_argument);
  t.p->reattach(tk2);
  TwoGroups::retire_all(*t.p, b);
}

TEST_CASE("TakeOverSharedKV: whole-Chunk requests move without a copy; refusals change nothing") {
  TwoGroups t(30, 15, 15);
  auto a = TwoGroups::alloc(*t.p, 6);  // two whole 3-page Chunks
  base::SharedKVPageGroup::PageTakeover tk;
  t.p->detach_for_takeover(a, &tk);
  REQUIRE(tk.copy_ids.empty());
  serving::KVPoolDescriptor pool{0, 3, 16, 2, 64, base::DataType::kDataTypeBf16,
                                 base::BlockStorageMode::kPlain};
  serving::SharedArenaBinding binding{fake_view(30 * TwoGroups::kPage), 11, -1};
  std::vector<int32_t> table;
  uint64_t copied = 7;
  REQUIRE(serving::TakeOverSharedKV(t.d.get(), binding, tk, pool, nullptr, &table, &copied));
  t.p->finish_takeover(tk);
  CHECK(table == a);
  CHECK_EQ(copied, 0u);
  CHECK_EQ(t.owner->leased_bytes("d"), 6 * TwoGroups::kPage);
  // a receiver without quota refuses; the source takes its Chunks back
  TwoGroups u(30, 15, 2);
  auto b = TwoGroups::alloc(*u.p, 3);
  base::SharedKVPageGroup::PageTakeover tk2;
  u.p->detach_for_takeover(b, &tk2);
  serving::SharedArenaBinding ub{fake_view(30 * TwoGroups::kPage), 11, -1};
  auto st = serving::TakeOverSharedKV(u.d.get(), ub, tk2, pool, nullptr, &table, &copied);
  CHECK(!st);
  CHECK(table.empty());
  CHECK_EQ(u.d->leased_bytes(), 0u);
  u.p->reattach(tk2);
  TwoGroups::retire_all(*u.p, b);
  u.p->collect();
  CHECK_EQ(u.owner->lease_count(), 0u);
  // layer-count mismatch is rejected before anything is adopted
  TwoGroups v(30, 15, 15);
  auto c = TwoGroups::alloc(*v.p, 3);
  base::SharedKVPageGroup::PageTakeover tk3;
  v.p->detach_for_takeover(c, &tk3);
  auto bad_pool = pool;
  bad_pool.layer_num = 4;
  CHECK(!serving::TakeOverSharedKV(v.d.get(), binding, tk3, bad_pool, nullptr, &table, &copied));
  CHECK_EQ(v.d->leased_bytes(), 0u);
  v.p->reattach(tk3);
  TwoGroups::retire_all(*v.p, c);
}

TEST_CASE("page index: multiply-shift quotient equals id / stride, -1 off the page grid") {
  // every id below 2^20 for every even stride 2..256 (2L for 1..128 layers),
  // and a spread of ids up to INT32_MAX
  std::mt19937 rng(11);
  for (int32_t stride = 2; stride <= 256; stride += 2) {
    const base::PageIndex pi(stride);
    for (int32_t id = 0; id < (1 << 20); ++id)
      REQUIRE(pi.of(id) == (id % stride == 0 ? id / stride : -1));
    for (int k = 0; k < 20000; ++k) {
      const int32_t id = static_cast<int32_t>(rng() & 0x7fffffffu);
      REQUIRE(pi.of(id) == (id % stride == 0 ? id / stride : -1));
      const int32_t page = id / stride;
      REQUIRE(pi.of(page * stride) == page);
    }
    CHECK_EQ(pi.of(-stride), -1);
    CHECK_EQ(pi.of(INT32_MAX - INT32_MAX % stride), INT32_MAX / stride);
  }
  CHECK_EQ(base::PageIndex(1).of(12345), 12345);
}

TEST_CASE("xcd grouping: the copy kernels' workgroup renumbering is a bijection") {
  // every grid size up to 5,000 workgroups and a few large ones, for group
  // sizes 1..128 (the copy kernels use 24 and 48)
  std::vector<uint32_t> sizes;
  for (uint32_t nb = 1; nb <= 5000; ++nb) sizes.push_back(nb);
  for (uint32_t nb : {17640u, 35281u, 65536u, 1048575u}) sizes.push_back(nb);
  std::vector<uint32_t> seen;
  for (uint32_t g : {1u, 2u, 3u, 16u, 24u, 48u, 64u, 128u}) {
    for (uint32_t nb : sizes) {
      if (nb > 5000 && g != 24 && g != 48) continue;
      seen.assign(nb, 0);
      for (uint32_t b = 0; b < nb; ++b) {
        const uint32_t at = pbe::xcd_grouped(b, nb, g);
        REQUIRE(at < nb);
        ++seen[at];
      }
      REQUIRE(std::all_of(seen.begin(), seen.end(), [](uint32_t c) { return c == 1; }));
    }
  }
  // a full round: XCD x (workgroups x, x + 8, ...) holds positions [16x, 16x + 16)
  for (uint32_t b = 0; b < 128; ++b) {
    const uint32_t at = pbe::xcd_grouped(b, 128, 16);
    REQUIRE(at / 16 == b % pbe::kXcds);
    REQUIRE(at % 16 == b / pbe::kXcds);
  }
  // the trailing partial round keeps dispatch order
  CHECK_EQ(pbe::xcd_grouped(130, 131, 16), 130u);
  CHECK_EQ(pbe::xcd_grouped(5, 7, 1), 5u);
}

TEST_CASE("block allocator (shared arena): per-layer ids, refcounts, payload pointers") {
  auto owner = std::make_shared<base::LocalChunkOwner>(12 * Group::kPage, 9);
  owner->register_model("d", 12 * Group::kPage);
  // segmented mapping: 4 segments of 3 pages; group geometry: 3 layers, half 4 KiB
  pbe_arena_view view = fake_view(12 * Group::kPage, 3 * Group::kPage);
  auto client = std::make_shared<base::SharedKVArenaClient>(owner, view, "d", 12 * Group::kPage, -1);
  auto group = std::make_shared<base::SharedKVPageGroup>(client, 3, Group::kHalf, 3 * Group::kPage, nullptr);
  // block_size 16 x 1 head x 128 dims x 2 B = 4 KiB = half
  CHECK_THROWS_AS(base::BlockAllocator(16, 2, 128, group, 0), std::invalid_argument);
  CHECK_THROWS_AS(base::BlockAllocator(16, 1, 128, group, 3), std::invalid_argument);
  std::vector<std::unique_ptr<base::BlockAllocator>> layers;
  for (int l = 0; l < 3; ++l) layers.push_back(std::make_unique<base::BlockAllocator>(16, 1, 128, group, l));
  CHECK_EQ(layers[0]->num_total_blocks(), 12);
  const int a = layers[0]->allocate();
  const int b = layers[0]->allocate();
  CHECK_EQ(layers[1]->allocate(), a);
  CHECK_EQ(layers[2]->allocate(), a);
  CHECK_EQ(layers[1]->allocate(), b);
  CHECK_EQ(layers[2]->allocate(), b);
  // payload pointers: K of layer l = half-plane id + 2l, V = id + 2l + 1, through the segments
  for (int l = 0; l < 3; ++l) {
    for (int id : {a, b}) {
      auto p = layers[l]->get_block_payload_ptrs(id);
      const uint64_t koff = (uint64_t)(id + 2 * l) * Group::kHalf, voff = koff + Group::kHalf;
      const uint64_t seg = 3 * Group::kPage;
      CHECK(p.key == static_cast<char*>(view.base[koff / seg]) + koff % seg);
      CHECK(p.value == static_cast<char*>(view.base[voff / seg]) + voff % seg);
      CHECK_EQ(p.key_value_bytes, (size_t)Group::kHalf);
      CHECK(p.key_scale == nullptr);
    }
  }
  auto h = layers[0]->handle(a);
  CHECK(layers[0]->is_current(h));
  layers[0]->incref(a);
  CHECK_EQ(layers[0]->ref_count(a), 2);
  layers[0]->free(a);
  CHECK(layers[0]->is_current(h));
  for (int l = 0; l < 3; ++l) layers[l]->free(a);  // last references retire the page
  CHECK(!layers[0]->is_current(h));
  CHECK_THROWS_AS(layers[0]->free(a), std::logic_error);
  CHECK_THROWS_AS(layers[0]->get_block_payload_ptrs(-1), std::out_of_range);
  // the retired page is the lowest free id again, with a new generation
  CHECK_EQ(layers[0]->allocate(), a);
  CHECK(!layers[0]->is_current(h));
  CHECK_EQ(layers[0]->shared_arena_epoch(), 9u);
  CHECK_EQ(layers[0]->shared_arena_bytes(), (size_t)(12 * Group::kPage));
  // ids that are not page ids (not multiples of 2L = 6) are never allocated:
  // no references, no handle, and incref/free refuse them like a free block;
  // ids past the arena are out of range
  for (int l = 0; l < 3; ++l) {
    for (int id : {a + 1, a + 5, b + 3}) {
      CHECK_EQ(layers[l]->ref_count(id), 0);
      CHECK_THROWS_AS(layers[l]->incref(id), std::logic_error);
      CHECK_THROWS_AS(layers[l]->free(id), std::logic_error);
      CHECK_THROWS_AS(layers[l]->handle(id), std::logic_error);
      CHECK(!layers[l]->is_current(base::BlockHandle{id, 1, h.pool_id}));
    }
    CHECK_THROWS_AS(layers[l]->ref_count(1 << 30), std::out_of_range);
  }
  // the page counts stay per page: b still holds one reference per layer
  for (int l = 0; l < 3; ++l) CHECK_EQ(layers[l]->ref_count(b), 1);
}

TEST_CASE("block allocator: the pool view binds the planes without owning the allocation queue") {
  // test_kv_pool_view.cpp:5-25, in shared-arena mode over a one-segment mapping
  Group g(12, 12 * Group::kPage);
  std::shared_ptr<base::SharedKVPageGroup> group(std::move(g.group));
  base::BlockAllocator layer1(16, 1, 128, group, 1);
  const int32_t free_before = layer1.num_free_blocks();
  const base::KVPoolView view = layer1.pool_view();
  REQUIRE(view.valid());
  CHECK(view.device_type() == base::DeviceType::kDeviceHIP);
  CHECK(view.key_pool() == group->key_base(1));
  CHECK(view.value_pool() == group->value_base(1));
  CHECK(!view.uses_fp8_storage());
  CHECK_EQ(view.block_stride(), (size_t)Group::kHalf);
  CHECK_EQ(layer1.num_free_blocks(), free_before);
  base::BlockAllocator layer0(16, 1, 128, group, 0);
  const int32_t block = layer0.allocate();
  REQUIRE(block >= 0);
  CHECK_EQ(layer1.allocate(), block);
  CHECK_EQ(layer1.num_free_blocks(), free_before - 1);
  // copying the descriptor does not affect physical ownership
  const base::KVPoolView imported = view;
  CHECK(imported.key_pool() == view.key_pool());
  CHECK_EQ(layer1.num_free_blocks(), free_before - 1);
}


// ------------------------------------------------------------ KV cache manager

TEST_CASE("kv cache manager: append_slots grows page tables by ceil((n+k)/16) - ceil(n/16)") {
  Group g(24, 24 * Group::kPage);
  auto kv = manager_over(g.group);
  CHECK_EQ(kv->num_layers(), 3);
  CHECK_EQ(kv->block_size(), 16);
  kv->set_radix_cache_enabled(false);  // the shared-arena setup's call (qwen2.cpp:1137)
  CHECK_THROWS_AS(kv->set_radix_cache_enabled(true), std::invalid_argument);
  const base::RequestId a = kv->register_request();
  CHECK(kv->is_valid_request(a));
  CHECK(kv->append_slots(a, 41));  // 3 pages
  CHECK_EQ(kv->get_context_len(a), 41);
  CHECK_EQ(kv->num_tokens_in_last_block(a), 9);
  for (int l = 0; l < 3; ++l) CHECK(kv->get_block_ids(a, l) == (std::vector<int32_t>{0, 6, 12}));
  CHECK(kv->append_slots(a, 7));  // 48 tokens: still 3 pages
  CHECK_EQ(kv->get_block_ids(a, 0).size(), 3u);
  CHECK_EQ(kv->num_tokens_in_last_block(a), 16);
  CHECK(kv->append_slot(a));      // 49: a fourth page
  CHECK(kv->get_block_ids(a, 2) == (std::vector<int32_t>{0, 6, 12, 18}));
  CHECK(kv->get_slot(a, 1, 17) == std::make_pair(6, 1));
  CHECK(kv->current_slot(a, 0) == std::make_pair(18, 0));
  CHECK(!kv->append_slots(a, 0));
  CHECK(!kv->append_slots(a, -3));
  // each layer's K plane of block b is plane b + 2l of the page-major arena
  const auto p0 = kv->allocator(0).get_block_payload_ptrs(6);
  const auto p2 = kv->allocator(2).get_block_payload_ptrs(6);
  CHECK_EQ(static_cast<char*>(p2.key) - static_cast<char*>(p0.key), 4 * 4096);
  const base::RequestId b = kv->register_request();
  CHECK(kv->append_slots(b, 16));
  CHECK(kv->build_seq_lens({a, b}) == (std::vector<int32_t>{49, 16}));
  const auto tables = kv->build_block_tables({a, b}, 1);
  CHECK_EQ(tables.second, 4);
  CHECK(tables.first == (std::vector<int32_t>{0, 6, 12, 18, 24, -1, -1, -1}));
  CHECK(kv->build_slot_mapping({a, b}, 0) == (std::vector<int32_t>{18 * 16 + 0, 24 * 16 + 15}));
  CHECK_EQ(kv->num_active_requests(), 2);
  kv->free_request(a);
  kv->free_request(b);
  CHECK_EQ(kv->num_active_requests(), 0);
  CHECK_EQ(g.owner->lease_count(), 0u);  // every Chunk back at the owner
}

TEST_CASE("kv cache manager: commit_kv only moves forward within the appended slots") {
  Group g(24, 24 * Group::kPage);
  auto kv = manager_over(g.group);
  const base::RequestId a = kv->register_request();
  CHECK(kv->append_slots(a, 41));
  CHECK_EQ(kv->kv_committed_tokens(a), 0);
  CHECK(!kv->commit_kv(a, 42));
  CHECK(kv->commit_kv(a, 41));
  CHECK_EQ(kv->kv_committed_tokens(a), 41);
  CHECK(!kv->commit_kv(a, 40));
  CHECK(kv->commit_kv(a, 41));
  kv->free_request(a);
  CHECK(!kv->commit_kv(a, 41));  // stale id
}

TEST_CASE("kv cache manager: stale ids never alias a reused slot") {
  Group g(24, 24 * Group::kPage);
  auto kv = manager_over(g.group);
  const base::RequestId a = kv->register_request();
  kv->free_request(a);
  const base::RequestId b = kv->register_request();  // same slot, next generation
  CHECK(a != b);
  CHECK(!kv->is_valid_request(a));
  CHECK(kv->is_valid_request(b));
  CHECK_THROWS_AS(kv->free_request(a), std::invalid_argument);
  CHECK_THROWS_AS(kv->get_block_ids(a, 0), std::invalid_argument);
  CHECK_THROWS_AS(kv->get_block_ids(b, 3), std::out_of_range);
  CHECK(!kv->is_valid_request(-1));
  CHECK(!kv->is_valid_request(12345));
  kv->free_request(b);
}

TEST_CASE("kv cache manager: exhaustion holds nothing new") {
  Group g(6, 3 * Group::kPage);  // limit: 3 pages
  auto kv = manager_over(g.group);
  const base::RequestId a = kv->register_request();
  CHECK(kv->append_slots(a, 32));  // 2 pages
  CHECK(!kv->append_slots(a, 33));  // would need 3 more
  CHECK_EQ(kv->get_context_len(a), 32);
  for (int l = 0; l < 3; ++l) CHECK_EQ(kv->get_block_ids(a, l).size(), 2u);
  CHECK(kv->append_slots(a, 16));  // the third page still fits
  kv->free_request(a);
  CHECK_EQ(g.owner->lease_count(), 0u);
  std::vector<std::unique_ptr<base::BlockAllocator>> none;
  CHECK_THROWS_AS(base::KVCacheManager(16, 3, std::move(none)), std::invalid_argument);
}

TEST_CASE("block allocator: local pools, FIFO reuse and payload copy with scales (host)") {
  base::BlockAllocator plain(4, 16, 2, 8, base::DataType::kDataTypeBf16, base::DeviceType::kDeviceCPU);
  CHECK(!plain.uses_shared_arena());
  CHECK_EQ(plain.num_total_blocks(), 4);
  CHECK_EQ(plain.key_value_bytes_per_block(), 16u * 2 * 8 * 2);
  CHECK_EQ(plain.scale_bytes_per_block(), 0u);
  const int a = plain.allocate(), b = plain.allocate();
  CHECK_EQ(a, 0);
  CHECK_EQ(b, 1);
  CHECK_EQ(plain.num_free_blocks(), 2);
  auto pa = plain.get_block_payload_ptrs(a), pb = plain.get_block_payload_ptrs(b);
  for (size_t i = 0; i < pa.key_value_bytes; ++i) {
    static_cast<uint8_t*>(pa.key)[i] = static_cast<uint8_t>(i * 7 + 1);
    static_cast<uint8_t*>(pa.value)[i] = static_cast<uint8_t>(i * 5 + 3);
  }
  plain.copy_block_payload(a, b);
  CHECK(std::memcmp(pa.key, pb.key, pa.key_value_bytes) == 0);
  CHECK(std::memcmp(pa.value, pb.value, pa.key_value_bytes) == 0);
  CHECK_EQ(plain.payload_copy_bytes(), 2 * pa.key_value_bytes);
  CHECK_THROWS_AS(plain.copy_block_payload(a, a), std::logic_error);
  CHECK_THROWS_AS(plain.copy_block_payload(a, 2), std::logic_error);  // block 2 is free
  plain.free(a);
  CHECK_EQ(plain.allocate(), 2);  // FIFO: 2 and 3 were queued before 0
  // FP8 pools need a GPU device (kv_cache_format.h rule)
  CHECK_THROWS_AS(base::BlockAllocator(4, 16, 2, 8, base::DataType::kDataTypeBf16,
                                       base::DeviceType::kDeviceCPU,
                                       base::BlockStorageMode::kFp8E4M3PerTokenHead),
                  std::invalid_argument);
  CHECK_THROWS_AS(base::BlockAllocator(0, 16, 2, 8, base::DataType::kDataTypeBf16,
                                       base::DeviceType::kDeviceCPU),
                  std::invalid_argument);
}

// ------------------------------------------------------------ copy_shared_kv in the reference's order

namespace {
serving::SharedKVPrefillResult prefill_result(uint64_t epoch, const std::vector<int32_t>& ids) {
  serving::SharedKVPrefillResult r;
  r.shared_arena_epoch = epoch;
  r.client_request_id.value = "req";
  r.handoff_id.value = 3;
  r.prompt_tokens.assign(40, 1);
  r.computed_tokens = 40;  // 3 pages
  r.src_pool = pool3();
  for (int l = 0; l < 3; ++l) r.layers.push_back({l, ids});
  return r;
}
}  // namespace

TEST_CASE("copy_shared_kv order: rejected inputs reserve nothing; a refused copy releases the pages") {
  Group g(24, 24 * Group::kPage);  // metadata-only group: no device
  auto kv = manager_over(g.group);
  serving::DecodeKVReservation res;
  const std::vector<int32_t> src{60, 66, 72};
  auto bad = prefill_result(5, src);  // the arena's epoch is 9
  CHECK_THROWS_AS(serving::CopySharedKVToDecode(kv.get(), pool3(), bad, nullptr, &res), std::runtime_error);
  bad = prefill_result(9, src);
  bad.layers.pop_back();
  CHECK_THROWS_AS(serving::CopySharedKVToDecode(kv.get(), pool3(), bad, nullptr, &res), std::runtime_error);
  bad = prefill_result(9, src);
  bad.layers[1].layer_idx = 2;
  CHECK_THROWS_AS(serving::CopySharedKVToDecode(kv.get(), pool3(), bad, nullptr, &res), std::runtime_error);
  bad = prefill_result(9, {60, 66, 73});  // not a page id
  CHECK_THROWS_AS(serving::CopySharedKVToDecode(kv.get(), pool3(), bad, nullptr, &res), std::runtime_error);
  bad = prefill_result(9, src);
  bad.layers[2].src_block_ids = {60, 72, 66};  // layers disagree
  CHECK_THROWS_AS(serving::CopySharedKVToDecode(kv.get(), pool3(), bad, nullptr, &res), std::runtime_error);
  bad = prefill_result(9, {60, 66, 24 * 6});  // past the arena
  CHECK_THROWS_AS(serving::CopySharedKVToDecode(kv.get(), pool3(), bad, nullptr, &res), std::runtime_error);
  CHECK_EQ(kv->num_active_requests(), 0);
  CHECK(!res.valid());
  // Valid input: the reservation is made, then the copy is refused (this
  // group has no GPU mapping), so the reservation is released again.
  try {
    serving::CopySharedKVToDecode(kv.get(), pool3(), prefill_result(9, src), nullptr, &res);
    CHECK(false);
  } catch (const std::runtime_error& e) {
    CHECK(std::string(e.what()).find("PD copy failed") != std::string::npos);
  }
  CHECK(!res.valid());
  CHECK_EQ(kv->num_active_requests(), 0);
  g.group->collect();
  CHECK_EQ(g.owner->lease_count(), 0u);
  CHECK_THROWS_AS(serving::CopySharedKVToDecode(nullptr, pool3(), prefill_result(9, src), nullptr, &res),
                  std::invalid_argument);
}

// ------------------------------------------------------------ split-PD admission
// The reference's cases (test/test_split_pd_admission.cpp:4-34), restated.

TEST_CASE("split PD admission: long outputs cannot consume short slots or tokens") {
  serving::SplitPDAdmission admission({2, 1}, {512, 4096});
  admission.acquire(1, 4096);
  CHECK(!admission.can_acquire(1, 16));
  CHECK(admission.can_acquire(0, 256));
  admission.acquire(0, 256);
  admission.acquire(0, 256);
  CHECK(!admission.can_acquire(0, 16));  // both short slots taken
  admission.release(0, 256);
  CHECK(admission.can_acquire(0, 256));
  CHECK_EQ(admission.used(1), 4096);
}

TEST_CASE("split PD admission: future output rounds to whole pages") {
  CHECK_EQ(serving::SplitPDAdmission::charge(17, 16, 16), 48);
  CHECK_EQ(serving::SplitPDAdmission::charge(16, 0, 16), 16);
  CHECK_EQ(serving::SplitPDAdmission::charge(5040, 1, 16), 5056);
  serving::SplitPDAdmission admission({4, 2}, {32, 64});
  CHECK(!admission.fits_request(0, 48));
  CHECK(admission.fits_request(1, 48));
  CHECK(!admission.fits_request(1, 0));
}

TEST_CASE("split PD admission: reclaim, and reject a double release") {
  serving::SplitPDAdmission admission({1, 1}, {128, 128});
  for (int round = 0; round < 10; ++round) {
    admission.acquire(0, 128);
    CHECK_THROWS_AS(admission.acquire(0, 1), std::logic_error);
    admission.release(0, 128);
  }
  CHECK_EQ(admission.active(0), 0);
  CHECK_EQ(admission.used(0), 0);
  CHECK_THROWS_AS(admission.release(0, 128), std::logic_error);
  CHECK_THROWS_AS(admission.acquire(2, 1), std::out_of_range);
}

TEST_CASE("block allocator: local pool view binds the pools without owning the allocation queue") {
  // test_kv_pool_view.cpp:5-25 as written: a local CPU pool of 4 FP32 blocks
  base::BlockAllocator owner(4, 16, 2, 8, base::DataType::kDataTypeFp32, base::DeviceType::kDeviceCPU);
  const int32_t free_before = owner.num_free_blocks();
  const base::KVPoolView view = owner.pool_view();
  REQUIRE(view.valid());
  CHECK(view.device_type() == base::DeviceType::kDeviceCPU);
  CHECK(view.key_pool() == owner.get_block_payload_ptrs(0).key);
  CHECK(view.value_pool() == owner.get_block_payload_ptrs(0).value);
  CHECK_EQ(owner.num_free_blocks(), free_before);
  const int32_t block = owner.allocate();
  REQUIRE(block >= 0);
  CHECK_EQ(owner.num_free_blocks(), free_before - 1);
  const base::KVPoolView imported = view;  // copying the descriptor owns nothing
  CHECK(imported.key_pool() == view.key_pool());
  CHECK_EQ(owner.num_free_blocks(), free_before - 1);
  owner.free(block);
  CHECK_EQ(owner.num_free_blocks(), free_before);
}

TEST_CASE("kv cache manager: randomized requests keep exact block accounting (model check)") {
  // Local host pools of 20 blocks per layer; a model of each live request's
  // token count predicts every outcome: append succeeds iff every layer has
  // ceil((n+k)/16) - ceil(n/16) free blocks, and a refusal changes nothing.
  constexpr int kLayers = 3, kBlocks = 20, kB = 16;
  std::vector<std::unique_ptr<base::BlockAllocator>> pools;
  for (int l = 0; l < kLayers; ++l)
    pools.push_back(std::make_unique<base::BlockAllocator>(kBlocks, kB, 1, 8, base::DataType::kDataTypeBf16,
                                                           base::DeviceType::kDeviceCPU));
  base::KVCacheManager kv(kB, kLayers, std::move(pools));
  struct Live { int32_t tokens = 0, committed = 0; };
  std::vector<std::pair<base::RequestId, Live>> live;
  std::vector<base::RequestId> dead;
  std::mt19937_64 rng(77);
  auto blocks = [](int32_t t) { return (t + kB - 1) / kB; };
  int appended_ok = 0, refused = 0;
  for (int step = 0; step < 4000; ++step) {
    const int op = static_cast<int>(rng() % 10);
    if (op == 0 || live.empty()) {
      live.push_back({kv.register_request(), {}});
    } else if (op <= 5) {
      auto& [id, m] = live[rng() % live.size()];
      const int32_t k = 1 + static_cast<int32_t>(rng() % 60);
      int32_t used = 0;
      for (auto& e : live) used += blocks(e.second.tokens);
      const bool fits = blocks(m.tokens + k) - blocks(m.tokens) <= kBlocks - used;
      const bool ok = kv.append_slots(id, k);
      CHECK_EQ(ok, fits);
      if (ok) m.tokens += k, ++appended_ok;
      else ++refused;
    } else if (op <= 7) {
      auto& [id, m] = live[rng() % live.size()];
      const int32_t t = static_cast<int32_t>(rng() % (m.tokens + 2));
      const bool want = t >= m.committed && t <= m.tokens;
      CHECK_EQ(kv.commit_kv(id, t), want);
      if (want) m.committed = t;
    } else {
      const size_t i = rng() % live.size();
      kv.free_request(live[i].first);
      dead.push_back(live[i].first);
      live.erase(live.begin() + static_cast<long>(i));
    }
    // invariants
    int32_t used = 0;
    for (auto& [id, m] : live) {
      used += blocks(m.tokens);
      CHECK(kv.is_valid_request(id));
      CHECK_EQ(kv.get_context_len(id), m.tokens);
      CHECK_EQ(kv.kv_committed_tokens(id), m.committed);
    }
    for (int l = 0; l < kLayers; ++l) {
      CHECK_EQ(kv.num_free_blocks(l), kBlocks - used);
      std::vector<char> seen(kBlocks, 0);
      for (auto& [id, m] : live) {
        const auto& ids = kv.get_block_ids(id, l);
        CHECK_EQ(static_cast<int32_t>(ids.size()), blocks(m.tokens));
        for (int32_t b : ids) {
          CHECK(b >= 0 && b < kBlocks);
          if (b >= 0 && b < kBlocks) CHECK(!seen[b]++);  // no block in two tables
        }
      }
    }
    for (base::RequestId d : dead) CHECK(!kv.is_valid_request(d));
    CHECK_EQ(kv.num_active_requests(), static_cast<int32_t>(live.size()));
  }
  CHECK(appended_ok > 100);
  CHECK(refused > 100);
  for (auto& [id, m] : live) kv.free_request(id);
  for (int l = 0; l < kLayers; ++l) CHECK_EQ(kv.num_free_blocks(l), kBlocks);
}

TEST_CASE("kv cache manager over a shared page group: randomized requests keep page-major tables (model check)") {
  // 30-page arena, this model limited to 18 pages, Chunks of 3 pages. Every
  // live request's table is identical in all layers, holds page ids only, and
  // no page serves two requests; leases cover the held pages and respect the
  // limit; a refused append changes nothing; freeing everything returns every
  // Chunk to the owner.
  Group g(30, 18 * Group::kPage);
  auto kv = manager_over(g.group);
  constexpr int B = 16;
  auto pages_for = [](int32_t t) { return (t + B - 1) / B; };
  std::vector<std::pair<base::RequestId, int32_t>> live;
  std::mt19937_64 rng(5);
  int grew = 0, refused = 0;
  for (int step = 0; step < 3000; ++step) {
    const int op = static_cast<int>(rng() % 10);
    if (op == 0 || live.empty()) {
      live.push_back({kv->register_request(), 0});
    } else if (op <= 6) {
      auto& [id, tokens] = live[rng() % live.size()];
      const int32_t k = 1 + static_cast<int32_t>(rng() % 70);
      std::vector<std::vector<int32_t>> before;
      for (int l = 0; l < 3; ++l) before.push_back(kv->get_block_ids(id, l));
      const size_t leased = g.group->leased_bytes();
      if (kv->append_slots(id, k)) {
        tokens += k;
        ++grew;
      } else {
        ++refused;
        for (int l = 0; l < 3; ++l) CHECK(kv->get_block_ids(id, l) == before[l]);
        CHECK_EQ(kv->get_context_len(id), tokens);
        CHECK(g.group->leased_bytes() <= std::max<size_t>(leased, 18 * Group::kPage));
      }
    } else {
      const size_t i = rng() % live.size();
      kv->free_request(live[i].first);
      live.erase(live.begin() + static_cast<long>(i));
    }
    std::vector<char> used(30, 0);
    int held = 0;
    for (auto& [id, tokens] : live) {
      const auto& ids0 = kv->get_block_ids(id, 0);
      CHECK_EQ(static_cast<int>(ids0.size()), pages_for(tokens));
      for (int l = 1; l < 3; ++l) CHECK(kv->get_block_ids(id, l) == ids0);
      for (int32_t b : ids0) {
        CHECK(b >= 0 && b % 6 == 0 && b / 6 < 30);
        if (b >= 0 && b % 6 == 0 && b / 6 < 30) CHECK(!used[b / 6]++);
      }
      held += static_cast<int>(ids0.size());
    }
    CHECK(g.group->leased_bytes() <= 18 * Group::kPage);
    CHECK(g.group->leased_bytes() >= static_cast<size_t>(held) * Group::kPage);
  }
  CHECK(grew > 200);
  CHECK(refused > 20);
  for (auto& [id, tokens] : live) kv->free_request(id);
  CHECK_EQ(kv->num_active_requests(), 0);
  CHECK_EQ(g.owner->lease_count(), 0u);
}

MINITEST_MAIN()
