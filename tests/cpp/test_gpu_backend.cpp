// GPU tests of the C++ drop-in API: the HIP TransferBackend (one kernel per
// BoundTransfer) and the shared-arena handoff connector. Scenarios follow the
// reference's test/test_page_migration_cuda.cpp:13-108 (byte fills, pending /
// failed-safe states) and test/test_serving/test_pd_handoff.cpp:429-564
// (pattern-filled pages compared element-wise after the handoff).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <numeric>
#include <vector>

#include "cache/page_migration.h"
#include "cache/transfer_plan.h"
#include "minitest.h"
#include "pbe_handoff.h"
#include "base/shared_kv_arena.h"
#include "serving/decode_kv_reservation.h"
#include "serving/pd_handoff.h"

using namespace cache;

#define HIP_OK(x) REQUIRE((x) == hipSuccess)

namespace {

PageSchema schema_of(bool fp8, int32_t layers = 2) {
  PageSchema s;
  MakeKVPageSchema(1, layers, 16, 2, 64,
                   base::MakeKVCacheStorageSpec(base::DataType::kDataTypeBf16,
                                                fp8 ? base::BlockStorageMode::kFp8E4M3PerTokenHead
                                                    : base::BlockStorageMode::kPlain),
                   &s);
  return s;
}

std::vector<size_t> iota_order(size_t n) {
  std::vector<size_t> o(n);
  std::iota(o.begin(), o.end(), 0);
  return o;
}

BackendResult wait_done(TransferBackend& b, MigrationId id) {
  BackendResult r = BackendResult::kPending;
  for (int i = 0; i < 2000000 && r == BackendResult::kPending; ++i) r = b.poll(id);
  return r;
}

}  // namespace

TEST_CASE("hip backend: device to device, to host and back to device") {
  for (bool fp8 : {false, true}) {
    const auto s = schema_of(fp8);
    LayoutDescriptor l;
    REQUIRE(MakePackedLayout(s, "packed", 7, iota_order(s.components.size()), {}, &l));
    const size_t n = l.total_bytes;
    uint8_t *d_src = nullptr, *d_dst = nullptr, *d_back = nullptr, *h_pin = nullptr;
    HIP_OK(hipMalloc(&d_src, n));
    HIP_OK(hipMalloc(&d_dst, n));
    HIP_OK(hipMalloc(&d_back, n));
    HIP_OK(hipHostMalloc(&h_pin, n, hipHostMallocDefault));
    std::vector<uint8_t> pattern(n);
    for (size_t i = 0; i < n; ++i) pattern[i] = static_cast<uint8_t>(i * 37u + 11u);
    HIP_OK(hipMemcpy(d_src, pattern.data(), n, hipMemcpyHostToDevice));
    HIP_OK(hipMemset(d_dst, 0x21, n));
    HIP_OK(hipMemset(d_back, 0x21, n));
    std::memset(h_pin, 0x21, n);

    TransferPlanner planner;
    TransferPlan plan;
    REQUIRE(planner.plan(s, s, &plan));
    auto backend = MakeHipTransferBackend(2, 0);
    CHECK(backend->supports(base::DeviceType::kDeviceHIP));
    CHECK(!backend->supports(base::DeviceType::kDeviceCPU));

    BoundTransfer d2d, d2h, h2d;
    REQUIRE(BoundTransfer::Bind(plan, s, {d_src, n, &l}, {d_dst, n, &l}, &d2d));
    REQUIRE(BoundTransfer::Bind(plan, s, {d_src, n, &l}, {h_pin, n, &l}, &d2h));
    REQUIRE(BoundTransfer::Bind(plan, s, {h_pin, n, &l}, {d_back, n, &l}, &h2d));

    CHECK(backend->submit(1, TransferDirection::kGpuToGpu, d2d) == BackendResult::kPending);
    CHECK(backend->submit(1, TransferDirection::kGpuToGpu, d2d) == BackendResult::kUnknown);  // live id
    CHECK(backend->submit(2, TransferDirection::kToHost, d2h) == BackendResult::kPending);
    CHECK(backend->submit(3, TransferDirection::kToHost, d2h) == BackendResult::kFailedSafe);  // no slot
    CHECK(wait_done(*backend, 1) == BackendResult::kSucceeded);
    CHECK(backend->drain(2) == BackendResult::kSucceeded);
    backend->release(1);
    backend->release(2);
    CHECK(std::memcmp(h_pin, pattern.data(), n) == 0);
    std::vector<uint8_t> got(n);
    HIP_OK(hipMemcpy(got.data(), d_dst, n, hipMemcpyDeviceToHost));
    CHECK(got == pattern);

    CHECK(backend->submit(4, TransferDirection::kToGpu, h2d) == BackendResult::kPending);
    CHECK(backend->drain(4) == BackendResult::kSucceeded);
    backend->release(4);
    HIP_OK(hipMemcpy(got.data(), d_back, n, hipMemcpyDeviceToHost));
    CHECK(got == pattern);

    // Wrong-direction or pageable endpoints are refused before any write.
    std::vector<uint8_t> pageable(n, 0x21);
    BoundTransfer bad;
    REQUIRE(BoundTransfer::Bind(plan, s, {d_src, n, &l}, {pageable.data(), n, &l}, &bad));
    CHECK(backend->submit(5, TransferDirection::kToHost, bad) == BackendResult::kFailedSafe);
    CHECK(backend->submit(6, TransferDirection::kToGpu, d2d) == BackendResult::kFailedSafe);
    CHECK(backend->submit(7, TransferDirection::kToHost, d2d) == BackendResult::kFailedSafe);
    backend->release(5);  // never submitted to a stream: no-op
    CHECK(std::all_of(pageable.begin(), pageable.end(), [](uint8_t b) { return b == 0x21; }));
    (void)hipFree(d_src);
    (void)hipFree(d_dst);
    (void)hipFree(d_back);
    (void)hipHostFree(h_pin);
  }
}

TEST_CASE("hip backend: a dependency event orders the copy after the producer") {
  const auto s = schema_of(false);
  LayoutDescriptor l;
  REQUIRE(MakePackedLayout(s, "packed", 7, iota_order(s.components.size()), {}, &l));
  const size_t n = l.total_bytes;
  uint8_t *d_src = nullptr, *d_dst = nullptr;
  HIP_OK(hipMalloc(&d_src, n));
  HIP_OK(hipMalloc(&d_dst, n));
  hipStream_t producer;
  hipEvent_t produced;
  HIP_OK(hipStreamCreateWithFlags(&producer, hipStreamNonBlocking));
  HIP_OK(hipEventCreateWithFlags(&produced, hipEventDisableTiming));
  HIP_OK(hipMemsetAsync(d_src, 0x5c, n, producer));  // the "prefill" writes the source
  HIP_OK(hipEventRecord(produced, producer));
  TransferPlanner planner;
  TransferPlan plan;
  REQUIRE(planner.plan(s, s, &plan));
  BoundTransfer t;
  REQUIRE(BoundTransfer::Bind(plan, s, {d_src, n, &l}, {d_dst, n, &l}, &t));
  {
    auto backend = MakeHipTransferBackend(1, 0, produced);
    CHECK(backend->submit(1, TransferDirection::kGpuToGpu, t) == BackendResult::kPending);
    CHECK(backend->drain(1) == BackendResult::kSucceeded);
    backend->release(1);
  }
  std::vector<uint8_t> got(n);
  HIP_OK(hipMemcpy(got.data(), d_dst, n, hipMemcpyDeviceToHost));
  CHECK(std::all_of(got.begin(), got.end(), [](uint8_t b) { return b == 0x5c; }));
  (void)hipEventDestroy(produced);
  (void)hipStreamDestroy(producer);
  (void)hipFree(d_src);
  (void)hipFree(d_dst);
}

namespace {
serving::KVBlockManifest manifest_for(int32_t layers, const std::vector<int32_t>& src,
                                      const std::vector<int32_t>& dst) {
  serving::KVBlockManifest m;
  m.client_request_id.value = "req";
  m.handoff_id.value = 1;
  m.prompt_tokens = static_cast<int32_t>(src.size()) * 16;
  m.computed_tokens = m.prompt_tokens - 3;
  m.src_pool = {0, layers, 16, 2, 64, base::DataType::kDataTypeBf16, base::BlockStorageMode::kPlain};
  m.dst_pool = m.src_pool;
  for (int32_t l = 0; l < layers; ++l) m.layer_mappings.push_back({l, src, dst});
  return m;
}
}  // namespace

TEST_CASE("shared-arena connector: page-major pages arrive intact, errors write nothing") {
  const int32_t layers = 3;
  const uint64_t half = 16 * 2 * 64 * 2, page = 2 * layers * half;
  const uint64_t pages = 40, bytes = pages * page;
  pbe_arena* arena = nullptr;
  REQUIRE(pbe_arena_create(0, bytes, 0, 123, &arena) == PBE_OK);
  serving::SharedArenaBinding bind;
  REQUIRE(pbe_arena_get_view(arena, &bind.view) == PBE_OK);
  bind.epoch = 123;
  bind.device = 0;
  // Byte (2l+plane)*half of page p holds p*3 + 64*plane + l (the page-major
  // pattern of demo/shared_kv_reuse_probe.cpp:76-83).
  std::vector<uint8_t> host(bytes);
  for (uint64_t p = 0; p < pages; ++p)
    for (int l = 0; l < layers; ++l)
      for (int plane = 0; plane < 2; ++plane)
        std::memset(host.data() + p * page + (2 * l + plane) * half,
                    static_cast<int>((p * 3 + 64 * plane + l) & 0xff), half);
  HIP_OK(hipMemcpy(bind.view.base[0], host.data(), bytes, hipMemcpyHostToDevice));
  const int32_t st = 2 * layers;
  const std::vector<int32_t> src = {2 * st, 3 * st, 4 * st, 9 * st, 10 * st};
  const std::vector<int32_t> dst = {20 * st, 21 * st, 30 * st, 31 * st, 5 * st};
  {
    serving::SharedArenaKVTransferConnector conn(bind);
    serving::HandoffId h;
    REQUIRE(conn.submit(manifest_for(layers, src, dst), &h));
    CHECK(conn.drain(h).ok());
    CHECK_EQ(conn.copied_bytes(), src.size() * page);
    conn.release(h);
    CHECK(conn.poll(h).state == serving::KVTransferState::kFailed);  // forgotten

    // Errors: stale epoch, non-page-major layers, ids outside the arena.
    serving::HandoffId bad;
    CHECK(!conn.submit_from(124, manifest_for(layers, src, dst), &bad));
    CHECK(conn.poll(bad).state == serving::KVTransferState::kFailed);
    auto skew = manifest_for(layers, src, dst);
    skew.layer_mappings[1].src_block_ids[0] += st;
    CHECK(!conn.submit(skew, &bad));
    auto out_of_arena = manifest_for(layers, src, {20 * st, 21 * st, 30 * st, 31 * st, 40 * st});
    CHECK(!conn.submit(out_of_arena, &bad));
    auto unaligned = manifest_for(layers, src, {20 * st, 21 * st, 30 * st, 31 * st, 5 * st + 1});
    CHECK(!conn.submit(unaligned, &bad));
    auto self = manifest_for(layers, src, src);
    CHECK(!conn.submit(self, &bad));
  }
  std::vector<uint8_t> got(bytes);
  HIP_OK(hipMemcpy(got.data(), bind.view.base[0], bytes, hipMemcpyDeviceToHost));
  std::vector<uint8_t> want = host;
  for (size_t i = 0; i < src.size(); ++i)
    std::memcpy(want.data() + (uint64_t)dst[i] / st * page, host.data() + (uint64_t)src[i] / st * page, page);
  CHECK(got == want);
  CHECK(pbe_arena_destroy(arena) == PBE_OK);
}

TEST_CASE("generic plan form: InProcKVBlockCopyConnector equals the run copy, BF16 and FP8 pools") {
  for (bool fp8 : {false, true}) {
    const int layers = 4;
    const uint64_t elem = fp8 ? 1 : 2;
    const uint64_t half = 16 * 2 * 64 * elem, page = 2 * layers * half, pages = 24;
    const uint64_t bytes = pages * page;
    const uint64_t scale_page = 2 * layers * 16 * 2 * 4;
    uint8_t *arena = nullptr, *scales = nullptr;
    HIP_OK(hipMalloc(&arena, bytes));
    HIP_OK(hipMalloc(&scales, pages * scale_page));
    std::vector<uint8_t> host(bytes), host_sc(pages * scale_page);
    for (size_t i = 0; i < host.size(); ++i) host[i] = static_cast<uint8_t>(i * 131u + 17u);
    for (size_t i = 0; i < host_sc.size(); ++i) host_sc[i] = static_cast<uint8_t>(i * 7u + 3u);
    HIP_OK(hipMemcpy(arena, host.data(), bytes, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(scales, host_sc.data(), host_sc.size(), hipMemcpyHostToDevice));
    serving::ArenaKVPool pool;
    pool.view.bytes = bytes;
    pool.view.segment_bytes = bytes;
    pool.view.nseg = 1;
    pool.view.base[0] = arena;
    pool.pool = {0, layers, 16, 2, 64, base::DataType::kDataTypeBf16,
                 fp8 ? base::BlockStorageMode::kFp8E4M3PerTokenHead : base::BlockStorageMode::kPlain};
    if (fp8) {
      pool.scales = scales;
      pool.scale_bytes = pages * scale_page;
    }
    const int st = 2 * layers;
    const std::vector<int32_t> src = {1 * st, 2 * st, 3 * st, 7 * st, 9 * st};
    const std::vector<int32_t> dst = {10 * st, 11 * st, 20 * st, 21 * st, 22 * st};
    serving::KVBlockManifest m;
    m.client_request_id.value = "g";
    m.handoff_id.value = 3;
    m.prompt_tokens = m.computed_tokens = 80;
    m.src_pool = m.dst_pool = pool.pool;
    for (int l = 0; l < layers; ++l) m.layer_mappings.push_back({l, src, dst});
    {
      serving::InProcKVBlockCopyConnector conn(pool, pool, 0);
      serving::HandoffId h;
      REQUIRE(conn.submit(m, &h));
      CHECK(conn.drain(h).ok());
      CHECK_EQ(conn.last_op_count(), src.size() * 2 * layers * (fp8 ? 2 : 1));
      conn.release(h);
    }
    std::vector<uint8_t> got(bytes), got_sc(host_sc.size());
    HIP_OK(hipMemcpy(got.data(), arena, bytes, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(got_sc.data(), scales, got_sc.size(), hipMemcpyDeviceToHost));
    std::vector<uint8_t> want = host, want_sc = host_sc;
    for (size_t i = 0; i < src.size(); ++i) {
      std::memcpy(want.data() + dst[i] / st * page, host.data() + src[i] / st * page, page);
      if (fp8)
        std::memcpy(want_sc.data() + dst[i] / st * scale_page, host_sc.data() + src[i] / st * scale_page,
                    scale_page);
    }
    CHECK(got == want);
    CHECK(got_sc == want_sc);
    (void)hipFree(arena);
    (void)hipFree(scales);
  }
}

TEST_CASE("end to end: prefill pages -> decode reservation -> connector copy -> fenced retire") {
  // Qwen2.5-0.5B geometry: 24 layers, 2 KV heads x 64, 16-token pages (192 KiB).
  const int layers = 24;
  const uint64_t half = 16 * 2 * 64 * 2, page = 2 * layers * half;
  const uint64_t arena_bytes = 64 * page;
  pbe_arena* arena = nullptr;
  REQUIRE(pbe_arena_create(0, arena_bytes, 16 * page, 4242, &arena) == PBE_OK);  // 4 segments
  pbe_arena_view view{};
  REQUIRE(pbe_arena_get_view(arena, &view) == PBE_OK);
  auto owner = std::make_shared<base::LocalChunkOwner>(arena_bytes, 4242);
  owner->register_model("prefill", 24 * page);
  owner->register_model("decode", 40 * page);
  void* p_stream = nullptr;
  void* d_stream = nullptr;
  REQUIRE(pbe_stream_create(0, &p_stream) == PBE_OK);
  REQUIRE(pbe_stream_create(0, &d_stream) == PBE_OK);
  {
    auto p_client = std::make_shared<base::SharedKVArenaClient>(owner, view, "prefill", 24 * page, 0);
    auto d_client = std::make_shared<base::SharedKVArenaClient>(owner, view, "decode", 40 * page, 0);
    base::SharedKVPageGroup p_pages(p_client, layers, half, 2 * 1024 * 1024, p_stream);  // 11-page Chunks
    base::SharedKVPageGroup d_pages(d_client, layers, half, 2 * 1024 * 1024, d_stream);
    // prefill: a 41-token prompt = 3 pages, every layer
    std::vector<int32_t> src;
    for (int i = 0; i < 3; ++i) src.push_back(p_pages.allocate(0));
    for (int l = 1; l < layers; ++l)
      for (int i = 0; i < 3; ++i) CHECK_EQ(p_pages.allocate(l), src[i]);
    // write the prefill KV: byte = page index * 3 + 64 * plane + layer
    std::vector<uint8_t> host(page);
    for (size_t i = 0; i < src.size(); ++i) {
      for (int l = 0; l < layers; ++l)
        for (int plane = 0; plane < 2; ++plane)
          std::memset(host.data() + (2 * l + plane) * half, static_cast<int>((i * 3 + 64 * plane + l) & 0xff), half);
      const uint64_t off = static_cast<uint64_t>(src[i]) * half;
      uint8_t* dst = static_cast<uint8_t*>(view.base[off / view.segment_bytes]) + off % view.segment_bytes;
      HIP_OK(hipMemcpy(dst, host.data(), page, hipMemcpyHostToDevice));
    }
    // decode: reserve destination pages and build the manifest
    serving::KVPoolDescriptor pool{0, layers, 16, 2, 64, base::DataType::kDataTypeBf16,
                                   base::BlockStorageMode::kPlain};
    serving::DecodeKVReservationManager reservations(&d_pages, pool);
    serving::DecodeKVReservationRequest req;
    req.client_request_id.value = "req-41";
    req.handoff_id.value = 1;
    req.prompt_tokens = 41;
    req.computed_tokens = 41;
    req.src_pool = pool;
    req.src_block_ids_per_layer.assign(layers, src);
    serving::DecodeKVReservation res;
    serving::KVBlockManifest manifest;
    REQUIRE(reservations.reserve(req, &res, &manifest));
    serving::SharedArenaBinding binding{view, 4242, 0};
    serving::SharedArenaKVTransferConnector conn(binding, d_stream);
    serving::HandoffId h;
    REQUIRE(conn.submit_from(p_client->epoch(), manifest, &h));
    CHECK(conn.drain(h).ok());
    CHECK_EQ(conn.copied_bytes(), 3 * page);
    // verify destination pages
    const auto& dst_ids = manifest.layer_mappings[0].dst_block_ids;
    for (size_t i = 0; i < dst_ids.size(); ++i) {
      const uint64_t off = static_cast<uint64_t>(dst_ids[i]) * half;
      const uint8_t* d = static_cast<uint8_t*>(view.base[off / view.segment_bytes]) + off % view.segment_bytes;
      HIP_OK(hipMemcpy(host.data(), d, page, hipMemcpyDeviceToHost));
      bool ok = true;
      for (int l = 0; l < layers && ok; ++l)
        for (int plane = 0; plane < 2 && ok; ++plane)
          ok = std::all_of(host.begin() + (2 * l + plane) * half, host.begin() + (2 * l + plane + 1) * half,
                           [&](uint8_t b) { return b == static_cast<uint8_t>((i * 3 + 64 * plane + l) & 0xff); });
      CHECK(ok);
    }
    // prefill releases its pages after the copy: fences on its stream
    for (int l = 0; l < layers; ++l)
      for (int id : src) p_pages.retire(l, id);
    REQUIRE(pbe_stream_synchronize(0, p_stream) == PBE_OK);
    p_pages.collect();
    CHECK_EQ(p_pages.leased_bytes(), 0u);
    reservations.release(&res);
    REQUIRE(pbe_stream_synchronize(0, d_stream) == PBE_OK);
    d_pages.collect();
    CHECK_EQ(d_pages.leased_bytes(), 0u);
    conn.release(h);
  }
  CHECK_EQ(owner->lease_count(), 0u);
  CHECK_EQ(owner->free_bytes(), arena_bytes);
  pbe_stream_destroy(0, p_stream);
  pbe_stream_destroy(0, d_stream);
  CHECK(pbe_arena_destroy(arena) == PBE_OK);
}

TEST_CASE("zero-copy takeover: moved Chunks are read in place, shared pages are copied") {
  // Qwen2.5-0.5B geometry, 3-page Chunks: request A = 5 pages, request B = 1
  // page in A's last Chunk, so A's pages 3-4 must be copied and 0-2 move.
  const int layers = 24;
  const uint64_t half = 16 * 2 * 64 * 2, page = 2 * layers * half;
  const uint64_t arena_bytes = 48 * page;
  pbe_arena* arena = nullptr;
  REQUIRE(pbe_arena_create(0, arena_bytes, 16 * page, 5151, &arena) == PBE_OK);  // 3 segments
  pbe_arena_view view{};
  REQUIRE(pbe_arena_get_view(arena, &view) == PBE_OK);
  auto owner = std::make_shared<base::LocalChunkOwner>(arena_bytes, 5151);
  owner->register_model("prefill", 24 * page);
  owner->register_model("decode", 24 * page);
  void* p_stream = nullptr;
  void* d_stream = nullptr;
  REQUIRE(pbe_stream_create(0, &p_stream) == PBE_OK);
  REQUIRE(pbe_stream_create(0, &d_stream) == PBE_OK);
  auto addr = [&](int32_t id) {
    const uint64_t off = static_cast<uint64_t>(id) * half;
    return static_cast<uint8_t*>(view.base[off / view.segment_bytes]) + off % view.segment_bytes;
  };
  {
    auto p_client = std::make_shared<base::SharedKVArenaClient>(owner, view, "prefill", 24 * page, 0);
    auto d_client = std::make_shared<base::SharedKVArenaClient>(owner, view, "decode", 24 * page, 0);
    base::SharedKVPageGroup p_pages(p_client, layers, half, 3 * page, p_stream);
    base::SharedKVPageGroup d_pages(d_client, layers, half, 3 * page, d_stream);
    auto alloc = [&](int n) {
      std::vector<int32_t> ids;
      for (int i = 0; i < n; ++i) ids.push_back(p_pages.allocate(0));
      for (int l = 1; l < layers; ++l)
        for (int i = 0; i < n; ++i) CHECK_EQ(p_pages.allocate(l), ids[i]);
      return ids;
    };
    auto a = alloc(5);
    auto b = alloc(1);
    std::vector<uint8_t> host(page);
    for (size_t i = 0; i < a.size(); ++i) {
      for (uint64_t k = 0; k < page; ++k) host[k] = static_cast<uint8_t>((k * 7 + i * 31) >> 3);
      HIP_OK(hipMemcpy(addr(a[i]), host.data(), page, hipMemcpyHostToDevice));
    }
    base::SharedKVPageGroup::PageTakeover tk;
    p_pages.detach_for_takeover(a, &tk);
    CHECK_EQ(tk.moved_ids.size(), 3u);
    CHECK_EQ(tk.copy_ids.size(), 2u);
    serving::KVPoolDescriptor pool{0, layers, 16, 2, 64, base::DataType::kDataTypeBf16,
                                   base::BlockStorageMode::kPlain};
    serving::SharedArenaBinding binding{view, 5151, 0};
    std::vector<int32_t> table;
    uint64_t copied = 0;
    REQUIRE(serving::TakeOverSharedKV(&d_pages, binding, tk, pool, d_stream, &table, &copied));
    p_pages.finish_takeover(tk);
    CHECK_EQ(copied, 2 * page);
    REQUIRE(table.size() == a.size());
    for (int i = 0; i < 3; ++i) CHECK_EQ(table[i], a[i]);  // used in place
    REQUIRE(pbe_stream_synchronize(0, d_stream) == PBE_OK);
    for (size_t i = 0; i < a.size(); ++i) {
      HIP_OK(hipMemcpy(host.data(), addr(table[i]), page, hipMemcpyDeviceToHost));
      bool ok = true;
      for (uint64_t k = 0; k < page && ok; ++k) ok = host[k] == static_cast<uint8_t>((k * 7 + i * 31) >> 3);
      CHECK(ok);
    }
    CHECK_EQ(owner->leased_bytes("decode"), 6 * page);  // adopted Chunk + a Chunk for the 2 copies
    CHECK_EQ(owner->leased_bytes("prefill"), 3 * page);
    // prefill retires the copied pages and B; decode retires the whole request
    for (int l = 0; l < layers; ++l) {
      for (int32_t id : tk.copy_ids) p_pages.retire(l, id);
      for (int32_t id : b) p_pages.retire(l, id);
      for (int32_t id : table) d_pages.retire(l, id);
    }
    REQUIRE(pbe_stream_synchronize(0, p_stream) == PBE_OK);
    REQUIRE(pbe_stream_synchronize(0, d_stream) == PBE_OK);
    p_pages.collect();
    d_pages.collect();
    CHECK_EQ(p_pages.leased_bytes(), 0u);
    CHECK_EQ(d_pages.leased_bytes(), 0u);
  }
  CHECK_EQ(owner->lease_count(), 0u);
  CHECK_EQ(owner->free_bytes(), arena_bytes);
  pbe_stream_destroy(0, p_stream);
  pbe_stream_destroy(0, d_stream);
  CHECK(pbe_arena_destroy(arena) == PBE_OK);
}

MINITEST_MAIN()
