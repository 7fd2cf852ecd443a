// Host-side costs of the handoff's C++ paths at config-2 size (Qwen2.5-1.5B,
// 28 layers, 315 pages), run by `bench.py --host-paths`; prints one JSON object.
//   - the generic plan form (InProcKVBlockCopyConnector, pd_handoff.cpp:192-213):
//     per-page BindComponents binding, BindManifestCopyOps, pbe_copy_ops of the
//     op list, and the connector's submit -> drain; the 315 per-page
//     BoundTransfers through the HIP TransferBackend (submit all, drain), and
//     their 17,640 component ops as one hipMemcpyAsync each, the reference
//     CudaTransferBackend's pattern (cuda_transfer_backend.cpp:19-128);
//   - the reference's copy_shared_kv call order (split_pd_engine.cpp:49-115)
//     through serving::CopySharedKVToDecode: append_slots over 28 layers, the
//     whole call, and free_request afterwards; and the reservation while the
//     previous request's pages still wait on their fences behind a 1 GiB copy.
// Every figure is the median over the iterations, in microseconds.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <memory>
#include <numeric>
#include <random>
#include <vector>

#include "base/kv_cache_manager.h"
#include "base/shared_kv_arena.h"
#include "cache/page_migration.h"
#include "cache/transfer_plan.h"
#include "pbe_handoff.h"
#include "serving/pd_handoff.h"
#include "serving/split_pd_handoff.h"

namespace {

constexpr int kLayers = 28, kHeads = 2, kDim = 128, kPages = 315, kIters = 25;

double now_us() {
  return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

double median(std::vector<double> v) {
  std::sort(v.begin(), v.end());
  return v[v.size() / 2];
}

std::unique_ptr<base::KVCacheManager> manager_over(const std::shared_ptr<base::SharedKVPageGroup>& g) {
  std::vector<std::unique_ptr<base::BlockAllocator>> layers;
  for (int l = 0; l < g->layers(); ++l) layers.push_back(std::make_unique<base::BlockAllocator>(16, kHeads, kDim, g, l));
  return std::make_unique<base::KVCacheManager>(16, g->layers(), std::move(layers));
}

#define CHECK_OR(cond, code) \
  do {                       \
    if (!(cond)) {           \
      std::fprintf(stderr, "failed: %s\n", #cond); \
      return code;           \
    }                        \
  } while (0)

}  // namespace

int main() {
  const uint64_t half = 16 * kHeads * kDim * 2, page = 2ull * kLayers * half;
  const serving::KVPoolDescriptor pool_desc{0, kLayers, 16, kHeads, kDim, base::DataType::kDataTypeBf16,
                                            base::BlockStorageMode::kPlain};
  // ---- generic plan form over a 1000-page device arena, made as the library
  // makes pools (pbe_arena_create: its allocation is in the library's registry)
  std::vector<double> bind_us, ops_us, call_us, conn_us, backend_us, per_op_us;
  {
    const uint64_t pages = 1000, bytes = pages * page;
    pbe_arena* arena = nullptr;
    CHECK_OR(pbe_arena_create(0, bytes, bytes, 1, &arena) == PBE_OK, 2);
    serving::ArenaKVPool pool;
    pbe_arena_get_view(arena, &pool.view);
    pool.pool = pool_desc;
    std::vector<int> perm(pages);
    std::iota(perm.begin(), perm.end(), 0);
    std::shuffle(perm.begin(), perm.end(), std::mt19937(5));
    std::vector<int32_t> src, dst;
    for (int i = 0; i < kPages; ++i) {
      src.push_back(perm[i] * 2 * kLayers);
      dst.push_back(perm[kPages + i] * 2 * kLayers);
    }
    serving::KVBlockManifest m;
    m.client_request_id.value = "c2";
    m.handoff_id.value = 1;
    m.prompt_tokens = m.computed_tokens = 5040;
    m.src_pool = m.dst_pool = pool_desc;
    for (int l = 0; l < kLayers; ++l) m.layer_mappings.push_back({l, src, dst});
    serving::InProcKVBlockCopyConnector conn(pool, pool, 0);
    auto backend = cache::MakeHipTransferBackend(512, 0);
    CHECK_OR(backend != nullptr, 10);
    hipStream_t ref_stream = nullptr;
    CHECK_OR(hipStreamCreateWithFlags(&ref_stream, hipStreamNonBlocking) == hipSuccess, 11);
    for (int it = 0; it < kIters; ++it) {
      cache::TransferPlanner planner;
      std::vector<cache::BoundTransfer> t;
      double a = now_us();
      CHECK_OR(serving::BindManifestTransfers(m, pool, pool, &planner, &t), 3);
      bind_us.push_back(now_us() - a);
      std::vector<pbe_copy_op> ops;
      a = now_us();
      CHECK_OR(serving::BindManifestCopyOps(m, pool, pool, &planner, &ops), 4);
      ops_us.push_back(now_us() - a);
      CHECK_OR(hipDeviceSynchronize() == hipSuccess, 5);
      a = now_us();
      CHECK_OR(pbe_copy_ops(ops.data(), static_cast<int64_t>(ops.size()), 0, nullptr) == PBE_OK, 6);
      call_us.push_back(now_us() - a);
      CHECK_OR(hipDeviceSynchronize() == hipSuccess, 7);
      a = now_us();
      serving::HandoffId h;
      CHECK_OR(conn.submit(m, &h), 8);
      CHECK_OR(conn.drain(h).ok(), 9);
      conn_us.push_back(now_us() - a);
      conn.release(h);
    }
    // Then, apart (their thousands of runtime calls would otherwise sit
    // between the legs above): the page transfers through the HIP backend,
    // and the same ops as one async memcpy each.
    {
      cache::TransferPlanner planner;
      std::vector<cache::BoundTransfer> t;
      CHECK_OR(serving::BindManifestTransfers(m, pool, pool, &planner, &t), 16);
      for (int it = 0; it < kIters; ++it) {
        // the page transfers through the HIP backend: one launch per transfer
        // on its in-order stream, the last drain waits for all
        const cache::MigrationId base_id = 1000ull * (it + 1);
        double a = now_us();
        for (size_t i = 0; i < t.size(); ++i) {
          const auto r = backend->submit(base_id + i, cache::TransferDirection::kGpuToGpu, t[i]);
          CHECK_OR(r == cache::BackendResult::kPending || r == cache::BackendResult::kSucceeded, 12);
        }
        for (size_t i = 0; i < t.size(); ++i)
          CHECK_OR(backend->drain(base_id + i) == cache::BackendResult::kSucceeded, 13);
        backend_us.push_back(now_us() - a);
        for (size_t i = 0; i < t.size(); ++i) backend->release(base_id + i);
        // the reference backend's pattern: one async memcpy per component op
        a = now_us();
        for (const auto& bt : t)
          for (const auto& op : bt.operations())
            CHECK_OR(hipMemcpyAsync(op.destination, op.source, op.bytes, hipMemcpyDeviceToDevice, ref_stream) ==
                         hipSuccess, 14);
        CHECK_OR(hipStreamSynchronize(ref_stream) == hipSuccess, 15);
        per_op_us.push_back(now_us() - a);
      }
    }
    (void)hipStreamDestroy(ref_stream);
    pbe_arena_destroy(arena);
  }
  // ---- the reference's call order over KVCacheManager and a shared arena
  std::vector<double> reserve_us, e2e_us, free_us, busy_us, copy_us;
  std::vector<double> step_request_us, step_reserve_us, step_launch_us, step_wait_us, step_commit_us;
  {
    const uint64_t arena_bytes = 2000 * page;
    pbe_arena* arena = nullptr;
    CHECK_OR(pbe_arena_create(0, arena_bytes, arena_bytes, 77, &arena) == PBE_OK, 10);
    pbe_arena_view view{};
    pbe_arena_get_view(arena, &view);
    auto owner = std::make_shared<base::LocalChunkOwner>(arena_bytes, 77);
    owner->register_model("prefill", 900 * page);
    owner->register_model("decode", 1000 * page);
    void *ps = nullptr, *ds = nullptr;
    CHECK_OR(pbe_stream_create(0, &ps) == PBE_OK && pbe_stream_create(0, &ds) == PBE_OK, 11);
    uint8_t *big_a = nullptr, *big_b = nullptr;
    const uint64_t big = 1ull << 30;
    CHECK_OR(hipMalloc(&big_a, big) == hipSuccess && hipMalloc(&big_b, big) == hipSuccess, 12);
    {
      auto pc = std::make_shared<base::SharedKVArenaClient>(owner, view, "prefill", 900 * page, 0);
      auto dc = std::make_shared<base::SharedKVArenaClient>(owner, view, "decode", 1000 * page, 0);
      auto pg = std::make_shared<base::SharedKVPageGroup>(pc, kLayers, half, 2 * 1024 * 1024, ps);
      auto dg = std::make_shared<base::SharedKVPageGroup>(dc, kLayers, half, 2 * 1024 * 1024, ds);
      auto p_kv = manager_over(pg);
      auto d_kv = manager_over(dg);
      const base::RequestId pr = p_kv->register_request();
      CHECK_OR(p_kv->append_slots(pr, 5040), 13);
      serving::SharedKVPrefillResult r;
      r.shared_arena_epoch = pc->epoch();
      r.client_request_id.value = "c2";
      r.handoff_id.value = 1;
      r.prompt_tokens.assign(5040, 7);
      r.computed_tokens = 5040;
      r.first_token = 1;
      r.src_pool = pool_desc;
      for (int l = 0; l < kLayers; ++l) r.layers.push_back({l, p_kv->get_block_ids(pr, l)});
      for (int it = 0; it < kIters; ++it) {
        double a = now_us();
        const base::RequestId q = d_kv->register_request();
        CHECK_OR(d_kv->append_slots(q, 5040), 14);
        reserve_us.push_back(now_us() - a);
        d_kv->free_request(q);
        pbe_stream_synchronize(0, ds);
        dg->collect();
        serving::DecodeKVReservation res;
        a = now_us();
        CHECK_OR(serving::CopySharedKVToDecode(d_kv.get(), pool_desc, r, ds, &res) == kPages * page, 15);
        e2e_us.push_back(now_us() - a);
        // the copy and its wait alone, same pages (cold: a 1 GiB copy first)
        {
          pbe_copy_op flush{reinterpret_cast<uint64_t>(big_a), reinterpret_cast<uint64_t>(big_b), big};
          CHECK_OR(pbe_copy_ops(&flush, 1, 0, ds) == PBE_OK, 18);
          CHECK_OR(pbe_stream_synchronize(0, ds) == PBE_OK, 19);
          const pbe_kv_shape shape{kLayers, kHeads, kDim, 16};
          const auto& s_ids = r.layers[0].src_block_ids;
          const auto& d_ids = res.dst_block_ids_per_layer[0];
          uint64_t copied = 0;
          a = now_us();
          CHECK_OR(pbe_copy_shared_kv(&view, s_ids.data(), d_ids.data(), kPages, &shape, 0, ds,
                                      &copied) == PBE_OK, 20);
          CHECK_OR(pbe_stream_synchronize(0, ds) == PBE_OK, 21);
          copy_us.push_back(now_us() - a);
        }
        // the stream busy: the freed pages' fences stay pending behind a 1 GiB copy
        CHECK_OR(pbe_stream_synchronize(0, ds) == PBE_OK, 22);
        pbe_copy_op op{reinterpret_cast<uint64_t>(big_a), reinterpret_cast<uint64_t>(big_b), big};
        CHECK_OR(pbe_copy_ops(&op, 1, 0, ds) == PBE_OK, 16);
        a = now_us();
        d_kv->free_request(res.decode_request_id);
        free_us.push_back(now_us() - a);
        a = now_us();
        const base::RequestId busy = d_kv->register_request();
        CHECK_OR(d_kv->append_slots(busy, 5040), 17);
        busy_us.push_back(now_us() - a);
        d_kv->free_request(busy);
        pbe_stream_synchronize(0, ds);
        dg->collect();
      }
      // The same steps as CopySharedKVToDecode, through the same public calls,
      // with a timer between them (cold: a 1 GiB copy first).
      for (int it = 0; it < kIters; ++it) {
        pbe_copy_op flush{reinterpret_cast<uint64_t>(big_a), reinterpret_cast<uint64_t>(big_b), big};
        CHECK_OR(pbe_copy_ops(&flush, 1, 0, ds) == PBE_OK, 23);
        CHECK_OR(pbe_stream_synchronize(0, ds) == PBE_OK, 24);
        double t0 = now_us();
        serving::DecodeKVReservationRequest req;
        req.client_request_id = r.client_request_id;
        req.handoff_id = r.handoff_id;
        req.prompt_tokens = static_cast<int32_t>(r.prompt_tokens.size());
        req.computed_tokens = r.computed_tokens;
        req.first_token = r.first_token;
        req.src_pool = r.src_pool;
        for (const auto& layer : r.layers) req.src_block_ids_per_layer.push_back(layer.src_block_ids);
        double t1 = now_us();
        serving::DecodeKVReservationManager reservations(d_kv.get(), pool_desc);
        serving::DecodeKVReservation res;
        serving::KVBlockManifest manifest;
        CHECK_OR(static_cast<bool>(reservations.reserve(req, &res, &manifest)), 25);
        double t2 = now_us();
        const pbe_kv_shape shape{kLayers, kHeads, kDim, 16};
        uint64_t copied = 0;
        CHECK_OR(pbe_copy_shared_kv(&view, manifest.layer_mappings[0].src_block_ids.data(),
                                    manifest.layer_mappings[0].dst_block_ids.data(), kPages, &shape, 0,
                                    ds, &copied) == PBE_OK, 26);
        double t3 = now_us();
        CHECK_OR(pbe_stream_synchronize(0, ds) == PBE_OK, 27);
        double t4 = now_us();
        CHECK_OR(d_kv->commit_kv(res.decode_request_id, r.computed_tokens), 28);
        double t5 = now_us();
        step_request_us.push_back(t1 - t0);
        step_reserve_us.push_back(t2 - t1);
        step_launch_us.push_back(t3 - t2);
        step_wait_us.push_back(t4 - t3);
        step_commit_us.push_back(t5 - t4);
        d_kv->free_request(res.decode_request_id);
        pbe_stream_synchronize(0, ds);
        dg->collect();
      }
    }
    (void)hipFree(big_a);
    (void)hipFree(big_b);
    pbe_stream_destroy(0, ps);
    pbe_stream_destroy(0, ds);
    pbe_arena_destroy(arena);
  }
  std::printf(
      "{\"workload\": \"c2_host_paths\", \"pages\": %d, \"layers\": %d, \"iterations\": %d, "
      "\"generic_plan_form_us\": {\"per_page_binding\": %.1f, \"copy_op_binding\": %.1f, "
      "\"copy_ops_call\": %.1f, \"connector_submit_drain\": %.1f, "
      "\"hip_backend_315_transfers\": %.1f, \"per_op_memcpy_17640\": %.1f}, "
      "\"reference_call_order_us\": {\"reserve_28_layers\": %.1f, \"end_to_end\": %.1f, "
      "\"copy_and_sync_alone\": %.1f, \"free_request\": %.1f, "
      "\"reserve_under_pending_fences\": %.1f, \"steps\": {\"request_copies\": %.1f, "
      "\"reserve_and_manifest\": %.1f, \"pbe_copy_shared_kv_call\": %.1f, \"stream_wait\": %.1f, "
      "\"commit_kv\": %.1f}}}\n",
      kPages, kLayers, kIters, median(bind_us), median(ops_us), median(call_us), median(conn_us),
      median(backend_us), median(per_op_us),
      median(reserve_us), median(e2e_us), median(copy_us), median(free_us), median(busy_us),
      median(step_request_us), median(step_reserve_us), median(step_launch_us), median(step_wait_us),
      median(step_commit_us));
  return 0;
}
