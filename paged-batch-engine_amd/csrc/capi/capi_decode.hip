// C ABI: the decode-side reader (split counts, workspace sizes, the arena,
// pool and allocation-free entry points).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "capi_internal.h"
#include "../kernels/decode_kernels.h"

using namespace pbe_capi;


namespace {
// Compute units of the calling thread's current GPU (256 on MI355X), cached
// per device; 256 when the runtime cannot say.
int64_t decode_cus() {
  static std::mutex mu;
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      n = 256;
    }
    cus[dev] = n;
  }
  return cus[dev];
}
}  // namespace

extern "C" {

int32_t pbe_paged_decode_splits(int32_t batch, int32_t kv_heads, int32_t max_blocks_per_seq,
                                int32_t kv_dtype) {
  if (batch <= 0 || kv_heads <= 0 || max_blocks_per_seq <= 0) return 1;
  // One wave per SIMD (4 per CU) of the current GPU, rounded down so no
  // partial extra round of waves trails the launch; FP8 pages take two per
  // SIMD when every split still holds at least 8 blocks; at least 4 blocks
  // (64 tokens) per split. Measured on MI355X (256 CUs), FP8, both launches:
  // 5040-token sequences, batch 64: 16 splits 39.1 us against 40.9 us at 8;
  // batch 32: 32 splits 26.7 us against 30.2 us at 16; batch 128: 8 splits
  // 65.9 us against 84.1 us at 4 and 72.9 us at 16; batch 16: 32 splits
  // 20.9 us, 20.7 us at 64. 2048-token sequences, batch 64: 16 splits 24.6 us
  // against 27.0 us at 8 and 28.1 us at 32. One 160,000-token sequence (10,000
  // blocks): 1024 splits 29.5 us against 31.6 us at 512. BF16 batch 64: 54.6
  // us stage 1 at 8 splits against 56.5 us at 16. One 32768-token sequence:
  // 512 splits (4 blocks each) 12.0 + 5.9 us against 13.5 + 4.7 at 256.
  const int64_t simds = 4ll * decode_cus();
  const int64_t units = (int64_t)batch * kv_heads;
  int64_t splits = std::max<int64_t>(1, simds / units);
  if (kv_dtype == PBE_KV_FP8_E4M3) {
    const int64_t two = std::max<int64_t>(1, 2 * simds / units);
    if ((max_blocks_per_seq + two - 1) / two >= 8) splits = two;
  }
  splits = std::min<int64_t>(splits, (max_blocks_per_seq + 3) / 4);
  splits = std::min<int64_t>(splits, pbe::kDecodeMaxSplits);
  return (int32_t)std::max<int64_t>(1, splits);
}

uint64_t pbe_paged_decode_workspace_bytes(int32_t batch, int32_t q_heads, int32_t head_dim,
                                          int32_t splits) {
  if (batch <= 0 || q_heads <= 0 || head_dim <= 0 || splits <= 0) return 0;
  return pbe::decode_workspace_bytes(batch, q_heads, head_dim, splits);
}

}  // extern "C"

// The split-K partials of the allocation-free decode entry point: one copy of
// this array per GPU, for the life of the process. Host code never uses its
// name as an address: scratch_address() resolves the device copy once per GPU
// (hipGetSymbolAddress, with that GPU current) and every launch passes that.
static __device__ __align__(256) uint8_t scratch[PBE_DECODE_SCRATCH_BYTES];

namespace {

// Per-GPU state of the scratch array: its device address, and the last call
// that used it: an event recorded on that call's stream after its launches,
// and the stream. A call on another stream is refused (PBE_ERR_BUSY) while
// that event has not completed; on the same stream, stream order already
// serialises the two. `mu` makes check, launch and record one step for
// racing host threads.
struct ScratchState {
  std::mutex mu;
  void* ptr = nullptr;
  hipEvent_t last_use = nullptr;
  void* last_stream = nullptr;
  bool used = false;
};

ScratchState& scratch_state(int device) {
  static ScratchState states[64];
  return states[device];
}

// Resolves the array's address and creates the guard event once per GPU
// (with that GPU current); later calls allocate nothing.
int scratch_setup(int device, ScratchState** out) {
  if (device < 0 || device >= 64) return fail(PBE_ERR_INVALID, "device %d out of range", device);
  ScratchState& st = scratch_state(device);
  if (!st.ptr) {
    PBE_DEVICE_SCOPE(device);
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    hipEvent_t ev = nullptr;
    PBE_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    st.last_use = ev;
    st.ptr = ptr;
  }
  *out = &st;
  return PBE_OK;
}

// Per-layer K/V pools (pbe_paged_decode_pools): block b's K rows at
// key + b * half, its V rows at value + b * half, its FP8 scales at
// key_scales + b * 16 * kv_heads and value_scales + b * 16 * kv_heads.
struct DecodePools {
  const void* key;
  const void* value;
  uint64_t bytes;  // addressable from each of key and value
  const float* key_scales;
  const float* value_scales;
  uint64_t scale_bytes;  // addressable from each scale pointer
  // the append form's writable views of the same K pool and K scale pool
  // (null for the read-only entry points)
  void* key_w = nullptr;
  float* key_scales_w = nullptr;
};

// Shared body of the decode entry points. `static_scratch`: the workspace is
// this GPU's scratch array (known valid, not an allocation the runtime can
// describe), so it skips the pointer check and names its limit on overflow.
// `pools` non-null: per-layer pools instead of the page-major arena `kv`
// (shape->layers is then 1 and layer 0).
int paged_decode_call(const pbe_arena_view* kv, int32_t kv_dtype, const float* scales,
                      uint64_t scale_bytes, const pbe_kv_shape* shape, int32_t layer,
                      const void* queries, void* outputs, int32_t batch, int32_t q_heads,
                      const int32_t* block_tables, const int32_t* seq_lens,
                      int32_t max_blocks_per_seq, int32_t splits, void* workspace,
                      uint64_t workspace_bytes, int device, void* stream, bool static_scratch,
                      const DecodePools* pools = nullptr, const void* new_keys = nullptr,
                      const void* new_values = nullptr, float* append_scales = nullptr) {
  if ((!pools && !view_ok(kv)) || !shape_ok(shape))
    return fail(PBE_ERR_INVALID, "invalid decode arena view or shape");
  if (kv_dtype != PBE_KV_BF16 && kv_dtype != PBE_KV_FP8_E4M3)
    return fail(PBE_ERR_INVALID, "unknown KV dtype %d", (int)kv_dtype);
  const bool fp8 = kv_dtype == PBE_KV_FP8_E4M3;
  if (shape->page_tokens != 16 || (shape->head_dim != 64 && shape->head_dim != 128))
    return fail(PBE_ERR_UNSUPPORTED, "decode reader supports 16-token pages and head_dim 64 or 128");
  if (layer < 0 || layer >= shape->layers) return fail(PBE_ERR_INVALID, "layer %d out of range", (int)layer);
  if (batch <= 0 || q_heads <= 0 || max_blocks_per_seq <= 0)
    return fail(PBE_ERR_INVALID, "batch, q_heads and max_blocks_per_seq must be positive");
  if (q_heads % shape->kv_heads != 0 || q_heads / shape->kv_heads > pbe::kDecodeMaxKvMul)
    return fail(PBE_ERR_UNSUPPORTED, "q_heads must be 1..%d times kv_heads", pbe::kDecodeMaxKvMul);
  if (!queries || !outputs || !block_tables || !seq_lens || !workspace)
    return fail(PBE_ERR_INVALID, "null decode operand");
  if ((reinterpret_cast<uintptr_t>(queries) | reinterpret_cast<uintptr_t>(outputs)) % 16)
    return fail(PBE_ERR_INVALID, "queries and outputs must be 16-byte aligned");
  const bool append = new_keys || new_values;
  if (append && (!new_keys || !new_values))
    return fail(PBE_ERR_INVALID, "the new token needs both its keys and its values");
  if (append && (reinterpret_cast<uintptr_t>(new_keys) | reinterpret_cast<uintptr_t>(new_values)) % 16)
    return fail(PBE_ERR_INVALID, "new keys and values must be 16-byte aligned");
  if (fp8 && !pools && (!scales || scale_bytes == 0))
    return fail(PBE_ERR_INVALID, "FP8 pages need a scale pool");
  if (fp8 && pools && (!pools->key_scales || !pools->value_scales || pools->scale_bytes == 0))
    return fail(PBE_ERR_INVALID, "FP8 pools need K and V scale pools");
  if (pools && (!pools->key || !pools->value ||
                ((reinterpret_cast<uintptr_t>(pools->key) | reinterpret_cast<uintptr_t>(pools->value)) % 16) ||
                (fp8 && ((reinterpret_cast<uintptr_t>(pools->key_scales) |
                          reinterpret_cast<uintptr_t>(pools->value_scales)) % 4))))
    return fail(PBE_ERR_INVALID, "K/V pools must be 16-byte aligned and scale pools 4-byte aligned");
  if (splits == 0) {
    splits = pbe_paged_decode_splits(batch, shape->kv_heads, max_blocks_per_seq, kv_dtype);
    // The allocation-free form lowers an automatic count until the partials
    // fit its fixed scratch (the partials grow linearly with the splits).
    if (static_scratch) {
      const uint64_t per_split = pbe::decode_workspace_bytes(batch, q_heads, shape->head_dim, 1);
      splits = (int32_t)std::max<uint64_t>(1, std::min<uint64_t>(splits, workspace_bytes / per_split));
    }
  }
  if (splits < 0 || splits > pbe::kDecodeMaxSplits)
    return fail(PBE_ERR_INVALID, "splits must be 0..%d", pbe::kDecodeMaxSplits);
  const uint64_t need = pbe::decode_workspace_bytes(batch, q_heads, shape->head_dim, splits);
  if (workspace_bytes < need) {
    if (static_scratch)
      return fail(PBE_ERR_INVALID,
                  "decode needs %llu bytes of partials; the static scratch holds %llu "
                  "(use pbe_paged_decode with a workspace, or fewer splits)",
                  (unsigned long long)need, (unsigned long long)workspace_bytes);
    return fail(PBE_ERR_INVALID, "decode workspace holds %llu of %llu bytes",
                (unsigned long long)workspace_bytes, (unsigned long long)need);
  }
  const uint64_t half = half_bytes(*shape, fp8 ? 1u : 2u);
  const uint64_t page = 2ull * shape->layers * half;
  const uint64_t block_scale_bytes = 16ull * shape->kv_heads * 4;
  if (pools) {
    if (pools->bytes < half) return fail(PBE_ERR_INVALID, "decode pools must hold at least one block");
    if (fp8 && pools->scale_bytes < block_scale_bytes)
      return fail(PBE_ERR_INVALID, "scale pools must hold at least one block of scales");
  } else {
    if (kv->nseg > 1 && kv->segment_bytes % page)
      return fail(PBE_ERR_INVALID, "arena segments must hold whole pages");
    if (kv->bytes < page || (kv->nseg > 1 && kv->segment_bytes < page))
      return fail(PBE_ERR_INVALID, "decode arena must hold at least one page");
    if (fp8 && scale_bytes < 2ull * shape->layers * block_scale_bytes)
      return fail(PBE_ERR_INVALID, "scale pool must hold at least one page of scales");
  }
  const uint64_t row_bytes = (uint64_t)batch * q_heads * shape->head_dim * 2;
  const uint64_t new_bytes = (uint64_t)batch * shape->kv_heads * shape->head_dim * 2;
  {
    PBE_DEVICE_SCOPE(device);
    std::vector<Range> known;
    const bool pages_ok =
        pools ? accessible(pools->key, pools->bytes, device, &known) &&
                    accessible(pools->value, pools->bytes, device, &known) &&
                    (!fp8 || (accessible(pools->key_scales, pools->scale_bytes, device, &known) &&
                              accessible(pools->value_scales, pools->scale_bytes, device, &known)))
              : view_accessible(*kv, device, &known) &&
                    (!fp8 || accessible(scales, scale_bytes, device, &known));
    if (!pages_ok || !accessible(queries, row_bytes, device, &known) ||
        !accessible(outputs, row_bytes, device, &known) ||
        !accessible(block_tables, (uint64_t)batch * max_blocks_per_seq * 4, device, &known) ||
        !accessible(seq_lens, (uint64_t)batch * 4, device, &known) ||
        (!static_scratch && !accessible(workspace, need, device, &known)) ||
        (append && (!accessible(new_keys, new_bytes, device, &known) ||
                    !accessible(new_values, new_bytes, device, &known))))
      return fail(PBE_ERR_INVALID, "decode operands must be memory of device %d", device);
  }
  pbe::DecodeParams p{};
  if (pools) {
    p.kv.base[0] = static_cast<const char*>(pools->key);
    p.kv.segment_bytes = p.kv.bytes = pools->bytes;
    p.scales = fp8 ? pools->key_scales : nullptr;
    p.scale_bytes = fp8 ? pools->scale_bytes : 0;
    p.v_delta = static_cast<const char*>(pools->value) - static_cast<const char*>(pools->key);
    p.vscale_delta = fp8 ? pools->value_scales - pools->key_scales : 0;
  } else {
    for (uint32_t i = 0; i < kv->nseg; ++i) p.kv.base[i] = static_cast<const char*>(kv->base[i]);
    p.kv.segment_bytes = kv->segment_bytes;
    p.kv.bytes = kv->bytes;
    p.scales = fp8 ? scales : nullptr;
    p.scale_bytes = fp8 ? scale_bytes : 0;
    p.v_delta = (int64_t)half;                            // V plane follows the K plane
    p.vscale_delta = 16ll * shape->kv_heads;              // and its scales one plane later
  }
  p.q = static_cast<const uint16_t*>(queries);
  p.out = static_cast<uint16_t*>(outputs);
  p.tables = block_tables;
  p.seq_lens = seq_lens;
  p.new_k = static_cast<const uint16_t*>(new_keys);
  p.new_v = static_cast<const uint16_t*>(new_values);
  if (append) {  // the memory the append form writes, through non-const pointers
    if (pools) {
      p.wbase[0] = static_cast<char*>(pools->key_w);
      p.wscales = fp8 ? pools->key_scales_w : nullptr;
    } else {
      for (uint32_t i = 0; i < kv->nseg; ++i) p.wbase[i] = static_cast<char*>(kv->base[i]);
      p.wscales = fp8 ? append_scales : nullptr;
    }
  }
  const uint64_t rows = (uint64_t)batch * q_heads * splits;
  p.part_acc = static_cast<float*>(workspace);
  p.part_m = p.part_acc + rows * shape->head_dim;
  p.part_l = p.part_m + rows;
  p.batch = batch;
  p.q_heads = q_heads;
  p.kv_heads = shape->kv_heads;
  p.head_dim = shape->head_dim;
  p.layers = shape->layers;
  p.layer = layer;
  p.max_blocks = max_blocks_per_seq;
  p.splits = splits;
  p.half = half;
  p.scale = (1.f / std::sqrt((float)shape->head_dim)) * 1.4426950408889634f;  // as launch_fp8_stage1
  // Largest id whose rows fit: page-major, the whole page (all 2*layers
  // planes) inside the arena and the scale pool; per-layer pools, the block's
  // K and V rows and scales inside the pools.
  const int64_t stride = pools ? 1 : 2ll * shape->layers;
  const uint64_t row_span = pools ? pools->bytes : kv->bytes;
  const uint64_t scale_span = pools ? pools->scale_bytes : scale_bytes;
  int64_t id_max = (int64_t)(row_span / half) - stride;
  if (fp8) id_max = std::min<int64_t>(id_max, (int64_t)(scale_span / block_scale_bytes) - stride);
  p.id_max = (int32_t)std::min<int64_t>(id_max, INT32_MAX);
  p.by_stride = pbe::make_fast_div((uint32_t)stride);
  p.by_seg_pages = pbe::make_fast_div(!pools && kv->nseg > 1 ? (uint32_t)(kv->segment_bytes / page) : 0x7fffffffu);
  PBE_DEVICE_SCOPE(device);
  PBE_HIP(pbe::launch_paged_decode(p, fp8, static_cast<hipStream_t>(stream)));
  return PBE_OK;
}

}  // namespace

extern "C" {

int pbe_paged_decode(const pbe_arena_view* kv, int32_t kv_dtype, const float* scales,
                     uint64_t scale_bytes, const pbe_kv_shape* shape, int32_t layer,
                     const void* queries, void* outputs, int32_t batch, int32_t q_heads,
                     const int32_t* block_tables, const int32_t* seq_lens,
                     int32_t max_blocks_per_seq, int32_t splits, void* workspace,
                     uint64_t workspace_bytes, int device, void* stream) {
  return paged_decode_call(kv, kv_dtype, scales, scale_bytes, shape, layer, queries, outputs, batch,
                           q_heads, block_tables, seq_lens, max_blocks_per_seq, splits, workspace,
                           workspace_bytes, device, stream, false);
}

int pbe_paged_decode_noalloc(const pbe_arena_view* kv, int32_t kv_dtype, const float* scales,
                             uint64_t scale_bytes, const pbe_kv_shape* shape, int32_t layer,
                             const void* queries, void* outputs, int32_t batch, int32_t q_heads,
                             const int32_t* block_tables, const int32_t* seq_lens,
                             int32_t max_blocks_per_seq, int32_t splits, int device, void* stream) {
  if (device < 0 || device >= 64) return fail(PBE_ERR_INVALID, "device %d out of range", device);
  ScratchState& st = scratch_state(device);
  std::lock_guard<std::mutex> lock(st.mu);
  ScratchState* ready = nullptr;
  int rc = scratch_setup(device, &ready);
  if (rc != PBE_OK) return rc;
  PBE_DEVICE_SCOPE(device);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // Under graph capture nothing runs now: the guard neither checks nor
  // records (replays of the graph are ordered by whoever launches them).
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  PBE_HIP(hipStreamIsCapturing(s, &capture));
  const bool live = capture == hipStreamCaptureStatusNone;
  if (live && st.used && st.last_stream != stream) {
    const hipError_t q = hipEventQuery(st.last_use);
    if (q == hipErrorNotReady)
      return fail(PBE_ERR_BUSY,
                  "the static decode scratch of device %d is still in use by a call on another "
                  "stream; wait for that stream or issue both calls on one stream", device);
    if (q != hipSuccess) return hip_fail(q, "hipEventQuery(decode scratch guard)");
  }
  rc = paged_decode_call(kv, kv_dtype, scales, scale_bytes, shape, layer, queries, outputs, batch,
                         q_heads, block_tables, seq_lens, max_blocks_per_seq, splits, st.ptr,
                         PBE_DECODE_SCRATCH_BYTES, device, stream, true);
  if (rc != PBE_OK || !live) return rc;
  PBE_HIP(hipEventRecord(st.last_use, s));
  st.last_stream = stream;
  st.used = true;
  return PBE_OK;
}

int pbe_paged_decode_pools(const void* key_pool, const void* value_pool, uint64_t pool_bytes,
                           const float* key_scales, const float* value_scales,
                           uint64_t scale_pool_bytes, int32_t kv_dtype, int32_t kv_heads,
                           int32_t head_dim, const void* queries, void* outputs, int32_t batch,
                           int32_t q_heads, const int32_t* block_tables, const int32_t* seq_lens,
                           int32_t max_blocks_per_seq, int32_t splits, void* workspace,
                           uint64_t workspace_bytes, int device, void* stream) {
  const pbe_kv_shape shape{1, kv_heads, head_dim, 16};
  const DecodePools pools{key_pool, value_pool, pool_bytes, key_scales, value_scales, scale_pool_bytes};
  return paged_decode_call(nullptr, kv_dtype, nullptr, 0, &shape, 0, queries, outputs, batch, q_heads,
                           block_tables, seq_lens, max_blocks_per_seq, splits, workspace,
                           workspace_bytes, device, stream, false, &pools);
}

int pbe_paged_decode_append_arena(const pbe_arena_view* kv, int32_t kv_dtype, float* scales,
                                  uint64_t scale_bytes, const pbe_kv_shape* shape, int32_t layer,
                                  const void* new_keys, const void* new_values, const void* queries,
                                  void* outputs, int32_t batch, int32_t q_heads,
                                  const int32_t* block_tables, const int32_t* seq_lens,
                                  int32_t max_blocks_per_seq, int32_t splits, void* workspace,
                                  uint64_t workspace_bytes, int device, void* stream) {
  if (!new_keys || !new_values) return fail(PBE_ERR_INVALID, "null new keys or values");
  return paged_decode_call(kv, kv_dtype, scales, scale_bytes, shape, layer, queries, outputs, batch, q_heads,
                           block_tables, seq_lens, max_blocks_per_seq, splits, workspace, workspace_bytes,
                           device, stream, false, nullptr, new_keys, new_values, scales);
}

int pbe_paged_decode_append(void* key_pool, void* value_pool, uint64_t pool_bytes,
                            float* key_scales, float* value_scales, uint64_t scale_pool_bytes,
                            int32_t kv_dtype, int32_t kv_heads, int32_t head_dim, const void* new_keys,
                            const void* new_values, const void* queries, void* outputs, int32_t batch,
                            int32_t q_heads, const int32_t* block_tables, const int32_t* seq_lens,
                            int32_t max_blocks_per_seq, int32_t splits, void* workspace,
                            uint64_t workspace_bytes, int device, void* stream) {
  if (!new_keys || !new_values) return fail(PBE_ERR_INVALID, "null new keys or values");
  const pbe_kv_shape shape{1, kv_heads, head_dim, 16};
  DecodePools pools{key_pool, value_pool, pool_bytes, key_scales, value_scales, scale_pool_bytes};
  pools.key_w = key_pool;
  pools.key_scales_w = key_scales;
  return paged_decode_call(nullptr, kv_dtype, nullptr, 0, &shape, 0, queries, outputs, batch, q_heads,
                           block_tables, seq_lens, max_blocks_per_seq, splits, workspace,
                           workspace_bytes, device, stream, false, &pools, new_keys, new_values);
}

}  // extern "C"
