// C ABI: the page writer (new tokens' K/V into their page slots).
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
#include "../kernels/scatter_kernels.h"

using namespace pbe_capi;

namespace {

// Shared body of both page-writer entry points: slots in device memory, or
// (slots == nullptr) one token at fixed_slot.
int scatter_call(const void* keys, const void* values, int32_t in_dtype, int32_t n_tokens,
                 const int32_t* slots, int32_t fixed_slot, int32_t block_size, int32_t kv_heads,
                 int32_t head_dim, int32_t kv_dtype, void* key_pool, uint64_t key_pool_bytes,
                 void* value_pool, uint64_t value_pool_bytes, float* key_scales,
                 uint64_t key_scale_bytes, float* value_scales, uint64_t value_scale_bytes,
                 int device, void* stream) {
  if (in_dtype != PBE_IN_BF16 && in_dtype != PBE_IN_F32)
    return fail(PBE_ERR_INVALID, "unknown input dtype %d", (int)in_dtype);
  if (kv_dtype != PBE_KV_BF16 && kv_dtype != PBE_KV_FP8_E4M3)
    return fail(PBE_ERR_INVALID, "unknown KV dtype %d", (int)kv_dtype);
  if (n_tokens < 0 || block_size <= 0 || kv_heads <= 0 || head_dim <= 0 || device < 0)
    return fail(PBE_ERR_INVALID, "n_tokens >= 0, block_size, kv_heads, head_dim > 0 and a device");
  if (n_tokens == 0) return PBE_OK;
  const bool f32 = in_dtype == PBE_IN_F32, fp8 = kv_dtype == PBE_KV_FP8_E4M3;
  const uint64_t e_in = f32 ? 4 : 2, e_out = fp8 ? 1 : e_in;
  const uint64_t kv_dim = (uint64_t)kv_heads * head_dim;
  const uint64_t row_in = kv_dim * e_in, row_out = kv_dim * e_out;
  if (row_in % 16) return fail(PBE_ERR_INVALID, "a K/V row must be a multiple of 16 bytes");
  uint32_t lanes = 1;
  if (fp8) {
    const uint64_t l = (uint64_t)head_dim * e_in / 16;
    if ((uint64_t)head_dim * e_in % 16 || l == 0 || l > 64 || (l & (l - 1)))
      return fail(PBE_ERR_UNSUPPORTED, "FP8 pages need head_dim * input bytes / 16 to be a power of two up to 64");
    lanes = (uint32_t)l;
    if (!key_scales || !value_scales) return fail(PBE_ERR_INVALID, "FP8 pools need K and V scale pools");
  }
  const uint64_t units = (uint64_t)n_tokens * 2 * (row_in / 16);
  if (units >= 0x80000000ull) return fail(PBE_ERR_INVALID, "too many tokens for one launch");
  if (!keys || !values || !key_pool || !value_pool) return fail(PBE_ERR_INVALID, "null K/V operand");
  const uintptr_t out_align = fp8 ? (f32 ? 4 : 8) : 16;
  if (((reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(values)) % 16) ||
      ((reinterpret_cast<uintptr_t>(key_pool) | reinterpret_cast<uintptr_t>(value_pool)) % out_align) ||
      (fp8 && ((reinterpret_cast<uintptr_t>(key_scales) | reinterpret_cast<uintptr_t>(value_scales)) % 4)))
    return fail(PBE_ERR_INVALID, "inputs must be 16-byte aligned and pools aligned to their stores");
  {
    PBE_DEVICE_SCOPE(device);
    std::vector<Range> known;
    const uint64_t in_bytes = (uint64_t)n_tokens * row_in;
    if (!accessible(keys, in_bytes, device, &known) || !accessible(values, in_bytes, device, &known) ||
        (slots && !accessible(slots, (uint64_t)n_tokens * 4, device, &known)) ||
        (key_pool_bytes && !accessible(key_pool, key_pool_bytes, device, &known)) ||
        (value_pool_bytes && !accessible(value_pool, value_pool_bytes, device, &known)) ||
        (fp8 && key_scale_bytes && !accessible(key_scales, key_scale_bytes, device, &known)) ||
        (fp8 && value_scale_bytes && !accessible(value_scales, value_scale_bytes, device, &known)))
      return fail(PBE_ERR_INVALID, "page writer operands must be memory of device %d", device);
  }
  pbe::ScatterParams p{};
  p.keys = static_cast<const uint8_t*>(keys);
  p.values = static_cast<const uint8_t*>(values);
  p.key_pool = static_cast<uint8_t*>(key_pool);
  p.value_pool = static_cast<uint8_t*>(value_pool);
  p.key_pool_bytes = key_pool_bytes;
  p.value_pool_bytes = value_pool_bytes;
  p.key_scales = fp8 ? key_scales : nullptr;
  p.value_scales = fp8 ? value_scales : nullptr;
  p.key_scale_count = fp8 ? key_scale_bytes / 4 : 0;
  p.value_scale_count = fp8 ? value_scale_bytes / 4 : 0;
  p.slots = slots;
  p.fixed_slot = fixed_slot;
  p.units = (uint32_t)units;
  p.vecs_per_row = (uint32_t)(row_in / 16);
  p.row_in_bytes = (uint32_t)row_in;
  p.row_out_bytes = (uint32_t)row_out;
  p.block_out_bytes = (uint64_t)block_size * row_out;
  p.block_size = (uint32_t)block_size;
  p.kv_heads = (uint32_t)kv_heads;
  p.by_row_pair = pbe::make_fast_div(2 * p.vecs_per_row);
  p.by_block_size = pbe::make_fast_div((uint32_t)block_size);
  PBE_DEVICE_SCOPE(device);
  PBE_HIP(pbe::launch_scatter_kv(p, f32, fp8, lanes, static_cast<hipStream_t>(stream)));
  return PBE_OK;
}

}  // namespace

extern "C" {

int pbe_scatter_kv(const void* keys, const void* values, int32_t in_dtype, int32_t n_tokens,
                   const int32_t* slot_mapping, int32_t block_size, int32_t kv_heads,
                   int32_t head_dim, int32_t kv_dtype, void* key_pool, uint64_t key_pool_bytes,
                   void* value_pool, uint64_t value_pool_bytes, float* key_scales,
                   uint64_t key_scale_bytes, float* value_scales, uint64_t value_scale_bytes,
                   int device, void* stream) {
  if (n_tokens > 0 && !slot_mapping) return fail(PBE_ERR_INVALID, "null slot mapping");
  return scatter_call(keys, values, in_dtype, n_tokens, slot_mapping, 0, block_size, kv_heads,
                      head_dim, kv_dtype, key_pool, key_pool_bytes, value_pool, value_pool_bytes,
                      key_scales, key_scale_bytes, value_scales, value_scale_bytes, device, stream);
}

int pbe_scatter_kv_to_page(const void* keys, const void* values, int32_t in_dtype,
                           int32_t physical_block_id, int32_t offset_in_block,
                           int32_t block_size, int32_t kv_heads, int32_t head_dim,
                           int32_t kv_dtype, void* key_pool, uint64_t key_pool_bytes,
                           void* value_pool, uint64_t value_pool_bytes, float* key_scales,
                           uint64_t key_scale_bytes, float* value_scales,
                           uint64_t value_scale_bytes, int device, void* stream) {
  if (block_size <= 0 || physical_block_id < 0 || offset_in_block < 0 || offset_in_block >= block_size ||
      (int64_t)physical_block_id * block_size + offset_in_block > INT32_MAX)
    return fail(PBE_ERR_INVALID, "block %d offset %d is not a slot", (int)physical_block_id,
                (int)offset_in_block);
  return scatter_call(keys, values, in_dtype, 1, nullptr, physical_block_id * block_size + offset_in_block,
                      block_size, kv_heads, head_dim, kv_dtype, key_pool, key_pool_bytes, value_pool,
                      value_pool_bytes, key_scales, key_scale_bytes, value_scales, value_scale_bytes,
                      device, stream);
}

}  // extern "C"
