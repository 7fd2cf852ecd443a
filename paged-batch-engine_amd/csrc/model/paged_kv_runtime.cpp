// CudaPagedKVRuntime::scatter / scatter_single_token / decode
// (paged_kv_runtime.cpp:207-357) over the C ABI's page writer and decode reader.
#include "model/paged_kv_runtime.h"

#include <algorithm>
#include <stdexcept>
#include <string>

#include "pbe_handoff.h"

namespace model {
namespace {

struct Operands {
  int32_t in_dtype;
  int32_t kv_dtype;
  float* key_scales;
  float* value_scales;
  uint64_t scale_bytes;
};

Operands check(const base::KVPoolView& pool, base::DataType input_dtype) {
  if (!pool.valid()) throw std::invalid_argument("KV pool view is not bound");
  if (!pool.key_pool_bytes() || !pool.value_pool_bytes())
    throw std::invalid_argument("KV pool view carries no pool sizes");
  if (input_dtype != base::DataType::kDataTypeBf16 && input_dtype != base::DataType::kDataTypeFp32)
    throw std::invalid_argument("K/V input must be BF16 or FP32");
  // A plain pool holds the input type (the reference's kernels are templated
  // on one element type for both): BF16 input into an FP32 pool, or the
  // reverse, would store the wrong bytes.
  if (!pool.uses_fp8_storage() && pool.storage_spec().storage_dtype != base::DataType::kDataTypeUnknown &&
      pool.storage_spec().storage_dtype != input_dtype)
    throw std::invalid_argument("K/V input dtype differs from the plain pool's element type");
  Operands o{input_dtype == base::DataType::kDataTypeFp32 ? PBE_IN_F32 : PBE_IN_BF16, PBE_KV_BF16,
             nullptr, nullptr, 0};
  if (pool.uses_fp8_storage()) {
    if (!pool.key_scale_pool() || !pool.value_scale_pool() || !pool.scale_pool_bytes())
      throw std::invalid_argument("FP8 KV pool view has no scale pools");
    o.kv_dtype = PBE_KV_FP8_E4M3;
    o.key_scales = static_cast<float*>(pool.key_scale_pool());
    o.value_scales = static_cast<float*>(pool.value_scale_pool());
    o.scale_bytes = pool.scale_pool_bytes();
  }
  return o;
}

void raise_if_failed(int rc) {
  if (rc != PBE_OK) throw std::runtime_error(std::string("KV scatter launch failed: ") + pbe_last_error());
}

}  // namespace

void HipPagedKVRuntime::scatter(const void* key, const void* value, base::DataType input_dtype,
                                const base::KVPoolView& pool, const int32_t* slot_mapping,
                                int32_t block_size, int32_t num_kv_heads, int32_t head_size,
                                int32_t batch_tokens) const {
  const Operands o = check(pool, input_dtype);
  raise_if_failed(pbe_scatter_kv(key, value, o.in_dtype, batch_tokens, slot_mapping, block_size,
                                 num_kv_heads, head_size, o.kv_dtype, pool.key_pool(),
                                 pool.key_pool_bytes(), pool.value_pool(), pool.value_pool_bytes(),
                                 o.key_scales, o.scale_bytes, o.value_scales, o.scale_bytes, device_,
                                 stream_));
}

void HipPagedKVRuntime::scatter_single_token(const void* key, const void* value,
                                             base::DataType input_dtype, const base::KVPoolView& pool,
                                             int32_t physical_block_id, int32_t offset_in_block,
                                             int32_t block_size, int32_t num_kv_heads,
                                             int32_t head_size) const {
  const Operands o = check(pool, input_dtype);
  raise_if_failed(pbe_scatter_kv_to_page(key, value, o.in_dtype, physical_block_id, offset_in_block,
                                         block_size, num_kv_heads, head_size, o.kv_dtype,
                                         pool.key_pool(), pool.key_pool_bytes(), pool.value_pool(),
                                         pool.value_pool_bytes(), o.key_scales, o.scale_bytes,
                                         o.value_scales, o.scale_bytes, device_, stream_));
}

bool HipPagedKVRuntime::decode(const base::KVPoolView& pool, const PagedKVDecodeRuntimeArgs& args) const {
  return read(pool, args, nullptr, nullptr);
}

bool HipPagedKVRuntime::decode_append(const base::KVPoolView& pool, const PagedKVDecodeRuntimeArgs& args,
                                      const void* new_keys, const void* new_values) const {
  if (!new_keys || !new_values) throw std::invalid_argument("decode_append needs the new token's K and V");
  return read(pool, args, new_keys, new_values);
}

bool HipPagedKVRuntime::read(const base::KVPoolView& pool, const PagedKVDecodeRuntimeArgs& args,
                             const void* new_keys, const void* new_values) const {
  if (!pool.valid() || !pool.key_pool_bytes() || !pool.value_pool_bytes())
    throw std::invalid_argument("KV pool view is not bound or carries no pool sizes");
  if (!args.queries || !args.outputs || !args.block_tables || !args.seq_lens || !args.workspace)
    throw std::invalid_argument("decode arguments hold a null tensor");
  if (args.num_kv_heads <= 0 || args.kv_mul <= 0 || args.head_num != args.kv_mul * args.num_kv_heads)
    throw std::invalid_argument("head_num must equal kv_mul * num_kv_heads");
  if (args.block_size != 16) return false;
  const bool fp8 = pool.uses_fp8_storage();
  // The reader takes BF16 or FP8 E4M3 pages; other plain pools (FP32) keep
  // the caller's path.
  if (!fp8 && pool.storage_spec().storage_dtype != base::DataType::kDataTypeBf16) return false;
  if (fp8 && (!pool.key_scale_pool() || !pool.value_scale_pool() || !pool.scale_pool_bytes()))
    throw std::invalid_argument("FP8 KV pool view has no scale pools");
  const uint64_t bytes = std::min(pool.key_pool_bytes(), pool.value_pool_bytes());
  float* ks = fp8 ? static_cast<float*>(pool.key_scale_pool()) : nullptr;
  float* vs = fp8 ? static_cast<float*>(pool.value_scale_pool()) : nullptr;
  const uint64_t sb = fp8 ? pool.scale_pool_bytes() : 0;
  const int32_t dt = fp8 ? PBE_KV_FP8_E4M3 : PBE_KV_BF16;
  const int rc =
      new_keys ? pbe_paged_decode_append(pool.key_pool(), pool.value_pool(), bytes, ks, vs, sb, dt, args.num_kv_heads,
                                         args.head_size, new_keys, new_values, args.queries, args.outputs,
                                         args.batch_size, args.head_num, args.block_tables, args.seq_lens,
                                         args.max_blocks_per_seq, args.splits, args.workspace, args.workspace_bytes,
                                         device_, stream_)
               : pbe_paged_decode_pools(pool.key_pool(), pool.value_pool(), bytes, ks, vs, sb, dt, args.num_kv_heads,
                                        args.head_size, args.queries, args.outputs, args.batch_size, args.head_num,
                                        args.block_tables, args.seq_lens, args.max_blocks_per_seq, args.splits,
                                        args.workspace, args.workspace_bytes, device_, stream_);
  if (rc == PBE_ERR_UNSUPPORTED) return false;
  if (rc == PBE_ERR_INVALID) throw std::invalid_argument(std::string("decode rejected: ") + pbe_last_error());
  raise_if_failed(rc);
  return true;
}

}  // namespace model
