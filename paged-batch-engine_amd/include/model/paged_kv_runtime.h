// The page-writing half of the reference's PagedKVRuntime
// (infMain/include/model/paged_kv_runtime.h:52-82): CudaPagedKVRuntime::scatter
// and scatter_single_token (paged_kv_runtime.cpp:207-290) over this build's
// KVPoolView, on one gfx950 kernel (pbe_scatter_kv / pbe_scatter_kv_to_page).
// Device pointers stand where the reference passes tensor::Tensor:
//   key, value     [batch_tokens][num_kv_heads * head_size] of input_dtype
//                  (kDataTypeBf16 or kDataTypeFp32), device memory;
//   slot_mapping   int32 [batch_tokens] in device memory, block * block_size + offset.
// Plain pools hold the input type; FP8 pools (pool.uses_fp8_storage()) get E4M3
// bytes and one fp32 scale per (token, head). Writes are bounded by the pool
// sizes the view carries; negative slots are skipped. Launches are asynchronous
// on the runtime's stream. decode() reads any KVPoolView through
// pbe_paged_decode_pools, and decode_append() writes the step's new tokens in
// the same launch; prefill attention is outside this build.
#ifndef PBE_INCLUDE_MODEL_PAGED_KV_RUNTIME_H_
#define PBE_INCLUDE_MODEL_PAGED_KV_RUNTIME_H_

#include <cstdint>

#include "base/base.h"
#include "base/block_allocator.h"

namespace model {

// PagedKVDecodeRuntimeArgs (paged_kv_runtime.h:12-27) with device pointers for
// the tensors. The reference's partial_out / partial_max / partial_sum become
// one workspace of pbe_paged_decode_workspace_bytes(batch_size, head_num,
// head_size, splits) bytes; splits = 0 lets the library choose.
struct PagedKVDecodeRuntimeArgs {
  int32_t batch_size = 0;
  int32_t head_num = 0;       // query heads
  int32_t head_size = 0;
  int32_t kv_mul = 0;         // head_num / num_kv_heads
  int32_t max_blocks_per_seq = 0;
  int32_t block_size = 0;     // 16
  int32_t num_kv_heads = 0;
  const void* queries = nullptr;       // bf16 [batch][head_num][head_size]
  void* outputs = nullptr;             // bf16 [batch][head_num][head_size]
  const int32_t* block_tables = nullptr;  // [batch][max_blocks_per_seq]
  const int32_t* seq_lens = nullptr;      // [batch]
  void* workspace = nullptr;
  uint64_t workspace_bytes = 0;
  int32_t splits = 0;
};

class HipPagedKVRuntime {
 public:
  // `stream`: a hipStream_t of `device` (nullptr: the null stream).
  HipPagedKVRuntime(int device, void* stream) : device_(device), stream_(stream) {}

  // Throws std::invalid_argument for an invalid view, a view without pool sizes,
  // an input dtype other than BF16/FP32 or one that differs from a plain pool's
  // element type, and std::runtime_error when the library rejects the launch
  // (the reference aborts on CHECK in both cases).
  void scatter(const void* key, const void* value, base::DataType input_dtype,
               const base::KVPoolView& pool, const int32_t* slot_mapping, int32_t block_size,
               int32_t num_kv_heads, int32_t head_size, int32_t batch_tokens) const;
  void scatter_single_token(const void* key, const void* value, base::DataType input_dtype,
                            const base::KVPoolView& pool, int32_t physical_block_id,
                            int32_t offset_in_block, int32_t block_size, int32_t num_kv_heads,
                            int32_t head_size) const;

  // One decode step over the pool (CudaPagedKVRuntime::decode,
  // paged_kv_runtime.cpp:293-357). Returns false, launching nothing, for a
  // pool or shape the reader does not cover (plain pools other than BF16,
  // head_size other than 64/128, block_size other than 16, more than 8 query
  // heads per KV head), so the caller keeps its own path; throws std::invalid_argument for an inconsistent call and
  // std::runtime_error when the launch fails.
  bool decode(const base::KVPoolView& pool, const PagedKVDecodeRuntimeArgs& args) const;

  // decode() preceded by writing each sequence's new token (bf16
  // [batch][num_kv_heads][head_size] K and V) at its last position,
  // seq_lens[b] - 1, in one launch pair (pbe_paged_decode_append): the same
  // pool bytes and outputs as scatter() of those tokens at the slots
  // append_slots handed out, then decode(). The reference runs the two
  // separately (paged_kv_runtime.cpp:207-245,293-357). Same return and throw
  // rules as decode().
  bool decode_append(const base::KVPoolView& pool, const PagedKVDecodeRuntimeArgs& args, const void* new_keys,
                     const void* new_values) const;

  int device() const { return device_; }
  void* stream() const { return stream_; }

 private:
  bool read(const base::KVPoolView& pool, const PagedKVDecodeRuntimeArgs& args, const void* new_keys,
            const void* new_values) const;

  int device_;
  void* stream_;
};

}  // namespace model

#endif  // PBE_INCLUDE_MODEL_PAGED_KV_RUNTIME_H_
