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
// on the runtime's stream. decode() is pbe_paged_decode in this build, and
// prefill attention is outside it.
#ifndef PBE_INCLUDE_MODEL_PAGED_KV_RUNTIME_H_
#define PBE_INCLUDE_MODEL_PAGED_KV_RUNTIME_H_

#include <cstdint>

#include "base/base.h"
#include "base/block_allocator.h"

namespace model {

class HipPagedKVRuntime {
 public:
  // `stream`: a hipStream_t of `device` (nullptr: the null stream).
  HipPagedKVRuntime(int device, void* stream) : device_(device), stream_(stream) {}

  // Throws std::invalid_argument for an invalid view, a view without pool sizes
  // or an input dtype other than BF16/FP32, and std::runtime_error when the
  // library rejects the launch (the reference aborts on CHECK in both cases).
  void scatter(const void* key, const void* value, base::DataType input_dtype,
               const base::KVPoolView& pool, const int32_t* slot_mapping, int32_t block_size,
               int32_t num_kv_heads, int32_t head_size, int32_t batch_tokens) const;
  void scatter_single_token(const void* key, const void* value, base::DataType input_dtype,
                            const base::KVPoolView& pool, int32_t physical_block_id,
                            int32_t offset_in_block, int32_t block_size, int32_t num_kv_heads,
                            int32_t head_size) const;

  int device() const { return device_; }
  void* stream() const { return stream_; }

 private:
  int device_;
  void* stream_;
};

}  // namespace model

#endif  // PBE_INCLUDE_MODEL_PAGED_KV_RUNTIME_H_
