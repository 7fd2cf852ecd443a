// Internal interface of the page writer (new tokens' K/V into page slots).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "decode_kernels.h"   // FastDiv
#include "handoff_kernels.h"  // kThreadsPerBlock

namespace pbe {

struct ScatterParams {
  const uint8_t* keys;        // [tokens][row_in_bytes], 16-byte aligned rows
  const uint8_t* values;
  uint8_t* key_pool;          // row (block, offset) at block * block_out_bytes + offset * row_out_bytes
  uint8_t* value_pool;
  uint64_t key_pool_bytes;    // rows ending beyond these are skipped
  uint64_t value_pool_bytes;
  float* key_scales;          // FP8: [block][offset][head]
  float* value_scales;
  uint64_t key_scale_count;   // floats; rows whose scale falls beyond are skipped
  uint64_t value_scale_count;
  const int32_t* slots;       // device [tokens], or null: every token takes fixed_slot
  int32_t fixed_slot;
  uint32_t units;             // tokens * 2 * vecs_per_row (< 2^31)
  uint32_t vecs_per_row;      // row_in_bytes / 16
  uint32_t row_in_bytes;
  uint32_t row_out_bytes;
  uint64_t block_out_bytes;
  uint32_t block_size;
  uint32_t kv_heads;
  FastDiv by_row_pair;        // 2 * vecs_per_row
  FastDiv by_block_size;
};

// lanes_per_head: head_dim * input bytes / 16, a power of two up to 64 (FP8 only).
hipError_t launch_scatter_kv(const ScatterParams& p, bool f32_input, bool fp8, uint32_t lanes_per_head,
                             hipStream_t stream);

}  // namespace pbe
