// Internal interface of the decode-side paged-attention reader (one query
// token per sequence) over the page-major arena layout the handoff writes.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pbe {

constexpr int kDecodeMaxSegments = 16;
constexpr int kDecodeMaxKvMul = 8;    // query heads per KV head held in registers
constexpr int kDecodeMaxSplits = 1024;  // split weights of one row held in LDS by the combine

struct DecodeView {
  const char* base[kDecodeMaxSegments];
  uint64_t segment_bytes;
  uint64_t bytes;
};

// Division by a fixed divisor d >= 1 for numerators below 2^31:
// q = (mulhi(n, mul) + n) >> shift (round-up reciprocal method).
struct FastDiv {
  uint32_t d = 1, mul = 1, shift = 0;
};
FastDiv make_fast_div(uint32_t d);

struct DecodeParams {
  DecodeView kv;           // payload arena (FP8: int8 E4M3 planes; BF16: bf16 planes)
  const float* scales;     // FP8 only: page-major [layer][K|V][token][kv_head] fp32
  uint64_t scale_bytes;
  const uint16_t* q;       // bf16 [batch][q_heads][head_dim]
  uint16_t* out;           // bf16 [batch][q_heads][head_dim]
  const int32_t* tables;   // [batch][max_blocks] page-major block ids
  const int32_t* seq_lens; // [batch]
  float* part_acc;         // [batch][q_heads][splits][head_dim]
  float* part_m;           // [batch][q_heads][splits]
  float* part_l;           // [batch][q_heads][splits]
  int32_t batch, q_heads, kv_heads, head_dim, layers, layer, max_blocks, splits;
  uint64_t half;           // bytes of one K or V plane of one block
  int64_t v_delta;         // V rows of a block relative to its K rows (bytes): half page-major
  int64_t vscale_delta;    // V scales relative to K scales (floats): one plane page-major
  float scale;             // log2(e) / sqrt(head_dim): scores in base 2
  int32_t id_max;          // largest valid block id (rows and scales inside the pools)
  FastDiv by_stride;       // block ids per page: 2 * layers page-major, 1 for per-layer pools
  FastDiv by_seg_pages;    // divides page indices by pages per segment
  // Append form (both set or both null): bf16 [batch][kv_heads][head_dim] K and V
  // of each sequence's new token, written at its last position before it is
  // read; the payload and scale pools above are then written as well.
  const uint16_t* new_k;
  const uint16_t* new_v;
  // Append form only: writable views of the payload bases and of the scale
  // pool (the same memory as kv.base and scales).
  char* wbase[kDecodeMaxSegments];
  float* wscales;
};

// Bytes of the split-K workspace (partial outputs, maxima and sums).
uint64_t decode_workspace_bytes(int32_t batch, int32_t q_heads, int32_t head_dim, int32_t splits);

hipError_t launch_paged_decode(const DecodeParams& p, bool fp8, hipStream_t stream);

}  // namespace pbe
