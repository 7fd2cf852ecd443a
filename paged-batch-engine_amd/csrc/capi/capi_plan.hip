// C ABI: host-side planning (id validation, run coalescing) and the compact
// page-list wire form. No device work.
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

using namespace pbe_capi;

extern "C" {

// ---------------------------------------------------------------- planning
int pbe_validate_ids(const int32_t* ids, int64_t n, const pbe_kv_shape* shape,
                     uint32_t elem_bytes, uint64_t arena_bytes, int64_t* bad_index) {
  if (bad_index) *bad_index = -1;
  if ((!ids && n) || n < 0 || !shape_ok(shape) || !elem_bytes)
    return fail(PBE_ERR_INVALID, "invalid id list or shape");
  const uint64_t half = half_bytes(*shape, elem_bytes);
  const int64_t stride = 2 * (int64_t)shape->layers;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t id = ids[i];
    if (id < 0 || id % stride != 0 || ((uint64_t)id + (uint64_t)stride) * half > arena_bytes) {
      if (bad_index) *bad_index = i;
      return fail(PBE_ERR_INVALID, "block id %lld at %lld outside the shared page layout",
                  (long long)id, (long long)i);
    }
  }
  return PBE_OK;
}

int pbe_build_runs(const int32_t* src_ids, const int32_t* dst_ids, int64_t n,
                   const pbe_kv_shape* shape, uint32_t elem_bytes, uint64_t segment_bytes,
                   pbe_run* out, int64_t* n_runs) {
  if (!n_runs || n < 0 || (n && (!src_ids || !dst_ids || !out)) || !shape_ok(shape) || !elem_bytes)
    return fail(PBE_ERR_INVALID, "invalid run-building arguments");
  const uint64_t half = half_bytes(*shape, elem_bytes);
  const int32_t stride = 2 * shape->layers;
  const uint64_t page_bytes = (uint64_t)stride * half;
  // A page may extend a run only if it is address-contiguous with the previous
  // page in the same segment, on both sides.
  auto same_segment = [&](int32_t prev, int32_t cur) {
    if (!segment_bytes) return true;
    return ((uint64_t)prev * half) / segment_bytes ==
           ((uint64_t)cur * half + page_bytes - 1) / segment_bytes;
  };
  int64_t runs = 0;
  for (int64_t i = 0; i < n;) {
    int64_t end = i + 1;
    while (end < n && src_ids[end] == src_ids[end - 1] + stride &&
           dst_ids[end] == dst_ids[end - 1] + stride && same_segment(src_ids[i], src_ids[end]) &&
           same_segment(dst_ids[i], dst_ids[end]))
      ++end;
    out[runs].src_block = src_ids[i];
    out[runs].dst_block = dst_ids[i];
    out[runs].pages = (int32_t)(end - i);
    ++runs;
    i = end;
  }
  *n_runs = runs;
  return PBE_OK;
}

}  // extern "C"

// ---------------------------------------------------------- page-list wire
namespace {

constexpr uint32_t kFnvBasis = 2166136261u, kFnvPrime = 16777619u;

uint32_t fnv1a(uint32_t h, const void* data, size_t n) {
  const unsigned char* p = static_cast<const unsigned char*>(data);
  for (size_t i = 0; i < n; ++i) h = (h ^ p[i]) * kFnvPrime;
  return h;
}

// Number of spans of a valid page-major list, or -1 when an id is invalid.
int64_t count_spans(const int32_t* ids, int64_t n, int32_t layers) {
  const int64_t stride = 2ll * layers;
  int64_t spans = 0;
  for (int64_t i = 0; i < n; ++i) {
    if (ids[i] < 0 || ids[i] % stride != 0) return -1;
    if (i == 0 || (int64_t)ids[i] != (int64_t)ids[i - 1] + stride) ++spans;
  }
  return spans;
}

uint32_t page_list_checksum(const pbe_page_list_header& h, const int32_t* spans, int64_t n_spans) {
  pbe_page_list_header z = h;
  z.checksum = 0;
  const uint32_t c = fnv1a(kFnvBasis, &z, sizeof(z));
  return fnv1a(c, spans, (size_t)n_spans * 2 * sizeof(int32_t));
}

}  // namespace

static_assert(sizeof(pbe_page_list_header) == 32, "wire header is 32 bytes");

extern "C" {

uint64_t pbe_page_list_bytes(const int32_t* ids, int64_t n, int32_t layers) {
  if (layers <= 0 || n < 0 || n > INT32_MAX || (n > 0 && !ids)) return 0;
  const int64_t spans = count_spans(ids, n, layers);
  if (spans < 0) return 0;
  return sizeof(pbe_page_list_header) + (uint64_t)spans * 2 * sizeof(int32_t);
}

int pbe_page_list_encode(const int32_t* ids, int64_t n, int32_t layers, uint64_t epoch, void* out,
                         uint64_t cap, uint64_t* out_bytes) {
  if (!out || !out_bytes) return fail(PBE_ERR_INVALID, "null output");
  *out_bytes = 0;
  if (layers <= 0) return fail(PBE_ERR_INVALID, "layers must be positive");
  if (n < 0 || n > INT32_MAX) return fail(PBE_ERR_INVALID, "page count %lld out of range", (long long)n);
  if (n > 0 && !ids) return fail(PBE_ERR_INVALID, "null ids");
  const int64_t n_spans = count_spans(ids, n, layers);
  if (n_spans < 0)
    return fail(PBE_ERR_INVALID, "PD source block outside shared page layout (not a page-major id)");
  const uint64_t bytes = sizeof(pbe_page_list_header) + (uint64_t)n_spans * 2 * sizeof(int32_t);
  if (cap < bytes)
    return fail(PBE_ERR_INVALID, "page list needs %llu bytes, buffer holds %llu",
                (unsigned long long)bytes, (unsigned long long)cap);
  std::vector<int32_t> spans((size_t)n_spans * 2);
  const int64_t stride = 2ll * layers;
  int64_t k = -1;
  for (int64_t i = 0; i < n; ++i) {
    if (i == 0 || (int64_t)ids[i] != (int64_t)ids[i - 1] + stride) {
      ++k;
      spans[2 * k] = ids[i];
      spans[2 * k + 1] = 0;
    }
    ++spans[2 * k + 1];
  }
  pbe_page_list_header h{};
  h.magic = PBE_PAGE_LIST_MAGIC;
  h.version = (uint16_t)PBE_PAGE_LIST_VERSION;
  h.header_bytes = (uint16_t)sizeof(pbe_page_list_header);
  h.layers = layers;
  h.n_pages = (int32_t)n;
  h.n_spans = (int32_t)n_spans;
  h.epoch = epoch;
  h.checksum = page_list_checksum(h, spans.data(), n_spans);
  unsigned char* o = static_cast<unsigned char*>(out);
  std::memcpy(o, &h, sizeof(h));
  if (n_spans) std::memcpy(o + sizeof(h), spans.data(), spans.size() * sizeof(int32_t));
  *out_bytes = bytes;
  return PBE_OK;
}

int pbe_page_list_decode(const void* data, uint64_t bytes, int32_t* ids, int64_t cap,
                         int64_t* n_pages, int32_t* layers, uint64_t* epoch) {
  if (!data || !n_pages || !layers || !epoch) return fail(PBE_ERR_INVALID, "null argument");
  pbe_page_list_header h;
  if (bytes < sizeof(h)) return fail(PBE_ERR_INVALID, "page list truncated (%llu bytes)", (unsigned long long)bytes);
  std::memcpy(&h, data, sizeof(h));
  if (h.magic != PBE_PAGE_LIST_MAGIC) return fail(PBE_ERR_INVALID, "not a page list (magic)");
  if (h.version != PBE_PAGE_LIST_VERSION || h.header_bytes != sizeof(h))
    return fail(PBE_ERR_INVALID, "unsupported page list version %u", (unsigned)h.version);
  if (h.layers <= 0 || h.n_pages < 0 || h.n_spans < 0 || h.n_spans > h.n_pages)
    return fail(PBE_ERR_INVALID, "page list header out of range");
  const uint64_t want = sizeof(h) + (uint64_t)h.n_spans * 2 * sizeof(int32_t);
  if (bytes != want)
    return fail(PBE_ERR_INVALID, "page list is %llu bytes, header says %llu",
                (unsigned long long)bytes, (unsigned long long)want);
  std::vector<int32_t> spans((size_t)h.n_spans * 2);
  if (h.n_spans)
    std::memcpy(spans.data(), static_cast<const unsigned char*>(data) + sizeof(h),
                spans.size() * sizeof(int32_t));
  if (page_list_checksum(h, spans.data(), h.n_spans) != h.checksum)
    return fail(PBE_ERR_INVALID, "page list checksum mismatch");
  const int64_t stride = 2ll * h.layers;
  int64_t total = 0;
  for (int32_t k = 0; k < h.n_spans; ++k) {
    const int64_t first = spans[2 * k], len = spans[2 * k + 1];
    if (len <= 0 || first < 0 || first % stride != 0 || first + (len - 1) * stride > INT32_MAX)
      return fail(PBE_ERR_INVALID, "page list span %d invalid", (int)k);
    total += len;
    if (total > h.n_pages) break;
  }
  if (total != h.n_pages)
    return fail(PBE_ERR_INVALID, "page list spans hold %lld pages, header says %d", (long long)total,
                (int)h.n_pages);
  *n_pages = h.n_pages;
  *layers = h.layers;
  *epoch = h.epoch;
  if (!ids) return PBE_OK;
  if (cap < h.n_pages) return fail(PBE_ERR_INVALID, "id buffer holds %lld of %d pages", (long long)cap, (int)h.n_pages);
  int64_t o = 0;
  for (int32_t k = 0; k < h.n_spans; ++k)
    for (int32_t j = 0; j < spans[2 * k + 1]; ++j) ids[o++] = (int32_t)(spans[2 * k] + j * stride);
  return PBE_OK;
}

}  // extern "C"
