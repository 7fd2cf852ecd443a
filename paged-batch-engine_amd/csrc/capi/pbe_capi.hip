// C ABI of the MI355X KV handoff: arena ownership and IPC, IPC events,
// host-side run planning and validation, device run lists and launches.
// Every entry point validates its whole input on the host before any device
// work is queued, so a rejected call never writes a destination byte.
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

#include "../kernels/decode_kernels.h"
#include "../kernels/handoff_kernels.h"
#include "../kernels/scatter_kernels.h"
#include "pbe_handoff.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(PBE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define PBE_HIP(call)                                        \
  do {                                                       \
    const hipError_t pbe_e_ = (call);                        \
    if (pbe_e_ != hipSuccess) return hip_fail(pbe_e_, #call); \
  } while (0)

// Makes `device` current for the scope and restores the caller's device.
class DeviceScope {
 public:
  explicit DeviceScope(int device) {
    if (hipGetDevice(&old_) != hipSuccess) {
      err_ = hipErrorNoDevice;
      return;
    }
    err_ = hipSetDevice(device);
  }
  ~DeviceScope() {
    if (err_ == hipSuccess) (void)hipSetDevice(old_);
  }
  hipError_t error() const { return err_; }

 private:
  int old_ = 0;
  hipError_t err_ = hipSuccess;
};

#define PBE_DEVICE_SCOPE(dev)                                          \
  DeviceScope pbe_scope_(dev);                                         \
  if (pbe_scope_.error() != hipSuccess) return hip_fail(pbe_scope_.error(), "select device")

bool shape_ok(const pbe_kv_shape* s) {
  return s && s->layers > 0 && s->kv_heads > 0 && s->head_dim > 0 && s->page_tokens > 0;
}

// half = one layer's K or V plane of one page (block_allocator.cpp:369-372).
uint64_t half_bytes(const pbe_kv_shape& s, uint32_t elem_bytes) {
  return (uint64_t)s.page_tokens * (uint64_t)s.kv_heads * (uint64_t)s.head_dim * elem_bytes;
}

bool view_ok(const pbe_arena_view* v) {
  if (!v || v->nseg == 0 || v->nseg > PBE_MAX_SEGMENTS || v->bytes == 0 || v->segment_bytes == 0)
    return false;
  if ((v->bytes + v->segment_bytes - 1) / v->segment_bytes != v->nseg) return false;
  for (uint32_t i = 0; i < v->nseg; ++i)
    if (!v->base[i]) return false;
  return true;
}

// Resolves [offset, offset+len) of a view to a device address; the span must
// lie inside one segment and inside the view.
bool resolve(const pbe_arena_view& v, uint64_t offset, uint64_t len, uint64_t* addr) {
  if (offset > v.bytes || len > v.bytes - offset) return false;
  const uint64_t seg = offset / v.segment_bytes;
  const uint64_t in_seg = offset % v.segment_bytes;
  if (seg >= v.nseg || len > v.segment_bytes - in_seg) return false;
  *addr = reinterpret_cast<uint64_t>(v.base[seg]) + in_seg;
  return true;
}

// Rejects any destination span overlapping another destination span or any
// source span (a copy must never race with itself).
bool spans_disjoint(std::vector<std::pair<uint64_t, uint64_t>> dst,
                    std::vector<std::pair<uint64_t, uint64_t>> src) {
  std::sort(dst.begin(), dst.end());
  for (size_t i = 1; i < dst.size(); ++i)
    if (dst[i].first < dst[i - 1].second) return false;
  std::sort(src.begin(), src.end());
  size_t j = 0;
  for (const auto& s : src) {
    while (j < dst.size() && dst[j].second <= s.first) ++j;
    if (j < dst.size() && dst[j].first < s.second) return false;
  }
  return true;
}

// Checks on the host that [ptr, ptr+bytes) lies inside one allocation a kernel
// on `device` may touch (device memory of that GPU, or pinned host memory), so
// a bad pointer is rejected instead of faulting the GPU. Verified allocation
// ranges are remembered in `known` for the rest of the call.
struct Range {
  uint64_t begin, end;
};

// Segments of arenas this library created or imported over IPC, per device.
// IPC mappings are device memory but need not be visible to the runtime's
// allocation-range queries, so they are recognised here first.
struct ArenaRegistry {
  std::mutex mu;
  struct Entry {
    uint64_t begin, end;
    int device;
  };
  std::vector<Entry> entries;
  void add(const void* p, uint64_t bytes, int device) {
    std::lock_guard<std::mutex> lock(mu);
    entries.push_back({reinterpret_cast<uint64_t>(p), reinterpret_cast<uint64_t>(p) + bytes, device});
  }
  void remove(const void* p) {
    std::lock_guard<std::mutex> lock(mu);
    const uint64_t b = reinterpret_cast<uint64_t>(p);
    entries.erase(std::remove_if(entries.begin(), entries.end(),
                                 [b](const Entry& e) { return e.begin == b; }),
                  entries.end());
  }
  bool contains(uint64_t p, uint64_t bytes, int device) { return device_of(p, bytes) == device; }
  // Device of the registered segment holding [p, p+bytes), or -1.
  int device_of(uint64_t p, uint64_t bytes) {
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : entries)
      if (p >= e.begin && bytes <= e.end - p && p < e.end) return e.device;
    return -1;
  }
};
ArenaRegistry& arena_registry() {
  static ArenaRegistry r;
  return r;
}

bool accessible(const void* ptr, uint64_t bytes, int device, std::vector<Range>* known) {
  const uint64_t p = reinterpret_cast<uint64_t>(ptr);
  if (!p || bytes > ~0ull - p) return false;
  for (const Range& r : *known)
    if (p >= r.begin && p + bytes <= r.end) return true;
  if (arena_registry().contains(p, bytes, device)) return true;
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<void*>(ptr)) != hipSuccess || !base) {
    (void)hipGetLastError();
    return false;
  }
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, ptr) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  const bool ok_type = (attr.type == hipMemoryTypeDevice && attr.device == device) ||
                       attr.type == hipMemoryTypeHost;
  const Range r{reinterpret_cast<uint64_t>(base), reinterpret_cast<uint64_t>(base) + size};
  if (!ok_type || p < r.begin || p + bytes > r.end) return false;
  known->push_back(r);
  return true;
}

bool view_accessible(const pbe_arena_view& v, int device, std::vector<Range>* known) {
  for (uint32_t i = 0; i < v.nseg; ++i) {
    const uint64_t len = std::min(v.segment_bytes, v.bytes - (uint64_t)i * v.segment_bytes);
    if (!accessible(v.base[i], len, device, known)) return false;
  }
  return true;
}

}  // namespace

struct pbe_arena {
  int device = 0;
  bool owner = false;
  uint64_t bytes = 0, segment_bytes = 0, epoch = 0;
  uint32_t nseg = 0;
  void* base[PBE_MAX_SEGMENTS] = {};
  uint8_t uuid[16] = {};
};

struct pbe_event {
  int device = 0;
  bool imported = false;
  bool interprocess = false;
  hipEvent_t event = nullptr;
};

struct pbe_signal {
  int device = 0;
  bool imported = false;
  void* word = nullptr;  // 8-byte sequence value at the start of a 4 KiB allocation
};

struct pbe_runlist {
  int device = 0;
  bool fp8 = false;
  bool has_scales = false;
  pbe::DevRun* runs = nullptr;  // device memory
  uint32_t n_runs = 0;
  uint32_t total_slices = 0;
  uint64_t page_bytes = 0;      // source bytes per page
  pbe_runlist_info info{};
  pbe_kv_shape kv{};
};

extern "C" {

const char* pbe_last_error(void) { return g_error.c_str(); }

const char* pbe_version(void) { return "pbe-handoff 1.0 gfx950"; }

int pbe_device_uuid(int device, uint8_t out[16]) {
  if (!out) return fail(PBE_ERR_INVALID, "null output");
  hipUUID uuid;
  PBE_HIP(hipDeviceGetUuid(&uuid, device));
  std::memcpy(out, uuid.bytes, 16);
  return PBE_OK;
}

}  // extern "C"

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

int pbe_current_device(int* device) {
  if (!device) return fail(PBE_ERR_INVALID, "null output");
  PBE_HIP(hipGetDevice(device));
  return PBE_OK;
}

// ---------------------------------------------------------------- arena
int pbe_arena_create(int device, uint64_t bytes, uint64_t segment_bytes, uint64_t epoch,
                     pbe_arena** out) {
  if (!out) return fail(PBE_ERR_INVALID, "null output");
  *out = nullptr;
  if (!bytes || !epoch) return fail(PBE_ERR_INVALID, "arena bytes and epoch must be non-zero");
  if (!segment_bytes) segment_bytes = bytes;
  if (segment_bytes % 256) return fail(PBE_ERR_INVALID, "segment size must be 256-byte aligned");
  const uint64_t nseg = (bytes + segment_bytes - 1) / segment_bytes;
  if (nseg > PBE_MAX_SEGMENTS) return fail(PBE_ERR_INVALID, "arena needs %llu > %d segments",
                                           (unsigned long long)nseg, PBE_MAX_SEGMENTS);
  PBE_DEVICE_SCOPE(device);
  pbe_arena* a = new (std::nothrow) pbe_arena;
  if (!a) return fail(PBE_ERR_NOMEM, "arena object");
  a->device = device;
  a->owner = true;
  a->bytes = bytes;
  a->segment_bytes = segment_bytes;
  a->epoch = epoch;
  a->nseg = (uint32_t)nseg;
  for (uint32_t i = 0; i < a->nseg; ++i) {
    const uint64_t len = std::min(segment_bytes, bytes - (uint64_t)i * segment_bytes);
    const hipError_t e = hipMalloc(&a->base[i], len);  // dedicated, never pool-cached
    if (e != hipSuccess) {
      for (uint32_t j = 0; j < i; ++j) (void)hipFree(a->base[j]);
      delete a;
      return hip_fail(e, "hipMalloc(arena segment)");
    }
  }
  for (uint32_t i = 0; i < a->nseg; ++i)
    arena_registry().add(a->base[i], std::min(segment_bytes, bytes - (uint64_t)i * segment_bytes), device);
  if (pbe_device_uuid(device, a->uuid) != PBE_OK) std::memset(a->uuid, 0, 16);
  *out = a;
  return PBE_OK;
}

int pbe_arena_export(const pbe_arena* a, pbe_arena_ipc* out) {
  if (!a || !out) return fail(PBE_ERR_INVALID, "null argument");
  if (!a->owner) return fail(PBE_ERR_INVALID, "only the owner exports an arena");
  PBE_DEVICE_SCOPE(a->device);
  pbe_arena_ipc ipc;
  std::memset(&ipc, 0, sizeof(ipc));
  ipc.version = 1;
  ipc.nseg = a->nseg;
  ipc.bytes = a->bytes;
  ipc.segment_bytes = a->segment_bytes;
  ipc.epoch = a->epoch;
  std::memcpy(ipc.gpu_uuid, a->uuid, 16);
  static_assert(sizeof(hipIpcMemHandle_t) <= PBE_IPC_HANDLE_BYTES, "IPC handle size");
  for (uint32_t i = 0; i < a->nseg; ++i) {
    hipIpcMemHandle_t h;
    PBE_HIP(hipIpcGetMemHandle(&h, a->base[i]));
    std::memcpy(ipc.handles[i], &h, sizeof(h));
  }
  *out = ipc;
  return PBE_OK;
}

int pbe_arena_import(const pbe_arena_ipc* ipc, int device, pbe_arena** out) {
  if (!ipc || !out) return fail(PBE_ERR_INVALID, "null argument");
  *out = nullptr;
  if (ipc->version != 1 || ipc->nseg == 0 || ipc->nseg > PBE_MAX_SEGMENTS || !ipc->bytes ||
      !ipc->segment_bytes || (ipc->bytes + ipc->segment_bytes - 1) / ipc->segment_bytes != ipc->nseg)
    return fail(PBE_ERR_INVALID, "malformed arena IPC descriptor");
  uint8_t uuid[16];
  int rc = pbe_device_uuid(device, uuid);
  if (rc != PBE_OK) return rc;
  if (std::memcmp(uuid, ipc->gpu_uuid, 16) != 0)
    return fail(PBE_ERR_INVALID, "arena owner and importer GPU UUID differ");
  PBE_DEVICE_SCOPE(device);
  pbe_arena* a = new (std::nothrow) pbe_arena;
  if (!a) return fail(PBE_ERR_NOMEM, "arena object");
  a->device = device;
  a->owner = false;
  a->bytes = ipc->bytes;
  a->segment_bytes = ipc->segment_bytes;
  a->epoch = ipc->epoch;
  a->nseg = ipc->nseg;
  std::memcpy(a->uuid, uuid, 16);
  for (uint32_t i = 0; i < a->nseg; ++i) {
    hipIpcMemHandle_t h;
    std::memcpy(&h, ipc->handles[i], sizeof(h));
    const hipError_t e = hipIpcOpenMemHandle(&a->base[i], h, hipIpcMemLazyEnablePeerAccess);
    if (e != hipSuccess) {
      for (uint32_t j = 0; j < i; ++j) (void)hipIpcCloseMemHandle(a->base[j]);
      delete a;
      return hip_fail(e, "hipIpcOpenMemHandle(arena segment)");
    }
  }
  for (uint32_t i = 0; i < a->nseg; ++i)
    arena_registry().add(a->base[i],
                         std::min(a->segment_bytes, a->bytes - (uint64_t)i * a->segment_bytes), device);
  *out = a;
  return PBE_OK;
}

int pbe_arena_get_view(const pbe_arena* a, pbe_arena_view* out) {
  if (!a || !out) return fail(PBE_ERR_INVALID, "null argument");
  std::memset(out, 0, sizeof(*out));
  out->bytes = a->bytes;
  out->segment_bytes = a->segment_bytes;
  out->nseg = a->nseg;
  for (uint32_t i = 0; i < a->nseg; ++i) out->base[i] = a->base[i];
  return PBE_OK;
}

uint64_t pbe_arena_epoch(const pbe_arena* a) { return a ? a->epoch : 0; }

int pbe_arena_destroy(pbe_arena* a) {
  if (!a) return PBE_OK;
  PBE_DEVICE_SCOPE(a->device);
  int rc = PBE_OK;
  for (uint32_t i = 0; i < a->nseg; ++i) {
    if (!a->base[i]) continue;
    arena_registry().remove(a->base[i]);
    const hipError_t e = a->owner ? hipFree(a->base[i]) : hipIpcCloseMemHandle(a->base[i]);
    if (e != hipSuccess) rc = hip_fail(e, a->owner ? "hipFree(arena)" : "hipIpcCloseMemHandle");
  }
  delete a;
  return rc;
}

// ---------------------------------------------------------------- events
namespace {
// Whether this runtime can record hipEventInterprocess events. ROCm 7.2 on
// MI355X creates them but rejects hipEventRecord with hipErrorInvalidValue, so
// they cannot carry a completion; the answer is probed once per device.
bool interprocess_events_work(int device) {
  static std::mutex mu;
  static int known[64] = {};  // 0 unknown, 1 yes, -1 no
  std::lock_guard<std::mutex> lock(mu);
  int& k = known[device & 63];
  if (k == 0) {
    hipEvent_t e = nullptr;
    bool ok = hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventInterprocess) == hipSuccess;
    ok = ok && hipEventRecord(e, nullptr) == hipSuccess && hipEventSynchronize(e) == hipSuccess;
    if (e) (void)hipEventDestroy(e);
    (void)hipGetLastError();
    k = ok ? 1 : -1;
  }
  return k > 0;
}
}  // namespace

int pbe_event_create(int device, int interprocess, pbe_event** out) {
  if (!out) return fail(PBE_ERR_INVALID, "null output");
  *out = nullptr;
  PBE_DEVICE_SCOPE(device);
  if (interprocess && !interprocess_events_work(device))
    return fail(PBE_ERR_UNSUPPORTED,
                "this HIP runtime cannot record interprocess events; use pbe_signal_* for "
                "cross-process completion");
  pbe_event* ev = new (std::nothrow) pbe_event;
  if (!ev) return fail(PBE_ERR_NOMEM, "event object");
  ev->device = device;
  ev->interprocess = interprocess != 0;
  const unsigned flags =
      hipEventDisableTiming | (interprocess ? (unsigned)hipEventInterprocess : 0u);
  const hipError_t e = hipEventCreateWithFlags(&ev->event, flags);
  if (e != hipSuccess) {
    delete ev;
    return hip_fail(e, "hipEventCreateWithFlags");
  }
  *out = ev;
  return PBE_OK;
}

int pbe_event_export(const pbe_event* ev, uint8_t out[PBE_IPC_HANDLE_BYTES]) {
  if (!ev || !out) return fail(PBE_ERR_INVALID, "null argument");
  if (!ev->interprocess) return fail(PBE_ERR_INVALID, "only interprocess events are exported");
  static_assert(sizeof(hipIpcEventHandle_t) <= PBE_IPC_HANDLE_BYTES, "event handle size");
  PBE_DEVICE_SCOPE(ev->device);
  hipIpcEventHandle_t h;
  PBE_HIP(hipIpcGetEventHandle(&h, ev->event));
  std::memset(out, 0, PBE_IPC_HANDLE_BYTES);
  std::memcpy(out, &h, sizeof(h));
  return PBE_OK;
}

int pbe_event_import(const uint8_t handle[PBE_IPC_HANDLE_BYTES], int device, pbe_event** out) {
  if (!handle || !out) return fail(PBE_ERR_INVALID, "null argument");
  *out = nullptr;
  PBE_DEVICE_SCOPE(device);
  if (!interprocess_events_work(device))
    return fail(PBE_ERR_UNSUPPORTED,
                "this HIP runtime cannot record interprocess events; use pbe_signal_* for "
                "cross-process completion");
  pbe_event* ev = new (std::nothrow) pbe_event;
  if (!ev) return fail(PBE_ERR_NOMEM, "event object");
  ev->device = device;
  ev->imported = true;
  ev->interprocess = true;
  hipIpcEventHandle_t h;
  std::memcpy(&h, handle, sizeof(h));
  const hipError_t e = hipIpcOpenEventHandle(&ev->event, h);
  if (e != hipSuccess) {
    delete ev;
    return hip_fail(e, "hipIpcOpenEventHandle");
  }
  *out = ev;
  return PBE_OK;
}

int pbe_event_record(pbe_event* ev, void* stream) {
  if (!ev) return fail(PBE_ERR_INVALID, "null event");
  PBE_DEVICE_SCOPE(ev->device);
  PBE_HIP(hipEventRecord(ev->event, static_cast<hipStream_t>(stream)));
  return PBE_OK;
}

int pbe_event_wait(pbe_event* ev, void* stream) {
  if (!ev) return fail(PBE_ERR_INVALID, "null event");
  PBE_DEVICE_SCOPE(ev->device);
  PBE_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(stream), ev->event, 0));
  return PBE_OK;
}

int pbe_event_query(pbe_event* ev) {
  if (!ev) return fail(PBE_ERR_INVALID, "null event");
  PBE_DEVICE_SCOPE(ev->device);
  const hipError_t e = hipEventQuery(ev->event);
  if (e == hipSuccess) return PBE_OK;
  if (e == hipErrorNotReady) return PBE_NOT_READY;
  fail(PBE_ERR_UNKNOWN, "hipEventQuery: %s", hipGetErrorString(e));
  return PBE_ERR_UNKNOWN;
}

int pbe_event_synchronize(pbe_event* ev) {
  if (!ev) return fail(PBE_ERR_INVALID, "null event");
  PBE_DEVICE_SCOPE(ev->device);
  const hipError_t e = hipEventSynchronize(ev->event);
  if (e != hipSuccess) return fail(PBE_ERR_UNKNOWN, "hipEventSynchronize: %s", hipGetErrorString(e));
  return PBE_OK;
}

int pbe_event_destroy(pbe_event* ev) {
  if (!ev) return PBE_OK;
  PBE_DEVICE_SCOPE(ev->device);
  const hipError_t e = hipEventDestroy(ev->event);
  delete ev;
  if (e != hipSuccess) return hip_fail(e, "hipEventDestroy");
  return PBE_OK;
}

// ---------------------------------------------------------------- signals
int pbe_signal_create(int device, pbe_signal** out) {
  if (!out) return fail(PBE_ERR_INVALID, "null output");
  *out = nullptr;
  PBE_DEVICE_SCOPE(device);
  pbe_signal* sg = new (std::nothrow) pbe_signal;
  if (!sg) return fail(PBE_ERR_NOMEM, "signal object");
  sg->device = device;
  hipError_t e = hipMalloc(&sg->word, 4096);
  if (e == hipSuccess) e = hipMemset(sg->word, 0, 4096);
  if (e != hipSuccess) {
    if (sg->word) (void)hipFree(sg->word);
    delete sg;
    return hip_fail(e, "signal allocation");
  }
  *out = sg;
  return PBE_OK;
}

int pbe_signal_export(const pbe_signal* sg, uint8_t out[PBE_IPC_HANDLE_BYTES]) {
  if (!sg || !out) return fail(PBE_ERR_INVALID, "null argument");
  if (sg->imported) return fail(PBE_ERR_INVALID, "only the creator exports a signal");
  PBE_DEVICE_SCOPE(sg->device);
  hipIpcMemHandle_t h;
  PBE_HIP(hipIpcGetMemHandle(&h, sg->word));
  std::memset(out, 0, PBE_IPC_HANDLE_BYTES);
  std::memcpy(out, &h, sizeof(h));
  return PBE_OK;
}

int pbe_signal_import(const uint8_t handle[PBE_IPC_HANDLE_BYTES], int device, pbe_signal** out) {
  if (!handle || !out) return fail(PBE_ERR_INVALID, "null argument");
  *out = nullptr;
  PBE_DEVICE_SCOPE(device);
  pbe_signal* sg = new (std::nothrow) pbe_signal;
  if (!sg) return fail(PBE_ERR_NOMEM, "signal object");
  sg->device = device;
  sg->imported = true;
  hipIpcMemHandle_t h;
  std::memcpy(&h, handle, sizeof(h));
  const hipError_t e = hipIpcOpenMemHandle(&sg->word, h, hipIpcMemLazyEnablePeerAccess);
  if (e != hipSuccess) {
    delete sg;
    return hip_fail(e, "hipIpcOpenMemHandle(signal)");
  }
  *out = sg;
  return PBE_OK;
}

int pbe_signal_set(pbe_signal* sg, uint64_t value, void* stream) {
  if (!sg) return fail(PBE_ERR_INVALID, "null signal");
  PBE_DEVICE_SCOPE(sg->device);
  PBE_HIP(hipStreamWriteValue64(static_cast<hipStream_t>(stream), sg->word, value, 0));
  return PBE_OK;
}

int pbe_signal_wait(pbe_signal* sg, uint64_t value, void* stream) {
  if (!sg) return fail(PBE_ERR_INVALID, "null signal");
  PBE_DEVICE_SCOPE(sg->device);
  PBE_HIP(hipStreamWaitValue64(static_cast<hipStream_t>(stream), sg->word, value,
                               hipStreamWaitValueGte, ~0ull));
  return PBE_OK;
}

int pbe_signal_read(pbe_signal* sg, uint64_t* value) {
  if (!sg || !value) return fail(PBE_ERR_INVALID, "null argument");
  PBE_DEVICE_SCOPE(sg->device);
  PBE_HIP(hipMemcpy(value, sg->word, sizeof(uint64_t), hipMemcpyDeviceToHost));
  return PBE_OK;
}

int pbe_signal_destroy(pbe_signal* sg) {
  if (!sg) return PBE_OK;
  PBE_DEVICE_SCOPE(sg->device);
  const hipError_t e = sg->imported ? hipIpcCloseMemHandle(sg->word) : hipFree(sg->word);
  delete sg;
  if (e != hipSuccess) return hip_fail(e, "signal release");
  return PBE_OK;
}

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

// ---------------------------------------------------------------- run lists
namespace {

struct Resolved {
  std::vector<pbe::DevRun> runs;
  pbe_runlist_info info{};
};

// Builds device run entries for either kernel. src pages are src_page_bytes
// long in the src view, dst pages dst_page_bytes long in the dst view;
// scale pages (FP8) scale_page_bytes long at scales.
int resolve_runs(const pbe_arena_view& src, const pbe_arena_view& dst, uint64_t src_half,
                 uint64_t dst_half, int32_t stride, const pbe_run* runs, int64_t n_runs,
                 uint64_t scales, uint64_t scales_bytes, uint64_t scale_page_bytes,
                 uint32_t slice, Resolved* out) {
  if (n_runs <= 0 || n_runs > 0x7fffffff) return fail(PBE_ERR_INVALID, "run count out of range");
  const uint64_t src_page = (uint64_t)stride * src_half;
  const uint64_t dst_page = (uint64_t)stride * dst_half;
  std::vector<std::pair<uint64_t, uint64_t>> dst_spans, src_spans;
  out->runs.resize((size_t)n_runs);
  uint64_t slices = 0;
  for (int64_t i = 0; i < n_runs; ++i) {
    const pbe_run& r = runs[i];
    if (r.src_block < 0 || r.dst_block < 0 || r.pages <= 0 || r.src_block % stride ||
        r.dst_block % stride)
      return fail(PBE_ERR_INVALID, "run %lld: ids must be non-negative page ids, pages > 0",
                  (long long)i);
    pbe::DevRun d{};
    const uint64_t sb = (uint64_t)r.pages * src_page, db = (uint64_t)r.pages * dst_page;
    if (!resolve(src, (uint64_t)r.src_block * src_half, sb, &d.src))
      return fail(PBE_ERR_INVALID, "run %lld: source span outside one arena segment", (long long)i);
    if (!resolve(dst, (uint64_t)r.dst_block * dst_half, db, &d.dst))
      return fail(PBE_ERR_INVALID, "run %lld: destination span outside one arena segment",
                  (long long)i);
    if (scale_page_bytes) {
      const uint64_t off = (uint64_t)(r.dst_block / stride) * scale_page_bytes;
      const uint64_t len = (uint64_t)r.pages * scale_page_bytes;
      if (off > scales_bytes || len > scales_bytes - off)
        return fail(PBE_ERR_INVALID, "run %lld: scale span outside the scale pool", (long long)i);
      d.aux = scales + off;
      dst_spans.emplace_back(d.aux, d.aux + len);
    }
    d.pages = (uint32_t)r.pages;
    d.slice_begin = (uint32_t)slices;
    slices += (sb + slice - 1) / slice;
    if (slices > 0xfffffff0ull) return fail(PBE_ERR_INVALID, "run list too large for one launch");
    src_spans.emplace_back(d.src, d.src + sb);
    dst_spans.emplace_back(d.dst, d.dst + db);
    out->info.src_bytes += sb;
    out->info.dst_bytes += db;
    out->info.pages += r.pages;
    if (scale_page_bytes) out->info.scale_bytes += (uint64_t)r.pages * scale_page_bytes;
    out->runs[(size_t)i] = d;
  }
  if (!spans_disjoint(dst_spans, src_spans))
    return fail(PBE_ERR_INVALID, "run list writes a byte twice or overwrites its own source");
  out->info.runs = n_runs;
  out->info.slices = slices;
  return PBE_OK;
}

int upload_runlist(Resolved& res, int device, bool fp8, bool has_scales, uint64_t page_bytes,
                   const pbe_kv_shape& kv, pbe_runlist** out) {
  PBE_DEVICE_SCOPE(device);
  pbe_runlist* list = new (std::nothrow) pbe_runlist;
  if (!list) return fail(PBE_ERR_NOMEM, "run list object");
  const size_t bytes = res.runs.size() * sizeof(pbe::DevRun);
  hipError_t e = hipMalloc(&list->runs, bytes);
  if (e == hipSuccess) e = hipMemcpy(list->runs, res.runs.data(), bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    if (list->runs) (void)hipFree(list->runs);
    delete list;
    return hip_fail(e, "upload run list");
  }
  list->device = device;
  list->fp8 = fp8;
  list->has_scales = has_scales;
  list->n_runs = (uint32_t)res.runs.size();
  list->total_slices = (uint32_t)res.info.slices;
  list->page_bytes = page_bytes;
  list->info = res.info;
  list->kv = kv;
  *out = list;
  return PBE_OK;
}

}  // namespace

extern "C" {

int pbe_runlist_create(const pbe_arena_view* src, const pbe_arena_view* dst, const pbe_run* runs,
                       int64_t n_runs, const pbe_kv_shape* shape, uint32_t elem_bytes, int device,
                       pbe_runlist** out) {
  if (!out) return fail(PBE_ERR_INVALID, "null output");
  *out = nullptr;
  if (!view_ok(src) || !view_ok(dst) || !runs || !shape_ok(shape) || !elem_bytes)
    return fail(PBE_ERR_INVALID, "invalid arena view, run list or shape");
  const uint64_t half = half_bytes(*shape, elem_bytes);
  if (half % 16) return fail(PBE_ERR_INVALID, "half-plane bytes must be a multiple of 16");
  {
    PBE_DEVICE_SCOPE(device);
    std::vector<Range> known;
    if (!view_accessible(*src, device, &known) || !view_accessible(*dst, device, &known))
      return fail(PBE_ERR_INVALID, "arena view is not device memory of device %d", device);
  }
  Resolved res;
  int rc = resolve_runs(*src, *dst, half, half, 2 * shape->layers, runs, n_runs, 0, 0, 0,
                        pbe::kCopySliceBytes, &res);
  if (rc != PBE_OK) return rc;
  return upload_runlist(res, device, false, false, 2ull * shape->layers * half, *shape, out);
}

int pbe_runlist_create_fp8(const pbe_arena_view* src, const pbe_arena_view* dst, void* dst_scales,
                           uint64_t dst_scales_bytes, const pbe_run* runs, int64_t n_runs,
                           const pbe_kv_shape* shape, int device, pbe_runlist** out) {
  if (!out) return fail(PBE_ERR_INVALID, "null output");
  *out = nullptr;
  if (!view_ok(src) || !view_ok(dst) || !runs || !shape_ok(shape))
    return fail(PBE_ERR_INVALID, "invalid arena view, run list or shape");
  const uint32_t lanes = (uint32_t)shape->head_dim / 8u;
  if (shape->head_dim % 8 || lanes == 0 || lanes > 64 || (lanes & (lanes - 1)))
    return fail(PBE_ERR_UNSUPPORTED, "FP8 handoff needs head_dim = 8 * 2^k <= 512");
  const uint64_t half16 = half_bytes(*shape, 2), half8 = half_bytes(*shape, 1);
  const uint64_t rows = (uint64_t)shape->page_tokens * shape->kv_heads;
  const uint64_t scale_page = dst_scales ? 2ull * shape->layers * rows * 4u : 0;
  if (dst_scales && (reinterpret_cast<uint64_t>(dst_scales) % 4))
    return fail(PBE_ERR_INVALID, "scale pool must be 4-byte aligned");
  if (half16 % 16) return fail(PBE_ERR_INVALID, "half-plane bytes must be a multiple of 16");
  {
    PBE_DEVICE_SCOPE(device);
    std::vector<Range> known;
    if (!view_accessible(*src, device, &known) || !view_accessible(*dst, device, &known) ||
        (dst_scales && !accessible(dst_scales, dst_scales_bytes, device, &known)))
      return fail(PBE_ERR_INVALID, "arena view or scale pool is not memory of device %d", device);
  }
  Resolved res;
  int rc = resolve_runs(*src, *dst, half16, half8, 2 * shape->layers, runs, n_runs,
                        reinterpret_cast<uint64_t>(dst_scales), dst_scales_bytes, scale_page,
                        pbe::kFp8SliceBytes, &res);
  if (rc != PBE_OK) return rc;
  return upload_runlist(res, device, true, dst_scales != nullptr, 2ull * shape->layers * half16,
                        *shape, out);
}

int pbe_runlist_get_info(const pbe_runlist* list, pbe_runlist_info* out) {
  if (!list || !out) return fail(PBE_ERR_INVALID, "null argument");
  *out = list->info;
  return PBE_OK;
}

int pbe_runlist_destroy(pbe_runlist* list) {
  if (!list) return PBE_OK;
  PBE_DEVICE_SCOPE(list->device);
  const hipError_t e = hipFree(list->runs);
  delete list;
  if (e != hipSuccess) return hip_fail(e, "hipFree(run list)");
  return PBE_OK;
}

int pbe_handoff_copy_timed(const pbe_runlist* list, void* stream, void* start_event,
                           void* stop_event) {
  if (!list) return fail(PBE_ERR_INVALID, "null run list");
  if (list->fp8) return fail(PBE_ERR_INVALID, "FP8 run list passed to the BF16 copy");
  PBE_DEVICE_SCOPE(list->device);
  const pbe::LaunchEvents ev{static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event)};
  PBE_HIP(pbe::launch_copy_runs(list->runs, list->n_runs, list->total_slices, list->page_bytes, ev,
                                static_cast<hipStream_t>(stream)));
  return PBE_OK;
}

int pbe_handoff_copy(const pbe_runlist* list, void* stream) {
  return pbe_handoff_copy_timed(list, stream, nullptr, nullptr);
}

int pbe_handoff_copy_fp8(const pbe_runlist* list, int scale_mode, const float* amax_table,
                         void* stream) {
  return pbe_handoff_copy_fp8_timed(list, scale_mode, amax_table, stream, nullptr, nullptr);
}

int pbe_handoff_copy_fp8_timed(const pbe_runlist* list, int scale_mode, const float* amax_table,
                               void* stream, void* start_event, void* stop_event) {
  if (!list) return fail(PBE_ERR_INVALID, "null run list");
  if (!list->fp8) return fail(PBE_ERR_INVALID, "BF16 run list passed to the FP8 copy");
  if (scale_mode == PBE_FP8_SCALE_PER_TOKEN_HEAD && !list->has_scales)
    return fail(PBE_ERR_INVALID, "per-token-head scales need a scale pool");
  if (scale_mode == PBE_FP8_SCALE_TABLE && !amax_table)
    return fail(PBE_ERR_INVALID, "table mode needs an amax table");
  if (scale_mode != PBE_FP8_SCALE_PER_TOKEN_HEAD && scale_mode != PBE_FP8_SCALE_TABLE)
    return fail(PBE_ERR_INVALID, "unknown scale mode %d", scale_mode);
  PBE_DEVICE_SCOPE(list->device);
  const pbe_kv_shape& kv = list->kv;
  const uint32_t rows_per_plane = (uint32_t)(kv.page_tokens * kv.kv_heads);
  const pbe::LaunchEvents ev{static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event)};
  PBE_HIP(pbe::launch_copy_runs_fp8(
      list->runs, list->n_runs, list->total_slices, list->page_bytes, (uint32_t)kv.head_dim / 8u,
      rows_per_plane, (uint32_t)kv.kv_heads, rows_per_plane * 2u * (uint32_t)kv.layers,
      scale_mode == PBE_FP8_SCALE_TABLE, amax_table, ev, static_cast<hipStream_t>(stream)));
  return PBE_OK;
}

}  // extern "C"

// ---------------------------------------------------------------- one-call forms
namespace {

// Per-device ring of pinned staging + device buffers for the one-call entry
// points. A slot is reused only after the launch that read it has completed,
// so back-to-back calls block the host only when the whole ring is in flight.
constexpr int kStagingSlots = 4;

struct StagingSlot {
  void* host = nullptr;
  void* dev = nullptr;
  size_t cap = 0;
  hipEvent_t done = nullptr;
  bool pending = false;
};

struct Staging {
  std::mutex mu;
  StagingSlot slots[kStagingSlots];
  int next = 0;
};

Staging& staging_for(int device) {
  static Staging per_device[64];
  return per_device[device & 63];
}

// Copies `bytes` of `data` into the next ring slot's device buffer, ordered on
// `stream`, and returns the slot. Caller holds st.mu and calls stage_done()
// after the launch that reads the buffer.
int stage(Staging& st, const void* data, size_t bytes, hipStream_t stream, StagingSlot** slot_out,
          void** dev_out) {
  StagingSlot& sl = st.slots[st.next];
  st.next = (st.next + 1) % kStagingSlots;
  if (sl.pending) {
    PBE_HIP(hipEventSynchronize(sl.done));
    sl.pending = false;
  }
  if (bytes > sl.cap) {
    if (sl.host) (void)hipHostFree(sl.host);
    if (sl.dev) (void)hipFree(sl.dev);
    sl.host = sl.dev = nullptr;
    sl.cap = 0;
    size_t cap = 4096;
    while (cap < bytes) cap *= 2;
    PBE_HIP(hipHostMalloc(&sl.host, cap, hipHostMallocDefault));
    PBE_HIP(hipMalloc(&sl.dev, cap));
    sl.cap = cap;
  }
  if (!sl.done) PBE_HIP(hipEventCreateWithFlags(&sl.done, hipEventDisableTiming));
  std::memcpy(sl.host, data, bytes);
  PBE_HIP(hipMemcpyAsync(sl.dev, sl.host, bytes, hipMemcpyHostToDevice, stream));
  *slot_out = &sl;
  *dev_out = sl.dev;
  return PBE_OK;
}

// The staging ring reuses its buffers after four calls: a graph captured with
// a staged list would replay stale or freed memory, so staged calls refuse a
// stream that is being captured (prebuilt run lists are the capturable form).
int refuse_capture(hipStream_t stream, const char* what) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  PBE_HIP(hipStreamIsCapturing(stream, &status));
  if (status != hipStreamCaptureStatusNone)
    return fail(PBE_ERR_UNSUPPORTED,
                "%s stages its list per call and cannot be captured into a graph; capture "
                "pbe_handoff_copy with a prebuilt run list instead", what);
  return PBE_OK;
}

int stage_done(StagingSlot& sl, hipStream_t stream) {
  PBE_HIP(hipEventRecord(sl.done, stream));
  sl.pending = true;
  return PBE_OK;
}

}  // namespace

extern "C" {

int pbe_copy_shared_kv(const pbe_arena_view* arena, const int32_t* src_ids, const int32_t* dst_ids,
                       int64_t n, const pbe_kv_shape* shape, int device, void* stream,
                       uint64_t* copied) {
  if (copied) *copied = 0;
  if (!view_ok(arena) || !shape_ok(shape) || n <= 0 || !src_ids || !dst_ids || device < 0)
    return fail(PBE_ERR_INVALID, "invalid handoff arguments");
  int64_t bad = -1;
  int rc = pbe_validate_ids(src_ids, n, shape, 2, arena->bytes, &bad);
  if (rc != PBE_OK) return rc;
  rc = pbe_validate_ids(dst_ids, n, shape, 2, arena->bytes, &bad);
  if (rc != PBE_OK) return rc;
  std::vector<pbe_run> runs((size_t)n);
  int64_t n_runs = 0;
  rc = pbe_build_runs(src_ids, dst_ids, n, shape, 2, arena->nseg > 1 ? arena->segment_bytes : 0,
                      runs.data(), &n_runs);
  if (rc != PBE_OK) return rc;
  const uint64_t half = half_bytes(*shape, 2);
  if (half % 16) return fail(PBE_ERR_INVALID, "half-plane bytes must be a multiple of 16");
  {
    PBE_DEVICE_SCOPE(device);
    std::vector<Range> known;
    if (!view_accessible(*arena, device, &known))
      return fail(PBE_ERR_INVALID, "arena view is not device memory of device %d", device);
  }
  Resolved res;
  rc = resolve_runs(*arena, *arena, half, half, 2 * shape->layers, runs.data(), n_runs, 0, 0, 0,
                    pbe::kCopySliceBytes, &res);
  if (rc != PBE_OK) return rc;
  PBE_DEVICE_SCOPE(device);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if ((uint64_t)n_runs <= pbe::kKernargRuns) {
    // Short lists ride in the kernel arguments: no staging copy, no fence.
    pbe::KernargRunList list{};
    list.n_runs = (uint32_t)n_runs;
    list.total_slices = (uint32_t)res.info.slices;
    list.page_bytes = 2ull * shape->layers * half;
    std::memcpy(list.runs, res.runs.data(), res.runs.size() * sizeof(pbe::DevRun));
    PBE_HIP(pbe::launch_copy_runs_kernarg(list, s));
    if (copied) *copied = res.info.src_bytes;
    return PBE_OK;
  }
  rc = refuse_capture(s, "pbe_copy_shared_kv with more than 112 runs");
  if (rc != PBE_OK) return rc;
  Staging& st = staging_for(device);
  std::lock_guard<std::mutex> lock(st.mu);
  void* dev = nullptr;
  StagingSlot* slot = nullptr;
  rc = stage(st, res.runs.data(), res.runs.size() * sizeof(pbe::DevRun), s, &slot, &dev);
  if (rc != PBE_OK) return rc;
  PBE_HIP(pbe::launch_copy_runs(static_cast<const pbe::DevRun*>(dev), (uint32_t)n_runs,
                                (uint32_t)res.info.slices, 2ull * shape->layers * half,
                                pbe::LaunchEvents{}, s));
  rc = stage_done(*slot, s);
  if (rc != PBE_OK) return rc;
  if (copied) *copied = res.info.src_bytes;
  return PBE_OK;
}

int32_t pbe_paged_decode_splits(int32_t batch, int32_t kv_heads, int32_t max_blocks_per_seq,
                                int32_t kv_dtype) {
  if (batch <= 0 || kv_heads <= 0 || max_blocks_per_seq <= 0) return 1;
  // One wave per SIMD (4 per CU) of the current GPU, rounded down so no
  // partial extra round of waves trails the launch; FP8 pages take two per
  // SIMD when every split still holds at least 16 blocks; at least 4 blocks
  // (64 tokens) per split. Measured on MI355X (256 CUs), 5040-token
  // sequences, both launches: FP8 batch 64 at 16 splits 35.7 us stage 1
  // against 40.9 us at 8; batch 128: 8 splits 66.7 us against 74.5 us at 4;
  // batch 32: 16 splits 28.9 us against 30.8 us at 32; batch 16: 32 splits
  // 22.9 us against 27.9 us at 64. BF16 batch 64: 54.6 us stage 1 at 8
  // splits against 56.5 us at 16.
  const int64_t simds = 4ll * decode_cus();
  const int64_t units = (int64_t)batch * kv_heads;
  int64_t splits = std::max<int64_t>(1, simds / units);
  if (kv_dtype == PBE_KV_FP8_E4M3) {
    const int64_t two = std::max<int64_t>(1, 2 * simds / units);
    if ((max_blocks_per_seq + two - 1) / two >= 16) splits = two;
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

int scratch_address(int device, void** out) {
  static std::mutex mu;
  static void* per_device[64] = {};
  if (device < 0 || device >= 64) return fail(PBE_ERR_INVALID, "device %d out of range", device);
  std::lock_guard<std::mutex> lock(mu);
  if (!per_device[device]) {
    PBE_DEVICE_SCOPE(device);
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    per_device[device] = ptr;
  }
  *out = per_device[device];
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
                      const DecodePools* pools = nullptr) {
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
        (!static_scratch && !accessible(workspace, need, device, &known)))
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
  void* ws = nullptr;
  const int rc = scratch_address(device, &ws);
  if (rc != PBE_OK) return rc;
  return paged_decode_call(kv, kv_dtype, scales, scale_bytes, shape, layer, queries, outputs, batch,
                           q_heads, block_tables, seq_lens, max_blocks_per_seq, splits, ws,
                           PBE_DECODE_SCRATCH_BYTES, device, stream, true);
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

}  // extern "C"

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

int pbe_copy_ops(const pbe_copy_op* ops, int64_t n_ops, int device, void* stream) {
  if (n_ops < 0 || (n_ops && !ops) || n_ops > 0x7fffffff)
    return fail(PBE_ERR_INVALID, "invalid op list");
  if (!n_ops) return PBE_OK;
  PBE_DEVICE_SCOPE(device);
  // Every op's endpoints are checked as given; then ops that continue the
  // previous one on both sides (the 2L component copies of one page, and
  // consecutive pages of a run, in a bound manifest) are merged, so the
  // overlap check, the staging and the kernel see runs instead of planes.
  std::vector<pbe_copy_op> merged;
  {
    std::vector<Range> known;
    for (int64_t i = 0; i < n_ops; ++i) {
      const pbe_copy_op& o = ops[i];
      if (!o.src || !o.dst || !o.bytes)
        return fail(PBE_ERR_INVALID, "op %lld: null pointer or zero bytes", (long long)i);
      if (o.bytes > ~0ull - o.src || o.bytes > ~0ull - o.dst)
        return fail(PBE_ERR_INVALID, "op %lld: span wraps the address space", (long long)i);
      if (!accessible(reinterpret_cast<const void*>(o.src), o.bytes, device, &known) ||
          !accessible(reinterpret_cast<const void*>(o.dst), o.bytes, device, &known))
        return fail(PBE_ERR_INVALID, "op %lld: endpoint is not device or pinned memory", (long long)i);
      if (!merged.empty()) {
        pbe_copy_op& last = merged.back();
        if (last.src + last.bytes == o.src && last.dst + last.bytes == o.dst) {
          last.bytes += o.bytes;
          continue;
        }
      }
      merged.push_back(o);
    }
  }
  {
    std::vector<std::pair<uint64_t, uint64_t>> dst, src;
    dst.reserve(merged.size());
    src.reserve(merged.size());
    for (const pbe_copy_op& o : merged) {
      dst.emplace_back(o.dst, o.dst + o.bytes);
      src.emplace_back(o.src, o.src + o.bytes);
    }
    if (!spans_disjoint(dst, src))
      return fail(PBE_ERR_INVALID, "op list writes a byte twice or overwrites its own source");
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // Spans whose addresses and sizes are all 16-byte multiples are runs of
  // 16-byte pages for the run kernel: 4 KiB per wave, one launch, and up to
  // kKernargRuns spans in the kernel arguments (no staging, so capturable).
  const bool aligned = std::all_of(merged.begin(), merged.end(), [](const pbe_copy_op& o) {
    return ((o.src | o.dst | o.bytes) & 15u) == 0 && o.bytes / 16 <= 0xffffffffull;
  });
  if (aligned) {
    std::vector<pbe::DevRun> runs(merged.size());
    uint64_t slices = 0;
    for (size_t i = 0; i < merged.size(); ++i) {
      const pbe_copy_op& o = merged[i];
      runs[i] = pbe::DevRun{o.src, o.dst, 0, (uint32_t)slices, (uint32_t)(o.bytes / 16)};
      slices += (o.bytes + pbe::kCopySliceBytes - 1) / pbe::kCopySliceBytes;
      if (slices > 0xfffffff0ull) return fail(PBE_ERR_INVALID, "op list too large for one launch");
    }
    if (runs.size() <= pbe::kKernargRuns) {
      pbe::KernargRunList list{};
      list.n_runs = (uint32_t)runs.size();
      list.total_slices = (uint32_t)slices;
      list.page_bytes = 16;
      std::memcpy(list.runs, runs.data(), runs.size() * sizeof(pbe::DevRun));
      PBE_HIP(pbe::launch_copy_runs_kernarg(list, s));
      return PBE_OK;
    }
    int rc = refuse_capture(s, "pbe_copy_ops with more than 112 spans");
    if (rc != PBE_OK) return rc;
    Staging& st = staging_for(device);
    std::lock_guard<std::mutex> lock(st.mu);
    void* dev = nullptr;
    StagingSlot* slot = nullptr;
    rc = stage(st, runs.data(), runs.size() * sizeof(pbe::DevRun), s, &slot, &dev);
    if (rc != PBE_OK) return rc;
    PBE_HIP(pbe::launch_copy_runs(static_cast<const pbe::DevRun*>(dev), (uint32_t)runs.size(),
                                  (uint32_t)slices, 16, pbe::LaunchEvents{}, s));
    return stage_done(*slot, s);
  }
  // Otherwise: split ops so that every wave moves at most kOpPieceBytes.
  std::vector<pbe::DevOp> pieces;
  for (const pbe_copy_op& o : merged)
    for (uint64_t off = 0; off < o.bytes; off += pbe::kOpPieceBytes)
      pieces.push_back({o.src + off, o.dst + off, std::min<uint64_t>(pbe::kOpPieceBytes, o.bytes - off)});
  if (pieces.size() > 0xffffffffull) return fail(PBE_ERR_INVALID, "op list too large");
  int rc = refuse_capture(s, "pbe_copy_ops with unaligned spans");
  if (rc != PBE_OK) return rc;
  Staging& st = staging_for(device);
  std::lock_guard<std::mutex> lock(st.mu);
  void* dev = nullptr;
  StagingSlot* slot = nullptr;
  rc = stage(st, pieces.data(), pieces.size() * sizeof(pbe::DevOp), s, &slot, &dev);
  if (rc != PBE_OK) return rc;
  PBE_HIP(pbe::launch_copy_ops(static_cast<const pbe::DevOp*>(dev), (uint32_t)pieces.size(), s));
  return stage_done(*slot, s);
}

// ---------------------------------------------------------------- streams
int pbe_stream_create(int device, void** out) {
  if (!out) return fail(PBE_ERR_INVALID, "null output");
  *out = nullptr;
  PBE_DEVICE_SCOPE(device);
  hipStream_t s = nullptr;
  PBE_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *out = s;
  return PBE_OK;
}

int pbe_stream_destroy(int device, void* stream) {
  if (!stream) return PBE_OK;
  PBE_DEVICE_SCOPE(device);
  PBE_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return PBE_OK;
}

int pbe_stream_synchronize(int device, void* stream) {
  PBE_DEVICE_SCOPE(device);
  const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(PBE_ERR_UNKNOWN, "hipStreamSynchronize: %s", hipGetErrorString(e));
  return PBE_OK;
}

int pbe_stream_wait_raw_event(int device, void* stream, void* hip_event) {
  if (!hip_event) return fail(PBE_ERR_INVALID, "null event");
  PBE_DEVICE_SCOPE(device);
  PBE_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(hip_event), 0));
  return PBE_OK;
}

int pbe_pointer_kind(const void* ptr, uint64_t bytes, int* kind, int* device_out) {
  if (!kind) return fail(PBE_ERR_INVALID, "null output");
  *kind = PBE_PTR_UNKNOWN;
  if (device_out) *device_out = -1;
  if (!ptr) return PBE_OK;
  const int arena_device = arena_registry().device_of(reinterpret_cast<uint64_t>(ptr), bytes);
  if (arena_device >= 0) {
    *kind = PBE_PTR_DEVICE;
    if (device_out) *device_out = arena_device;
    return PBE_OK;
  }
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<void*>(ptr)) != hipSuccess || !base) {
    (void)hipGetLastError();
    return PBE_OK;
  }
  const uint64_t p = reinterpret_cast<uint64_t>(ptr), b = reinterpret_cast<uint64_t>(base);
  if (bytes > ~0ull - p || p + bytes > b + size) return PBE_OK;
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, ptr) != hipSuccess) {
    (void)hipGetLastError();
    return PBE_OK;
  }
  if (attr.type == hipMemoryTypeDevice) {
    *kind = PBE_PTR_DEVICE;
    if (device_out) *device_out = attr.device;
  } else if (attr.type == hipMemoryTypeHost) {
    *kind = PBE_PTR_PINNED_HOST;
  }
  return PBE_OK;
}

}  // extern "C"
