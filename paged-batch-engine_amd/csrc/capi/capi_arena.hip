// C ABI: arenas (allocation, IPC export and import), in-process and
// interprocess events, and the cross-process completion signals.
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

}  // extern "C"
