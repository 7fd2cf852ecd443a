// Measurement-only kernels: HBM ceilings at the handoff's own geometry.
//
// A copy kernel moves every byte twice (one read, one write), so its rate is
// bounded by what HBM gives a pure read stream and a pure write stream of the
// same size. These two kernels are the copy kernel's halves at its geometry
// on a one-region plan (config 2): one wave per 1 KiB slice, 64 lanes x one
// 16-byte vector, 512-thread workgroups, the same
// buffer cache-policy bits (loads nt; stores sc1 + nt). bench.py times them
// on the config-2 byte count beside the handoff so the ceiling is measured in
// every run rather than asserted. They are not part of the handoff library:
// they live in lib/libpbe_ceiling.so, which only bench.py loads.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kWave = 64;
constexpr int kThreads = 256;
constexpr int kCopyThreads = 512;  // the product kernel's workgroup on a one-region plan
constexpr int kUnroll = 1;
constexpr uint32_t kSlice = kWave * 16u * kUnroll;  // 1 KiB per wave, as the product kernel on config 2
constexpr int kLoadPolicy = 0x02;                   // nt
constexpr int kStorePolicy = 0x12;                  // sc1 + nt

__global__ __launch_bounds__(kCopyThreads) void stream_read_kernel(const uint8_t* p, uint64_t bytes,
                                                               u32x4* sink) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint64_t s = (uint64_t)blockIdx.x * (kCopyThreads / kWave) + threadIdx.x / kWave;
  const uint64_t off = s * kSlice;
  if (off >= bytes) return;
  const uint64_t left = bytes - off;
  const uint32_t n = left >= kSlice ? kSlice : (uint32_t)left;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p + off), (short)0, n, 0x00020000);
  u32x4 v[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
    v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, (u * kWave + lane) * 16u, 0, kLoadPolicy);
  u32x4 acc = v[0];
#pragma unroll
  for (int u = 1; u < kUnroll; ++u) acc ^= v[u];
  // never true for the bench's data; keeps the loads alive
  if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u && acc.z == 0x85ebca6bu) sink[lane] = acc;
}

__global__ __launch_bounds__(kCopyThreads) void stream_write_kernel(uint8_t* p, uint64_t bytes,
                                                                uint32_t seed) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint64_t s = (uint64_t)blockIdx.x * (kCopyThreads / kWave) + threadIdx.x / kWave;
  const uint64_t off = s * kSlice;
  if (off >= bytes) return;
  const uint64_t left = bytes - off;
  const uint32_t n = left >= kSlice ? kSlice : (uint32_t)left;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(p + off, (short)0, n, 0x00020000);
  const u32x4 v = {seed, seed ^ lane, (uint32_t)s, (uint32_t)(s >> 32)};
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (u * kWave + lane) * 16u, 0, kStorePolicy);
}

// The copy kernel's geometry and cache policies over one contiguous span with
// no run list: wave w copies slice w. The difference to the product kernel on
// one contiguous run is the cost of finding the run.
__global__ __launch_bounds__(kCopyThreads) void slice_copy_kernel(const uint8_t* src, uint8_t* dst,
                                                              uint64_t bytes) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint64_t s = (uint64_t)blockIdx.x * (kCopyThreads / kWave) + threadIdx.x / kWave;
  const uint64_t off = s * kSlice;
  if (off >= bytes) return;
  const uint64_t left = bytes - off;
  const uint32_t n = left >= kSlice ? kSlice : (uint32_t)left;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src + off), (short)0, n, 0x00020000);
  const __amdgpu_buffer_rsrc_t rd =
      __builtin_amdgcn_make_buffer_rsrc(dst + off, (short)0, n, 0x00020000);
  u32x4 v[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
    v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, (u * kWave + lane) * 16u, 0, kLoadPolicy);
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
    __builtin_amdgcn_raw_buffer_store_b128(v[u], rd, (u * kWave + lane) * 16u, 0, kStorePolicy);
}

// Register-staged copy: each wave loads a 32 KiB chunk into VGPRs (32
// vectors per lane, two waves per SIMD), then stores all of it. Tests whether
// long read-only then write-only bursts per wave beat the copy kernel's
// short load-then-store slices (HBM pays a read/write turnaround when the two
// streams mix).
constexpr int kPhaseUnroll = 32;
constexpr uint32_t kPhaseChunk = kWave * 16u * kPhaseUnroll;  // 32 KiB per wave

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void phase_copy_kernel(const uint8_t* src, uint8_t* dst, uint64_t bytes) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint64_t c = (uint64_t)blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
  const uint64_t off = c * kPhaseChunk;
  if (off >= bytes) return;
  const uint64_t left = bytes - off;
  const uint32_t n = left >= kPhaseChunk ? kPhaseChunk : (uint32_t)left;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src + off), (short)0, n, 0x00020000);
  const __amdgpu_buffer_rsrc_t rd =
      __builtin_amdgcn_make_buffer_rsrc(dst + off, (short)0, n, 0x00020000);
  u32x4 v[kPhaseUnroll];
#pragma unroll
  for (int u = 0; u < kPhaseUnroll; ++u)
    v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, (u * kWave + lane) * 16u, 0, kLoadPolicy);
#pragma unroll
  for (int u = 0; u < kPhaseUnroll; ++u)
    __builtin_amdgcn_raw_buffer_store_b128(v[u], rd, (u * kWave + lane) * 16u, 0, kStorePolicy);
}

// Read-only streams in steps at the positions of a list (the decode reader's
// access: each wave streams its own sequence of scattered blocks), with
// kReadDepth steps in flight per wave (a ring of registers, as the reader
// keeps blocks in flight) and non-temporal loads. Wave w reads steps
// [w*steps_per_wave, (w+1)*steps_per_wave) of `order`.
//   kReaderShape false: step s is the 4 KiB at base + order[s] * 4 KiB.
//   kReaderShape true:  the FP8 reader's shape at 2 KV heads x 128 dims: step
//     s is one 8 KiB block at base + order[s] * 8 KiB (a 4 KiB K plane of
//     16 token rows x 2 heads x 128 B, then the V plane); waves 2p and 2p+1
//     read the same steps, each its own head's 128-byte half of every
//     256-byte token row (16 K rows, then 16 V rows).
// steps_per_wave = 1 gives short-lived waves; 8 and 20 the reader's
// long-lived ones.
constexpr int kReadDepth = 4;

template <bool kReaderShape>
__global__ __launch_bounds__(kThreads) void stream_read_steps_kernel(
    const uint8_t* base, const uint32_t* order, uint32_t n_steps, uint32_t steps_per_wave,
    u32x4* sink) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t w = blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
  const uint32_t list_w = kReaderShape ? w / 2 : w;
  const uint32_t s0 = __builtin_amdgcn_readfirstlane(list_w * steps_per_wave);
  if (s0 >= n_steps) return;
  const uint32_t s1 = __builtin_amdgcn_readfirstlane(min(s0 + steps_per_wave, n_steps));
  // reader shape: lane -> (token row, 16-byte piece) of this wave's head
  const uint32_t lane_off = kReaderShape ? (lane / 8) * 256u + (w & 1) * 128u + (lane % 8) * 16u
                                         : lane * 16u;
  u32x4 r[kReadDepth][4];
  u32x4 acc = {0, 0, 0, 0};
  // readfirstlane returns int: list entries are widened through uint32_t so
  // that none can sign-extend into an address
  auto load = [&](uint32_t s, u32x4* d) {
    if constexpr (kReaderShape) {
      const uint8_t* blk = base + (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(order[s]) * 8192u;
#pragma unroll
      for (int u = 0; u < 4; ++u)  // K rows 0-7, 8-15, then V rows 0-7, 8-15
        d[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
            blk + (u / 2) * 4096u + (u % 2) * 2048u + lane_off));
    } else {
      const uint8_t* st = base + (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(order[s]) * 4096u;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        d[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(st + u * 1024u + lane_off));
    }
  };
#pragma unroll
  for (int i = 0; i < kReadDepth; ++i)
    if (s0 + i < s1) load(s0 + i, r[i]);
  for (uint32_t b = s0; b < s1; b += kReadDepth) {
#pragma unroll
    for (int i = 0; i < kReadDepth; ++i) {
      if (b + i < s1) {
#pragma unroll
        for (int u = 0; u < 4; ++u) acc ^= r[i][u];
      }
      if (b + i + kReadDepth < s1) load(b + i + kReadDepth, r[i]);
    }
  }
  if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u && acc.z == 0x85ebca6bu) sink[lane] = acc;
}

// The copy kernel's one-region geometry (1 KiB slices, 512-thread
// workgroups, loads nt, stores sc1 + nt) over a contiguous source, each
// slice's destination taken from a per-slice table (a plan's destinations
// without its run lookup), with lane 0 of every wave recording the 100 MHz
// real-time counter when the wave starts, when its load has returned and when
// its store has completed: stamps[3 * s + 0..2]. A timeline of the copy: when
// the first slices complete (fill), the steady completion rate, and how the
// last ones drain.
__global__ __launch_bounds__(kCopyThreads) void timeline_copy_kernel(const uint8_t* src,
                                                                     const uint64_t* dst_of,
                                                                     uint32_t n_slices,
                                                                     uint64_t* stamps) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t s = __builtin_amdgcn_readfirstlane(blockIdx.x * (kCopyThreads / kWave) + threadIdx.x / kWave);
  if (s >= n_slices) return;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(src + (uint64_t)s * kSlice), (short)0, kSlice, 0x00020000);
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16u, 0, kLoadPolicy);
  const uint64_t dst = dst_of[s];
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
  const __amdgpu_buffer_rsrc_t rd =
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(dst), (short)0, kSlice, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(v, rd, lane * 16u, 0, kStorePolicy);
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const uint64_t t2 = __builtin_amdgcn_s_memrealtime();
  if (lane == 0) {
    stamps[3ull * s] = t0;
    stamps[3ull * s + 1] = t1;
    stamps[3ull * s + 2] = t2;
  }
}

// Nothing but the dispatch: the copy's grid and workgroup on the C2 plan.
__global__ __launch_bounds__(kCopyThreads) void empty_kernel(uint32_t n, uint32_t* sink) {
  if (n == 0xffffffffu) sink[threadIdx.x] = blockIdx.x;
}

dim3 grid_for(uint64_t bytes) {
  const uint64_t waves = (bytes + kSlice - 1) / kSlice;
  return dim3((unsigned)((waves + kCopyThreads / kWave - 1) / (kCopyThreads / kWave)));
}

}  // namespace

extern "C" {

// Reads `bytes` at p (sink: 1 KiB of device memory the kernel may write).
// start/stop may be null; otherwise they are stamped at the kernel's own
// start and end (hipExtLaunchKernel). Returns a hipError_t value.
int pbe_ceiling_read(const void* p, uint64_t bytes, void* sink, void* stream, void* start,
                     void* stop) {
  if (!p || !sink || bytes == 0 || (bytes >> 44)) return (int)hipErrorInvalidValue;
  hipExtLaunchKernelGGL(stream_read_kernel, grid_for(bytes), dim3(kCopyThreads), 0,
                        (hipStream_t)stream, (hipEvent_t)start, (hipEvent_t)stop, 0,
                        (const uint8_t*)p, bytes, (u32x4*)sink);
  return (int)hipGetLastError();
}

// Writes `bytes` at p with a pattern derived from seed.
int pbe_ceiling_write(void* p, uint64_t bytes, uint32_t seed, void* stream, void* start,
                      void* stop) {
  if (!p || bytes == 0 || (bytes >> 44)) return (int)hipErrorInvalidValue;
  hipExtLaunchKernelGGL(stream_write_kernel, grid_for(bytes), dim3(kCopyThreads), 0,
                        (hipStream_t)stream, (hipEvent_t)start, (hipEvent_t)stop, 0,
                        (uint8_t*)p, bytes, seed);
  return (int)hipGetLastError();
}

// Copies `bytes` from src to dst (contiguous, non-overlapping) with the copy
// kernel's slices and no run list.
int pbe_ceiling_slice_copy(const void* src, void* dst, uint64_t bytes, void* stream, void* start,
                           void* stop) {
  if (!src || !dst || bytes == 0 || (bytes >> 44)) return (int)hipErrorInvalidValue;
  hipExtLaunchKernelGGL(slice_copy_kernel, grid_for(bytes), dim3(kCopyThreads), 0, (hipStream_t)stream,
                        (hipEvent_t)start, (hipEvent_t)stop, 0, (const uint8_t*)src, (uint8_t*)dst,
                        bytes);
  return (int)hipGetLastError();
}

// Copies `bytes` from src to dst (contiguous, non-overlapping) with the
// register-staged kernel.
int pbe_ceiling_phase_copy(const void* src, void* dst, uint64_t bytes, void* stream, void* start,
                           void* stop) {
  if (!src || !dst || bytes == 0 || (bytes >> 44)) return (int)hipErrorInvalidValue;
  const uint64_t waves = (bytes + kPhaseChunk - 1) / kPhaseChunk;
  hipExtLaunchKernelGGL(phase_copy_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(kThreads), 0,
                        (hipStream_t)stream, (hipEvent_t)start, (hipEvent_t)stop, 0,
                        (const uint8_t*)src, (uint8_t*)dst, bytes);
  return (int)hipGetLastError();
}

// Reads n_steps steps at the positions in `order` (device uint32 list),
// steps_per_wave consecutive list entries per wave: 4 KiB contiguous steps
// (reader_shape 0, base + order[s] * 4096) or the FP8 reader's 8 KiB blocks
// read as two heads' half rows by wave pairs (reader_shape 1,
// base + order[s] * 8192).
int pbe_ceiling_read_steps(const void* base, const uint32_t* order, uint32_t n_steps,
                           uint32_t steps_per_wave, int reader_shape, void* sink, void* stream,
                           void* start, void* stop) {
  if (!base || !order || !sink || n_steps == 0 || steps_per_wave == 0)
    return (int)hipErrorInvalidValue;
  uint32_t waves = (n_steps + steps_per_wave - 1) / steps_per_wave;
  if (reader_shape) waves *= 2;
  const dim3 grid((waves + 3) / 4);
  if (reader_shape)
    hipExtLaunchKernelGGL(stream_read_steps_kernel<true>, grid, dim3(kThreads), 0,
                          (hipStream_t)stream, (hipEvent_t)start, (hipEvent_t)stop, 0,
                          (const uint8_t*)base, order, n_steps, steps_per_wave, (u32x4*)sink);
  else
    hipExtLaunchKernelGGL(stream_read_steps_kernel<false>, grid, dim3(kThreads), 0,
                          (hipStream_t)stream, (hipEvent_t)start, (hipEvent_t)stop, 0,
                          (const uint8_t*)base, order, n_steps, steps_per_wave, (u32x4*)sink);
  return (int)hipGetLastError();
}

// Timeline copy of n_slices 1 KiB slices from the contiguous src to
// dst_of[s] (device table of n_slices destination addresses); stamps: device
// buffer of 3 * n_slices uint64 (100 MHz real-time counter values).
int pbe_ceiling_timeline_copy(const void* src, const uint64_t* dst_of, uint32_t n_slices,
                              uint64_t* stamps, void* stream, void* start, void* stop) {
  if (!src || !dst_of || !stamps || n_slices == 0) return (int)hipErrorInvalidValue;
  constexpr uint32_t w = kCopyThreads / kWave;
  hipExtLaunchKernelGGL(timeline_copy_kernel, dim3((n_slices + w - 1) / w), dim3(kCopyThreads), 0,
                        (hipStream_t)stream, (hipEvent_t)start, (hipEvent_t)stop, 0,
                        (const uint8_t*)src, dst_of, n_slices, stamps);
  return (int)hipGetLastError();
}

// An empty kernel with the grid of n_slices one-slice waves in 512-thread
// workgroups: the dispatch alone.
int pbe_ceiling_empty(uint32_t n_slices, void* sink, void* stream, void* start, void* stop) {
  if (!sink || n_slices == 0) return (int)hipErrorInvalidValue;
  constexpr uint32_t w = kCopyThreads / kWave;
  hipExtLaunchKernelGGL(empty_kernel, dim3((n_slices + w - 1) / w), dim3(kCopyThreads), 0,
                        (hipStream_t)stream, (hipEvent_t)start, (hipEvent_t)stop, 0, n_slices,
                        (uint32_t*)sink);
  return (int)hipGetLastError();
}

}  // extern "C"
