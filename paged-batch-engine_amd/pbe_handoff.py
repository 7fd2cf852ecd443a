"""ctypes binding of the C ABI in include/pbe_handoff.h.

This module only marshals arguments: every computation happens in
lib/libpbe_handoff.so (HIP kernels on gfx950). Loading fails loudly when the
library is missing; there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libpbe_handoff.so"

PBE_OK = 0
PBE_NOT_READY = 1
PBE_ERR_INVALID = -1
PBE_ERR_HIP = -2
PBE_ERR_UNKNOWN = -3
PBE_ERR_NOMEM = -4
PBE_ERR_UNSUPPORTED = -5
PBE_ERR_BUSY = -6
PBE_MAX_SEGMENTS = 16
PBE_IPC_HANDLE_BYTES = 64
PBE_FP8_SCALE_PER_TOKEN_HEAD = 0
PBE_FP8_SCALE_TABLE = 1
PBE_KV_BF16 = 0
PBE_KV_FP8_E4M3 = 1


class KvShape(C.Structure):
    _fields_ = [("layers", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("page_tokens", C.c_int32)]

    def half_bytes(self, elem_bytes: int = 2) -> int:
        return self.page_tokens * self.kv_heads * self.head_dim * elem_bytes

    def page_bytes(self, elem_bytes: int = 2) -> int:
        return 2 * self.layers * self.half_bytes(elem_bytes)


class Run(C.Structure):
    _fields_ = [("src_block", C.c_int32), ("dst_block", C.c_int32), ("pages", C.c_int32)]


class ArenaView(C.Structure):
    _fields_ = [("bytes", C.c_uint64), ("segment_bytes", C.c_uint64), ("nseg", C.c_uint32),
                ("reserved", C.c_uint32), ("base", C.c_void_p * PBE_MAX_SEGMENTS)]


class ArenaIpc(C.Structure):
    _fields_ = [("version", C.c_uint32), ("nseg", C.c_uint32), ("bytes", C.c_uint64),
                ("segment_bytes", C.c_uint64), ("epoch", C.c_uint64),
                ("gpu_uuid", C.c_uint8 * 16),
                ("handles", (C.c_uint8 * PBE_IPC_HANDLE_BYTES) * PBE_MAX_SEGMENTS)]


class RunListInfo(C.Structure):
    _fields_ = [("runs", C.c_int64), ("pages", C.c_int64), ("src_bytes", C.c_uint64),
                ("dst_bytes", C.c_uint64), ("scale_bytes", C.c_uint64), ("slices", C.c_uint64)]


class CopyOp(C.Structure):
    _fields_ = [("src", C.c_uint64), ("dst", C.c_uint64), ("bytes", C.c_uint64)]


# (name, restype, argtypes) of every exported entry point of include/pbe_handoff.h
_P = C.c_void_p
_SIGNATURES = [
    ("pbe_last_error", C.c_char_p, []),
    ("pbe_version", C.c_char_p, []),
    ("pbe_device_uuid", C.c_int, [C.c_int, C.POINTER(C.c_uint8)]),
    ("pbe_current_device", C.c_int, [C.POINTER(C.c_int)]),
    ("pbe_arena_create", C.c_int, [C.c_int, C.c_uint64, C.c_uint64, C.c_uint64, C.POINTER(_P)]),
    ("pbe_arena_export", C.c_int, [_P, C.POINTER(ArenaIpc)]),
    ("pbe_arena_import", C.c_int, [C.POINTER(ArenaIpc), C.c_int, C.POINTER(_P)]),
    ("pbe_arena_get_view", C.c_int, [_P, C.POINTER(ArenaView)]),
    ("pbe_arena_epoch", C.c_uint64, [_P]),
    ("pbe_arena_destroy", C.c_int, [_P]),
    ("pbe_event_create", C.c_int, [C.c_int, C.c_int, C.POINTER(_P)]),
    ("pbe_event_export", C.c_int, [_P, C.POINTER(C.c_uint8)]),
    ("pbe_event_import", C.c_int, [C.POINTER(C.c_uint8), C.c_int, C.POINTER(_P)]),
    ("pbe_event_record", C.c_int, [_P, _P]),
    ("pbe_event_wait", C.c_int, [_P, _P]),
    ("pbe_event_query", C.c_int, [_P]),
    ("pbe_event_synchronize", C.c_int, [_P]),
    ("pbe_event_destroy", C.c_int, [_P]),
    ("pbe_signal_create", C.c_int, [C.c_int, C.POINTER(_P)]),
    ("pbe_signal_export", C.c_int, [_P, C.POINTER(C.c_uint8)]),
    ("pbe_signal_import", C.c_int, [C.POINTER(C.c_uint8), C.c_int, C.POINTER(_P)]),
    ("pbe_signal_set", C.c_int, [_P, C.c_uint64, _P]),
    ("pbe_signal_wait", C.c_int, [_P, C.c_uint64, _P]),
    ("pbe_signal_read", C.c_int, [_P, C.POINTER(C.c_uint64)]),
    ("pbe_signal_destroy", C.c_int, [_P]),
    ("pbe_validate_ids", C.c_int, [_P, C.c_int64, C.POINTER(KvShape), C.c_uint32, C.c_uint64,
                                   C.POINTER(C.c_int64)]),
    ("pbe_build_runs", C.c_int, [_P, _P, C.c_int64, C.POINTER(KvShape), C.c_uint32, C.c_uint64,
                                 C.POINTER(Run), C.POINTER(C.c_int64)]),
    ("pbe_page_list_bytes", C.c_uint64, [_P, C.c_int64, C.c_int32]),
    ("pbe_page_list_encode", C.c_int, [_P, C.c_int64, C.c_int32, C.c_uint64, _P, C.c_uint64,
                                       C.POINTER(C.c_uint64)]),
    ("pbe_page_list_decode", C.c_int, [_P, C.c_uint64, _P, C.c_int64, C.POINTER(C.c_int64),
                                       C.POINTER(C.c_int32), C.POINTER(C.c_uint64)]),
    ("pbe_runlist_create", C.c_int, [C.POINTER(ArenaView), C.POINTER(ArenaView), C.POINTER(Run),
                                     C.c_int64, C.POINTER(KvShape), C.c_uint32, C.c_int,
                                     C.POINTER(_P)]),
    ("pbe_runlist_create_fp8", C.c_int, [C.POINTER(ArenaView), C.POINTER(ArenaView), _P,
                                         C.c_uint64, C.POINTER(Run), C.c_int64,
                                         C.POINTER(KvShape), C.c_int, C.POINTER(_P)]),
    ("pbe_runlist_get_info", C.c_int, [_P, C.POINTER(RunListInfo)]),
    ("pbe_runlist_destroy", C.c_int, [_P]),
    ("pbe_handoff_copy", C.c_int, [_P, _P]),
    ("pbe_handoff_copy_fp8", C.c_int, [_P, C.c_int, _P, _P]),
    ("pbe_handoff_copy_timed", C.c_int, [_P, _P, _P, _P]),
    ("pbe_handoff_copy_fp8_timed", C.c_int, [_P, C.c_int, _P, _P, _P, _P]),
    ("pbe_copy_shared_kv", C.c_int, [C.POINTER(ArenaView), _P, _P, C.c_int64,
                                     C.POINTER(KvShape), C.c_int, _P, C.POINTER(C.c_uint64)]),
    ("pbe_copy_ops", C.c_int, [C.POINTER(CopyOp), C.c_int64, C.c_int, _P]),
    ("pbe_paged_decode_splits", C.c_int32, [C.c_int32, C.c_int32, C.c_int32, C.c_int32]),
    ("pbe_paged_decode_workspace_bytes", C.c_uint64, [C.c_int32, C.c_int32, C.c_int32, C.c_int32]),
    ("pbe_paged_decode", C.c_int, [C.POINTER(ArenaView), C.c_int32, _P, C.c_uint64,
                                   C.POINTER(KvShape), C.c_int32, _P, _P, C.c_int32, C.c_int32,
                                   _P, _P, C.c_int32, C.c_int32, _P, C.c_uint64, C.c_int, _P]),
    ("pbe_stream_synchronize", C.c_int, [C.c_int, _P]),
    ("pbe_paged_decode_noalloc", C.c_int, [C.POINTER(ArenaView), C.c_int32, _P, C.c_uint64,
                                           C.POINTER(KvShape), C.c_int32, _P, _P, C.c_int32,
                                           C.c_int32, _P, _P, C.c_int32, C.c_int32, C.c_int, _P]),
    ("pbe_paged_decode_pools", C.c_int, [_P, _P, C.c_uint64, _P, _P, C.c_uint64, C.c_int32,
                                         C.c_int32, C.c_int32, _P, _P, C.c_int32, C.c_int32, _P,
                                         _P, C.c_int32, C.c_int32, _P, C.c_uint64, C.c_int, _P]),
    ("pbe_paged_decode_append_arena", C.c_int, [C.POINTER(ArenaView), C.c_int32, _P, C.c_uint64,
                                                C.POINTER(KvShape), C.c_int32, _P, _P, _P, _P,
                                                C.c_int32, C.c_int32, _P, _P, C.c_int32, C.c_int32,
                                                _P, C.c_uint64, C.c_int, _P]),
    ("pbe_paged_decode_append", C.c_int, [_P, _P, C.c_uint64, _P, _P, C.c_uint64, C.c_int32,
                                          C.c_int32, C.c_int32, _P, _P, _P, _P, C.c_int32,
                                          C.c_int32, _P, _P, C.c_int32, C.c_int32, _P, C.c_uint64,
                                          C.c_int, _P]),
    ("pbe_scatter_kv", C.c_int, [_P, _P, C.c_int32, C.c_int32, _P, C.c_int32, C.c_int32,
                                 C.c_int32, C.c_int32, _P, C.c_uint64, _P, C.c_uint64, _P,
                                 C.c_uint64, _P, C.c_uint64, C.c_int, _P]),
    ("pbe_scatter_kv_to_page", C.c_int, [_P, _P, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                         C.c_int32, C.c_int32, C.c_int32, _P, C.c_uint64, _P,
                                         C.c_uint64, _P, C.c_uint64, _P, C.c_uint64, C.c_int,
                                         _P]),
]
EXPORTED = [name for name, _, _ in _SIGNATURES]


class PbeError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


_lib = None


def lib() -> C.CDLL:
    """Loads lib/libpbe_handoff.so (built by build.py); raises if it is absent."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run paged-batch-engine_amd/build.py "
                               "(the HIP library has no fallback)")
        handle = C.CDLL(str(LIB_PATH))
        for name, res, args in _SIGNATURES:
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc: int) -> int:
    if rc < 0:
        raise PbeError(rc, lib().pbe_last_error().decode())
    return rc


def shape(layers: int, kv_heads: int, head_dim: int, page_tokens: int = 16) -> KvShape:
    return KvShape(layers, kv_heads, head_dim, page_tokens)


def view_of(ptrs, total_bytes: int, segment_bytes: int | None = None) -> ArenaView:
    """Arena view over caller-owned device memory: one pointer per segment."""
    if isinstance(ptrs, int):
        ptrs = [ptrs]
    v = ArenaView()
    v.bytes = total_bytes
    v.segment_bytes = segment_bytes or total_bytes
    v.nseg = len(ptrs)
    for i, p in enumerate(ptrs):
        v.base[i] = p
    return v


def _i32(arr):
    """A contiguous int32 copy (or the array itself) and its address as an int
    (an int passes to a c_void_p parameter at a fraction of data_as' cost)."""
    import numpy as np
    a = np.ascontiguousarray(arr, dtype=np.int32)
    return a, a.ctypes.data


def build_runs(src_ids, dst_ids, kv: KvShape, elem_bytes: int = 2, segment_bytes: int = 0):
    """Coalesced runs as a list of (src_block, dst_block, pages) tuples."""
    s, sp = _i32(src_ids)
    d, dp = _i32(dst_ids)
    if s.shape != d.shape:
        raise ValueError("src/dst id lists differ in length")
    out = (Run * max(1, len(s)))()
    n = C.c_int64()
    check(lib().pbe_build_runs(sp, dp, len(s), C.byref(kv), elem_bytes, segment_bytes, out,
                               C.byref(n)))
    return [(out[i].src_block, out[i].dst_block, out[i].pages) for i in range(n.value)]


def encode_page_list(ids, layers: int, epoch: int) -> bytes:
    """Compact wire form of a page-major id list (pbe_page_list_encode)."""
    a, ap = _i32(ids)
    need = lib().pbe_page_list_bytes(ap, len(a), layers)
    if need == 0:
        raise PbeError(PBE_ERR_INVALID, "ids are not a page-major list")
    buf = C.create_string_buffer(need)
    n = C.c_uint64()
    check(lib().pbe_page_list_encode(ap, len(a), layers, epoch, buf, need, C.byref(n)))
    return buf.raw[:n.value]


def decode_page_list(data: bytes, max_pages: int = 1 << 22):
    """(ids, layers, epoch) of a page list; raises PbeError on any defect, and
    before allocating anything when the list claims more than max_pages pages
    (a few bytes of spans can claim millions)."""
    import numpy as np
    n, layers, epoch = C.c_int64(), C.c_int32(), C.c_uint64()
    src = C.create_string_buffer(bytes(data), len(data)) if data else C.create_string_buffer(1)
    check(lib().pbe_page_list_decode(src, len(data), None, 0, C.byref(n), C.byref(layers),
                                     C.byref(epoch)))
    if n.value > max_pages:
        raise PbeError(PBE_ERR_INVALID, f"page list claims {n.value} pages (> {max_pages})")
    ids = np.empty(max(1, n.value), np.int32)
    check(lib().pbe_page_list_decode(src, len(data), ids.ctypes.data_as(C.c_void_p), n.value,
                                     C.byref(n), C.byref(layers), C.byref(epoch)))
    return ids[:n.value], layers.value, epoch.value


def validate_ids(ids, kv: KvShape, arena_bytes: int, elem_bytes: int = 2) -> int:
    """-1 if every id passes the reference's checks, else the first bad index."""
    a, ap = _i32(ids)
    bad = C.c_int64(-1)
    rc = lib().pbe_validate_ids(ap, len(a), C.byref(kv), elem_bytes, arena_bytes, C.byref(bad))
    if rc == PBE_ERR_INVALID:
        return bad.value
    check(rc)
    return -1


def _runs_array(runs):
    arr = (Run * len(runs))()
    for i, (s, d, p) in enumerate(runs):
        arr[i] = Run(s, d, p)
    return arr


class RunList:
    """Device-resident run list (owns its device buffer)."""

    def __init__(self, handle: int):
        self.handle = handle

    @classmethod
    def bf16(cls, src: ArenaView, dst: ArenaView, runs, kv: KvShape, device: int = 0,
             elem_bytes: int = 2):
        h = C.c_void_p()
        arr = _runs_array(runs)
        check(lib().pbe_runlist_create(C.byref(src), C.byref(dst), arr, len(runs), C.byref(kv),
                                       elem_bytes, device, C.byref(h)))
        return cls(h.value)

    @classmethod
    def fp8(cls, src: ArenaView, dst: ArenaView, scales_ptr: int, scales_bytes: int, runs,
            kv: KvShape, device: int = 0):
        h = C.c_void_p()
        arr = _runs_array(runs)
        check(lib().pbe_runlist_create_fp8(C.byref(src), C.byref(dst), scales_ptr or None,
                                           scales_bytes, arr, len(runs), C.byref(kv), device,
                                           C.byref(h)))
        return cls(h.value)

    def info(self) -> RunListInfo:
        i = RunListInfo()
        check(lib().pbe_runlist_get_info(self.handle, C.byref(i)))
        return i

    def copy(self, stream: int = 0) -> None:
        check(lib().pbe_handoff_copy(self.handle, stream or None))

    def copy_fp8(self, mode: int, amax_table_ptr: int = 0, stream: int = 0) -> None:
        check(lib().pbe_handoff_copy_fp8(self.handle, mode, amax_table_ptr or None,
                                         stream or None))

    def copy_timed(self, stream: int, start_event: int, stop_event: int) -> None:
        """copy() with two hipEvent_t handles stamped at the kernel's start and end."""
        check(lib().pbe_handoff_copy_timed(self.handle, stream or None, start_event, stop_event))

    def copy_fp8_timed(self, mode: int, amax_table_ptr: int, stream: int, start_event: int,
                       stop_event: int) -> None:
        check(lib().pbe_handoff_copy_fp8_timed(self.handle, mode, amax_table_ptr or None,
                                               stream or None, start_event, stop_event))

    def close(self) -> None:
        if self.handle:
            check(lib().pbe_runlist_destroy(self.handle))
            self.handle = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def copy_shared_kv(view: ArenaView, src_ids, dst_ids, kv: KvShape, device: int = 0,
                   stream: int = 0) -> int:
    s, sp = _i32(src_ids)
    d, dp = _i32(dst_ids)
    copied = C.c_uint64()
    check(lib().pbe_copy_shared_kv(C.byref(view), sp, dp, len(s), C.byref(kv), device,
                                   stream or None, C.byref(copied)))
    return copied.value


def stream_synchronize(stream: int = 0, device: int = 0) -> None:
    """Waits for everything queued on `stream` (hipStreamSynchronize)."""
    check(lib().pbe_stream_synchronize(device, stream or None))


def op_array(ops):
    """Packs (src, dst, bytes) tuples into a reusable CopyOp array."""
    import numpy as np
    a = np.ascontiguousarray(np.asarray(ops, dtype=np.uint64).reshape(-1, 3))
    arr = (CopyOp * max(1, len(a))).from_buffer_copy(a.tobytes() or bytes(24))
    return arr, len(a)


def copy_ops(ops, device: int = 0, stream: int = 0) -> None:
    """ops: list of (src, dst, bytes) or the (array, n) pair from op_array()."""
    arr, n = ops if isinstance(ops, tuple) and len(ops) == 2 and not isinstance(ops[0], int) \
        else op_array(ops)
    check(lib().pbe_copy_ops(arr, n, device, stream or None))


class Arena:
    """Owner (create) or importer (from_ipc) of a segmented device arena."""

    def __init__(self, handle: int):
        self.handle = handle

    @classmethod
    def create(cls, bytes_: int, segment_bytes: int = 0, epoch: int = 1, device: int = 0):
        h = C.c_void_p()
        check(lib().pbe_arena_create(device, bytes_, segment_bytes, epoch, C.byref(h)))
        return cls(h.value)

    @classmethod
    def from_ipc(cls, ipc: ArenaIpc, device: int = 0):
        h = C.c_void_p()
        check(lib().pbe_arena_import(C.byref(ipc), device, C.byref(h)))
        return cls(h.value)

    def export(self) -> ArenaIpc:
        ipc = ArenaIpc()
        check(lib().pbe_arena_export(self.handle, C.byref(ipc)))
        return ipc

    def view(self) -> ArenaView:
        v = ArenaView()
        check(lib().pbe_arena_get_view(self.handle, C.byref(v)))
        return v

    @property
    def epoch(self) -> int:
        return lib().pbe_arena_epoch(self.handle)

    def close(self) -> None:
        if self.handle:
            check(lib().pbe_arena_destroy(self.handle))
            self.handle = 0


class Event:
    def __init__(self, handle: int):
        self.handle = handle

    @classmethod
    def create(cls, device: int = 0, interprocess: bool = False):
        h = C.c_void_p()
        check(lib().pbe_event_create(device, int(interprocess), C.byref(h)))
        return cls(h.value)

    @classmethod
    def from_ipc(cls, handle_bytes: bytes, device: int = 0):
        buf = (C.c_uint8 * PBE_IPC_HANDLE_BYTES).from_buffer_copy(handle_bytes)
        h = C.c_void_p()
        check(lib().pbe_event_import(buf, device, C.byref(h)))
        return cls(h.value)

    def export(self) -> bytes:
        buf = (C.c_uint8 * PBE_IPC_HANDLE_BYTES)()
        check(lib().pbe_event_export(self.handle, buf))
        return bytes(buf)

    def record(self, stream: int = 0) -> None:
        check(lib().pbe_event_record(self.handle, stream or None))

    def wait(self, stream: int = 0) -> None:
        check(lib().pbe_event_wait(self.handle, stream or None))

    def query(self) -> bool:
        return check(lib().pbe_event_query(self.handle)) == PBE_OK

    def synchronize(self) -> None:
        check(lib().pbe_event_synchronize(self.handle))

    def close(self) -> None:
        if self.handle:
            check(lib().pbe_event_destroy(self.handle))
            self.handle = 0


class Signal:
    """64-bit sequence word shared across processes (pbe_signal_*)."""

    def __init__(self, handle: int):
        self.handle = handle

    @classmethod
    def create(cls, device: int = 0):
        h = C.c_void_p()
        check(lib().pbe_signal_create(device, C.byref(h)))
        return cls(h.value)

    @classmethod
    def from_ipc(cls, handle_bytes: bytes, device: int = 0):
        buf = (C.c_uint8 * PBE_IPC_HANDLE_BYTES).from_buffer_copy(handle_bytes)
        h = C.c_void_p()
        check(lib().pbe_signal_import(buf, device, C.byref(h)))
        return cls(h.value)

    def export(self) -> bytes:
        buf = (C.c_uint8 * PBE_IPC_HANDLE_BYTES)()
        check(lib().pbe_signal_export(self.handle, buf))
        return bytes(buf)

    def set(self, value: int, stream: int = 0) -> None:
        check(lib().pbe_signal_set(self.handle, value, stream or None))

    def wait(self, value: int, stream: int = 0) -> None:
        check(lib().pbe_signal_wait(self.handle, value, stream or None))

    def read(self) -> int:
        v = C.c_uint64()
        check(lib().pbe_signal_read(self.handle, C.byref(v)))
        return v.value

    def close(self) -> None:
        if self.handle:
            check(lib().pbe_signal_destroy(self.handle))
            self.handle = 0


def device_uuid(device: int = 0) -> bytes:
    buf = (C.c_uint8 * 16)()
    check(lib().pbe_device_uuid(device, buf))
    return bytes(buf)



def decode_splits(batch: int, kv_heads: int, max_blocks: int, kv_dtype: int) -> int:
    return int(lib().pbe_paged_decode_splits(batch, kv_heads, max_blocks, kv_dtype))


def decode_workspace_bytes(batch: int, q_heads: int, head_dim: int, splits: int) -> int:
    return int(lib().pbe_paged_decode_workspace_bytes(batch, q_heads, head_dim, splits))


PBE_DECODE_SCRATCH_BYTES = 8 << 20


def paged_decode_noalloc(view: ArenaView, kv_dtype: int, scales: int, scale_bytes: int,
                         kv: KvShape, layer: int, queries: int, outputs: int, batch: int,
                         q_heads: int, tables: int, seq_lens: int, max_blocks: int, splits: int,
                         stream: int = 0, device: int = 0) -> None:
    """pbe_paged_decode with the partials in the library's static scratch
    (pbe_paged_decode_noalloc): allocates nothing; calls on one GPU must not overlap."""
    check(lib().pbe_paged_decode_noalloc(C.byref(view), kv_dtype, scales or None, scale_bytes,
                                         C.byref(kv), layer, queries, outputs, batch, q_heads,
                                         tables, seq_lens, max_blocks, splits, device,
                                         stream or None))


def paged_decode_pools(key_pool: int, value_pool: int, pool_bytes: int, key_scales: int,
                       value_scales: int, scale_pool_bytes: int, kv_dtype: int, kv_heads: int,
                       head_dim: int, queries: int, outputs: int, batch: int, q_heads: int,
                       tables: int, seq_lens: int, max_blocks: int, splits: int, workspace: int,
                       workspace_bytes: int, stream: int = 0, device: int = 0) -> None:
    """Decode over per-layer K/V pools (pbe_paged_decode_pools); device pointers in,
    asynchronous on `stream`."""
    check(lib().pbe_paged_decode_pools(key_pool or None, value_pool or None, pool_bytes,
                                       key_scales or None, value_scales or None, scale_pool_bytes,
                                       kv_dtype, kv_heads, head_dim, queries, outputs, batch,
                                       q_heads, tables, seq_lens, max_blocks, splits, workspace,
                                       workspace_bytes, device, stream or None))


def paged_decode_append(key_pool: int, value_pool: int, pool_bytes: int, key_scales: int,
                        value_scales: int, scale_pool_bytes: int, kv_dtype: int, kv_heads: int,
                        head_dim: int, new_keys: int, new_values: int, queries: int, outputs: int,
                        batch: int, q_heads: int, tables: int, seq_lens: int, max_blocks: int,
                        splits: int, workspace: int, workspace_bytes: int, stream: int = 0,
                        device: int = 0) -> None:
    """One decode step over per-layer pools that first writes each sequence's new
    token (bf16 [batch][kv_heads][head_dim]) at its last position
    (pbe_paged_decode_append); device pointers in, asynchronous on `stream`."""
    check(lib().pbe_paged_decode_append(key_pool or None, value_pool or None, pool_bytes,
                                        key_scales or None, value_scales or None, scale_pool_bytes,
                                        kv_dtype, kv_heads, head_dim, new_keys or None,
                                        new_values or None, queries, outputs, batch, q_heads,
                                        tables, seq_lens, max_blocks, splits, workspace,
                                        workspace_bytes, device, stream or None))


def paged_decode_append_arena(view, kv_dtype: int, scales: int, scale_bytes: int, kv, layer: int,
                              new_keys: int, new_values: int, queries: int, outputs: int,
                              batch: int, q_heads: int, tables: int, seq_lens: int,
                              max_blocks: int, splits: int, workspace: int, workspace_bytes: int,
                              stream: int = 0, device: int = 0) -> None:
    """pbe_paged_decode_append_arena: the arena form of paged_decode_append."""
    check(lib().pbe_paged_decode_append_arena(C.byref(view), kv_dtype, scales or None, scale_bytes,
                                              C.byref(kv), layer, new_keys or None,
                                              new_values or None, queries, outputs, batch, q_heads,
                                              tables, seq_lens, max_blocks, splits, workspace,
                                              workspace_bytes, device, stream or None))


PBE_IN_BF16 = 0
PBE_IN_F32 = 1


def scatter_kv(keys: int, values: int, in_dtype: int, n_tokens: int, slots: int, block_size: int,
               kv_heads: int, head_dim: int, kv_dtype: int, key_pool: int, key_pool_bytes: int,
               value_pool: int, value_pool_bytes: int, key_scales: int = 0,
               key_scale_bytes: int = 0, value_scales: int = 0, value_scale_bytes: int = 0,
               stream: int = 0, device: int = 0) -> None:
    """New tokens' K/V rows into their page slots (pbe_scatter_kv); device
    pointers in, asynchronous on `stream`."""
    check(lib().pbe_scatter_kv(keys or None, values or None, in_dtype, n_tokens, slots or None,
                               block_size, kv_heads, head_dim, kv_dtype, key_pool or None,
                               key_pool_bytes, value_pool or None, value_pool_bytes,
                               key_scales or None, key_scale_bytes, value_scales or None,
                               value_scale_bytes, device, stream or None))


def scatter_kv_to_page(keys: int, values: int, in_dtype: int, block_id: int, offset: int,
                       block_size: int, kv_heads: int, head_dim: int, kv_dtype: int,
                       key_pool: int, key_pool_bytes: int, value_pool: int,
                       value_pool_bytes: int, key_scales: int = 0, key_scale_bytes: int = 0,
                       value_scales: int = 0, value_scale_bytes: int = 0, stream: int = 0,
                       device: int = 0) -> None:
    """One token at (block_id, offset) (pbe_scatter_kv_to_page)."""
    check(lib().pbe_scatter_kv_to_page(keys or None, values or None, in_dtype, block_id, offset,
                                       block_size, kv_heads, head_dim, kv_dtype,
                                       key_pool or None, key_pool_bytes, value_pool or None,
                                       value_pool_bytes, key_scales or None, key_scale_bytes,
                                       value_scales or None, value_scale_bytes, device,
                                       stream or None))


def paged_decode(view: ArenaView, kv_dtype: int, scales: int, scale_bytes: int, kv: KvShape,
                 layer: int, queries: int, outputs: int, batch: int, q_heads: int, tables: int,
                 seq_lens: int, max_blocks: int, splits: int, workspace: int,
                 workspace_bytes: int, stream: int = 0, device: int = 0) -> None:
    """Device pointers in, asynchronous on `stream` (pbe_paged_decode)."""
    check(lib().pbe_paged_decode(C.byref(view), kv_dtype, scales or None, scale_bytes, C.byref(kv),
                                 layer, queries, outputs, batch, q_heads, tables, seq_lens,
                                 max_blocks, splits, workspace, workspace_bytes, device,
                                 stream or None))
