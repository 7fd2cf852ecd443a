"""TEST INFRASTRUCTURE ONLY: numpy front-end of the C oracle (pbe_oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, as the checker / CPU baseline. The product never imports it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_LIB_PATH = HERE / "_ref" / "libpbe_ref.so"
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        P = C.c_void_p
        L.orc_coalesce.restype = C.c_int64
        L.orc_coalesce.argtypes = [P, P, C.c_int64, C.c_int32, P, P, P]
        L.orc_copy_runs.restype = C.c_uint64
        L.orc_copy_runs.argtypes = [P, P, P, P, C.c_int64, C.c_uint64, C.c_int32]
        L.orc_copy_handoff.restype = C.c_uint64
        L.orc_copy_handoff.argtypes = [P, P, P, C.c_int64, C.c_uint64, C.c_int32, P, P, P]
        L.orc_copy_components.restype = C.c_uint64
        L.orc_copy_components.argtypes = [P, P, P, C.c_int64, C.c_uint64, C.c_int32]
        L.orc_validate_ids.restype = C.c_int64
        L.orc_validate_ids.argtypes = [P, C.c_int64, C.c_int32, C.c_uint64, C.c_uint64]
        L.orc_bf16_from_f32_array.restype = None
        L.orc_bf16_from_f32_array.argtypes = [P, P, C.c_int64]
        L.orc_e4m3_from_f32_array.restype = None
        L.orc_e4m3_from_f32_array.argtypes = [P, P, C.c_int64]
        L.orc_e4m3_to_f32.restype = C.c_float
        L.orc_e4m3_to_f32.argtypes = [C.c_uint8]
        L.orc_fp8_handoff_token_head.restype = None
        L.orc_fp8_handoff_token_head.argtypes = [P, P, P, P, P, C.c_int64, C.c_int32, C.c_int32,
                                                 C.c_int32, C.c_int32]
        L.orc_fp8_handoff_table.restype = None
        L.orc_fp8_handoff_table.argtypes = [P, P, P, P, P, C.c_int64, C.c_int32, C.c_int32,
                                            C.c_int32, C.c_int32]
        L.orc_fp8_table_scales.restype = None
        L.orc_fp8_table_scales.argtypes = [P, P, C.c_int64]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def coalesce(src, dst, layers: int):
    """[(src_block, dst_block, pages)] per split_pd_engine.cpp:96-101."""
    s, d = _i32(src), _i32(dst)
    n = len(s)
    rs, rd, rp = (np.zeros(max(n, 1), np.int32) for _ in range(3))
    k = lib().orc_coalesce(_p(s), _p(d), n, 2 * layers, _p(rs), _p(rd), _p(rp))
    return list(zip(rs[:k].tolist(), rd[:k].tolist(), rp[:k].tolist()))


def copy_handoff(arena: np.ndarray, src, dst, half: int, layers: int) -> int:
    """In-place reference handoff on a uint8 arena; returns copied bytes."""
    assert arena.dtype == np.uint8 and arena.flags.c_contiguous
    s, d = _i32(src), _i32(dst)
    n = len(s)
    scratch = [np.zeros(max(n, 1), np.int32) for _ in range(3)]
    return lib().orc_copy_handoff(_p(arena), _p(s), _p(d), n, half, layers,
                                  *[_p(x) for x in scratch])


def copy_runs(arena: np.ndarray, runs, half: int, layers: int) -> int:
    rs = _i32([r[0] for r in runs])
    rd = _i32([r[1] for r in runs])
    rp = _i32([r[2] for r in runs])
    return lib().orc_copy_runs(_p(arena), _p(rs), _p(rd), _p(rp), len(rs), half, layers)


def copy_components(arena: np.ndarray, src, dst, half: int, layers: int) -> int:
    s, d = _i32(src), _i32(dst)
    return lib().orc_copy_components(_p(arena), _p(s), _p(d), len(s), half, layers)


def validate_ids(ids, layers: int, half: int, arena_bytes: int) -> int:
    a = _i32(ids)
    return int(lib().orc_validate_ids(_p(a), len(a), layers, half, arena_bytes))


def bf16_from_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_bf16_from_f32_array(_p(x), _p(out), x.size)
    return out


def e4m3_from_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().orc_e4m3_from_f32_array(_p(x), _p(out), x.size)
    return out


def e4m3_to_f32(code: int) -> float:
    return float(lib().orc_e4m3_to_f32(code))


def fp8_handoff_token_head(src_arena, dst_arena, dst_scales, src, dst, layers, tokens, heads,
                           head_dim) -> None:
    s, d = _i32(src), _i32(dst)
    lib().orc_fp8_handoff_token_head(_p(src_arena), _p(dst_arena), _p(dst_scales), _p(s), _p(d),
                                     len(s), layers, tokens, heads, head_dim)


def fp8_handoff_table(src_arena, dst_arena, amax_table, src, dst, layers, tokens, heads,
                      head_dim) -> None:
    s, d = _i32(src), _i32(dst)
    t = np.ascontiguousarray(amax_table, dtype=np.float32)
    lib().orc_fp8_handoff_table(_p(src_arena), _p(dst_arena), _p(t), _p(s), _p(d), len(s),
                                layers, tokens, heads, head_dim)


def table_scales(amax_table) -> np.ndarray:
    t = np.ascontiguousarray(amax_table, dtype=np.float32)
    out = np.empty_like(t)
    lib().orc_fp8_table_scales(_p(t), _p(out), t.size)
    return out
