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
        L.orc_scatter_kv.restype = None
        L.orc_scatter_kv.argtypes = [P, P, C.c_int32, C.c_int64, P, C.c_int32, C.c_int32,
                                     C.c_int32, C.c_int32, P, C.c_uint64, P, C.c_uint64, P,
                                     C.c_uint64, P, C.c_uint64]
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


def scatter_kv(keys, values, slots, block_size: int, heads: int, head_dim: int, fp8: bool,
               key_pool: np.ndarray, value_pool: np.ndarray, key_scales=None,
               value_scales=None) -> None:
    """orc_scatter_kv in place. keys/values: [n][heads*head_dim] uint16 (BF16 bits)
    or float32; pools: uint8 arrays; scales: float32 arrays (FP8 only)."""
    k, v = np.ascontiguousarray(keys), np.ascontiguousarray(values)
    assert k.dtype == v.dtype and k.dtype in (np.uint16, np.float32) and k.shape == v.shape
    s = _i32(slots)
    assert key_pool.dtype == np.uint8 and value_pool.dtype == np.uint8
    assert key_pool.flags.c_contiguous and value_pool.flags.c_contiguous
    ks = key_scales if fp8 else np.zeros(1, np.float32)
    vs = value_scales if fp8 else np.zeros(1, np.float32)
    assert ks.dtype == np.float32 and vs.dtype == np.float32
    lib().orc_scatter_kv(_p(k), _p(v), int(k.dtype == np.float32), len(s), _p(s), block_size,
                         heads, head_dim, int(fp8), _p(key_pool), key_pool.nbytes, _p(value_pool),
                         value_pool.nbytes, _p(ks), ks.size if fp8 else 0, _p(vs),
                         vs.size if fp8 else 0)


def e4m3_table() -> np.ndarray:
    """float64 value of every E4M3 code (NaN for 0x7f / 0xff)."""
    return np.array([e4m3_to_f32(c) for c in range(256)], np.float64)


def _decode(fetch, fp8: bool, kv_heads: int, head_dim: int, q_bf16, tables, seq_lens) -> np.ndarray:
    """float64 split-K decode over rows that fetch(ids, tok, kvh) returns as
    (K bytes [n, D*E], V bytes, k_scale [n], v_scale [n])."""
    q = np.asarray(q_bf16, np.uint16)
    batch, q_heads, D = q.shape
    assert D == head_dim
    kvm = q_heads // kv_heads
    qf = (q.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    lut = e4m3_table() if fp8 else None
    scale = float(np.float32(np.float32(1.0) / np.sqrt(np.float32(head_dim))) * np.float32(1.4426950408889634))
    out = np.zeros((batch, q_heads, D), np.float64)
    for b in range(batch):
        n = int(seq_lens[b])
        if n <= 0:
            continue
        t = np.arange(n)
        ids = np.asarray(tables[b], np.int64)[t // 16]
        tok = t % 16
        for kvh in range(kv_heads):
            kb, vb, ks, vs = fetch(ids, tok, kvh)
            if fp8:
                K, V = lut[kb], lut[vb]
            else:
                K = (kb.view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
                V = (vb.view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
            for r in range(kvm):
                qh = kvh * kvm + r
                s = (K @ qf[b, qh]) * (scale * ks)
                p = np.exp2(s - np.max(s))
                out[b, qh] = (p * vs) @ V / p.sum()
    return out


def paged_decode(arena: np.ndarray, fp8: bool, scales, layers: int, kv_heads: int, head_dim: int,
                 layer: int, q_bf16: np.ndarray, tables: np.ndarray, seq_lens) -> np.ndarray:
    """float64 restatement of one split-K paged-attention decode step
    (paged_mha_fast_kernel.cu:558-799 for FP8 pages, :391-556 for BF16 pages):
    for query head qh of sequence b and its KV head qh // (q_heads / kv_heads),
      score_t = (q . k_t) * (1/sqrt(D) * log2(e), both as fp32) * k_scale_t
      p_t     = 2 ** (score_t - max_t score_t)
      out     = sum_t p_t * v_scale_t * v_t / sum_t p_t      (0 when seq_len == 0)
    over tokens t < seq_len of the blocks tables[b][t // 16], where block id
    `id` keeps layer l's K plane at byte (id + 2l) * half and the V plane at
    (id + 2l + 1) * half, token-major inside ([token][kv_head][D]); FP8 scale
    k_scale_t sits at fp32 index ((id + 2l) * 16 + tok) * kv_heads + kv_head,
    v_scale_t one plane (16 * kv_heads floats) later. Returns float64
    [batch][q_heads][D] (the caller rounds to BF16 for comparison)."""
    arena = np.ascontiguousarray(arena).view(np.uint8).ravel()
    E = 1 if fp8 else 2
    half = 16 * kv_heads * head_dim * E
    sc = None if scales is None else np.asarray(scales, np.float32).ravel().astype(np.float64)
    cols = np.arange(head_dim * E)

    def fetch(ids, tok, kvh):
        koff = (ids + 2 * layer) * half + (tok * kv_heads + kvh) * head_dim * E
        kb = arena[koff[:, None] + cols[None, :]]
        vb = arena[(koff + half)[:, None] + cols[None, :]]
        if not fp8:
            return kb, vb, np.ones(len(ids)), np.ones(len(ids))
        sidx = ((ids + 2 * layer) * 16 + tok) * kv_heads + kvh
        return kb, vb, sc[sidx], sc[sidx + 16 * kv_heads]

    return _decode(fetch, fp8, kv_heads, head_dim, q_bf16, tables, seq_lens)


def paged_decode_pools(key_pool: np.ndarray, value_pool: np.ndarray, fp8: bool, key_scales,
                       value_scales, kv_heads: int, head_dim: int, q_bf16: np.ndarray,
                       tables: np.ndarray, seq_lens) -> np.ndarray:
    """The same step over per-layer pools, the reference kernels' addressing
    (paged_mha_fast_kernel.cu:671-694): block b's K row of token tok and head h
    at key_pool byte b*half + (tok*H + h)*D*E, its V row likewise in value_pool,
    FP8 scales at key_scales / value_scales [b*16*H + tok*H + h]."""
    kp = np.ascontiguousarray(key_pool).view(np.uint8).ravel()
    vp = np.ascontiguousarray(value_pool).view(np.uint8).ravel()
    E = 1 if fp8 else 2
    half = 16 * kv_heads * head_dim * E
    ks_ = None if key_scales is None else np.asarray(key_scales, np.float32).ravel().astype(np.float64)
    vs_ = None if value_scales is None else np.asarray(value_scales, np.float32).ravel().astype(np.float64)
    cols = np.arange(head_dim * E)

    def fetch(ids, tok, kvh):
        off = ids * half + (tok * kv_heads + kvh) * head_dim * E
        kb = kp[off[:, None] + cols[None, :]]
        vb = vp[off[:, None] + cols[None, :]]
        if not fp8:
            return kb, vb, np.ones(len(ids)), np.ones(len(ids))
        sidx = ids * 16 * kv_heads + tok * kv_heads + kvh
        return kb, vb, ks_[sidx], vs_[sidx]

    return _decode(fetch, fp8, kv_heads, head_dim, q_bf16, tables, seq_lens)


def ref_cpu_handoff(lib_path, arena: np.ndarray, src, dst, layers: int, kv_heads: int,
                    head_size: int, page_tokens: int = 16, repeats: int = 1) -> int:
    """The generic CPU plan path (bind each page's planes, ExecuteCpuTransfer)
    from oracle/ref_driver.cpp, in the build at `lib_path`: the reference's own
    sources (oracle/_ref) or this repository's drop-in API. In place on a uint8
    host arena; returns the bytes one pass copies, -1 on error."""
    assert arena.dtype == np.uint8 and arena.flags.c_contiguous
    lib_ = C.CDLL(str(lib_path))
    f = lib_.ref_cpu_handoff
    f.restype = C.c_int64
    f.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p, C.c_int64, C.c_int32, C.c_int32,
                  C.c_int32, C.c_int32, C.c_int32]
    s, d = _i32(src), _i32(dst)
    return int(f(_p(arena), arena.nbytes, _p(s), _p(d), len(s), layers, kv_heads, head_size,
                 page_tokens, repeats))
