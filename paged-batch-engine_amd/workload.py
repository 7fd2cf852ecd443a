"""Seeded synthetic handoff workloads (the five configurations of the handoff
benchmark): page geometry, arena size, and page-major source/destination block
id lists as the decode side receives them (split_pd_engine.cpp:63-93).

A page id is a block id (byte offset / half) that is a multiple of 2*layers.
Source pages model a prefill whose Chunks were leased back to back by the
owner (GlobalChunkAllocator best fit on a fresh arena hands out adjacent
Chunks), so source pages are contiguous unless stated otherwise; destination
pages are placed so that the coalesced runs have the configured length law.
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass, field

import numpy as np

KIB = 1024
MIB = 1024 * 1024


@dataclass
class Geometry:
    layers: int
    kv_heads: int
    head_dim: int
    page_tokens: int = 16

    def half(self, elem_bytes: int = 2) -> int:
        return self.page_tokens * self.kv_heads * self.head_dim * elem_bytes

    def page_bytes(self, elem_bytes: int = 2) -> int:
        return 2 * self.layers * self.half(elem_bytes)

    @property
    def stride(self) -> int:  # block ids per page
        return 2 * self.layers


@dataclass
class Request:
    tokens: int
    src_ids: np.ndarray  # page-major block ids, one per page
    dst_ids: np.ndarray

    @property
    def pages(self) -> int:
        return len(self.src_ids)


@dataclass
class Workload:
    name: str
    geometry: Geometry
    arena_bytes: int
    segment_bytes: int  # 0 = one allocation
    requests: list[Request]
    sigma: float = 1.0
    outlier_fraction: float = 0.0
    outlier_value: float = 0.0
    amax_table: np.ndarray | None = None  # FP8 table mode, [2L][H] amax values
    fp8: bool = False
    meta: dict = field(default_factory=dict)

    @property
    def src_ids(self) -> np.ndarray:
        return np.concatenate([r.src_ids for r in self.requests]).astype(np.int32)

    @property
    def dst_ids(self) -> np.ndarray:
        return np.concatenate([r.dst_ids for r in self.requests]).astype(np.int32)

    @property
    def pages(self) -> int:
        return sum(r.pages for r in self.requests)

    def copied_bytes(self) -> int:
        return self.pages * self.geometry.page_bytes()

    def algorithmic_bytes(self) -> int:
        """Read + write of every copied page (FP8: BF16 read + FP8 write; the
        scale writes of the per-token-head mode are added by the caller)."""
        g = self.geometry
        if self.fp8:
            return self.pages * (g.page_bytes(2) + g.page_bytes(1))
        return 2 * self.copied_bytes()


def _pages_needed(tokens: int, page_tokens: int = 16) -> int:
    # blocks = ceil(computed / block_size) (decode_kv_reservation.cpp:50-55)
    return (tokens + page_tokens - 1) // page_tokens


def _runs_uniform(rng, total: int, lo: int, hi: int) -> list[int]:
    out = []
    while total > 0:
        k = int(rng.integers(lo, hi + 1))
        k = min(k, total)
        out.append(k)
        total -= k
    return out


def _runs_geometric(rng, total: int, p: float) -> list[int]:
    out = []
    while total > 0:
        k = min(int(rng.geometric(p)), total)
        out.append(k)
        total -= k
    return out


class _PageMap:
    """Free/used map over the pages of an arena (page index = id / stride)."""

    def __init__(self, n_pages: int, segment_pages: int = 0):
        self.used = np.zeros(n_pages, dtype=bool)
        self.segment_pages = segment_pages

    def take(self, start: int, k: int) -> None:
        assert not self.used[start:start + k].any()
        self.used[start:start + k] = True

    def free_extent_starts(self, k: int) -> np.ndarray:
        free = ~self.used
        if k == 1:
            starts = np.nonzero(free)[0]
        else:
            c = np.concatenate([[0], np.cumsum(free.astype(np.int64))])
            ok = (c[k:] - c[:-k]) == k
            starts = np.nonzero(ok)[0]
        if self.segment_pages:
            sp = self.segment_pages
            starts = starts[(starts // sp) == ((starts + k - 1) // sp)]
        return starts

    def place(self, rng, k: int, avoid_after: int | None = None) -> int:
        starts = self.free_extent_starts(k)
        if avoid_after is not None:
            starts = starts[starts != avoid_after]
        if len(starts) == 0:
            raise RuntimeError(f"no free extent of {k} pages")
        s = int(starts[rng.integers(len(starts))])
        self.take(s, k)
        return s


def _place_request(rng, pm: _PageMap, runs: list[int], stride: int,
                   src_contiguous_start: int | None = None):
    """Places one request: src pages contiguous at src_contiguous_start (or
    run-by-run on free extents), dst runs on free extents, never extending the
    previous run so each listed run stays maximal."""
    src_pages, dst_pages = [], []
    prev_src_end = prev_dst_end = None
    cursor = src_contiguous_start
    for k in runs:
        if cursor is not None:
            s = cursor
            cursor += k
        else:
            s = pm.place(rng, k, avoid_after=prev_src_end)
        d = pm.place(rng, k, avoid_after=prev_dst_end if (cursor is not None or s == prev_src_end)
                     else None)
        src_pages.extend(range(s, s + k))
        dst_pages.extend(range(d, d + k))
        prev_src_end, prev_dst_end = s + k, d + k
    return (np.asarray(src_pages, np.int64) * stride).astype(np.int32), \
           (np.asarray(dst_pages, np.int64) * stride).astype(np.int32)


def config1(seed: int = 0) -> Workload:
    """Qwen2.5-0.5B BF16, 41-token prefix (3 pages) on a 512 MiB arena of
    2112 KiB Chunks of 11 pages; src and dst are random free pages."""
    g = Geometry(24, 2, 64)
    rng = np.random.default_rng(seed)
    chunk = 11 * g.page_bytes()
    n_pages = (512 * MIB // chunk) * 11
    pages = rng.choice(n_pages, size=6, replace=False)
    src = (pages[:3] * g.stride).astype(np.int32)
    dst = (pages[3:] * g.stride).astype(np.int32)
    return Workload("c1_qwen05b_41tok", g, 512 * MIB, 0, [Request(41, src, dst)], sigma=1.0,
                    meta={"chunk_pages": 11, "n_pages": int(n_pages)})


def config2(seed: int = 0, tokens: int = 5040) -> Workload:
    """Qwen2.5-1.5B BF16, 5040-token prefix (315 pages) on a 2112 MiB arena of
    2240 KiB Chunks of 5 pages; destination runs uniform in 1..5 pages."""
    g = Geometry(28, 2, 128)
    rng = np.random.default_rng(seed)
    n_pages = (2112 * MIB // (5 * g.page_bytes())) * 5
    pm = _PageMap(n_pages)
    npg = _pages_needed(tokens)
    src_start = int(rng.integers(0, (n_pages - npg) // 5)) * 5
    pm.take(src_start, npg)
    runs = _runs_uniform(rng, npg, 1, 5)
    src, dst = _place_request(rng, pm, runs, g.stride, src_contiguous_start=src_start)
    return Workload("c2_qwen15b_5040tok", g, 2112 * MIB, 0, [Request(tokens, src, dst)],
                    sigma=1.5, meta={"chunk_pages": 5, "n_pages": n_pages, "runs": len(runs)})


def config3(seed: int = 0) -> Workload:
    """Three requests (7040, 5040, 41 tokens) into one decode process on the
    1.5B arena fragmented to 50% occupancy (half of the 5-page Chunks leased to
    other requests); runs Geometric(1/2) (mean 2)."""
    g = Geometry(28, 2, 128)
    rng = np.random.default_rng(seed)
    n_chunks = 2112 * MIB // (5 * g.page_bytes())
    n_pages = n_chunks * 5
    pm = _PageMap(n_pages)
    occupied = rng.choice(n_chunks, size=n_chunks // 2, replace=False)
    pm.used[(occupied[:, None] * 5 + np.arange(5)).ravel()] = True
    reqs = []
    for tokens in (7040, 5040, 41):
        runs = _runs_geometric(rng, _pages_needed(tokens), 0.5)
        src, dst = _place_request(rng, pm, runs, g.stride)
        reqs.append(Request(tokens, src, dst))
    return Workload("c3_qwen15b_multi", g, 2112 * MIB, 0, reqs, sigma=1.0,
                    meta={"n_pages": n_pages, "occupancy": 0.5})


def config4(seed: int = 0) -> Workload:
    """Fused BF16 -> FP8 E4M3 handoff of the config-2 plan. The destination is
    an FP8 pool of half the page bytes (dst ids in FP8 half units); values
    N(0,1) with 0.1% outliers at +-40; static amax table per (layer, K|V, head)."""
    base = config2(seed)
    g = base.geometry
    rng = np.random.default_rng(seed + 4)
    amax = rng.uniform(2.5, 5.0, size=(2 * g.layers, g.kv_heads)).astype(np.float32)
    return dataclasses.replace(base, name="c4_qwen15b_fp8", sigma=1.0, outlier_fraction=1e-3,
                               outlier_value=40.0, amax_table=amax, fp8=True)


def config5(seed: int = 0) -> Workload:
    """Qwen2.5-7B-like (28 layers, 4 KV heads x 128), 896 KiB pages; 32768- and
    512-token prefixes from two prefill processes; runs uniform 1..8. The arena
    is three segments of 2048 pages (1.75 GiB each, under the 2 GiB IPC limit)."""
    g = Geometry(28, 4, 128)
    rng = np.random.default_rng(seed)
    seg_pages = 2048
    n_pages = 3 * seg_pages
    pm = _PageMap(n_pages, segment_pages=seg_pages)
    reqs = []
    for tokens in (32768, 512):
        runs = _runs_uniform(rng, _pages_needed(tokens), 1, 8)
        src, dst = _place_request(rng, pm, runs, g.stride)
        reqs.append(Request(tokens, src, dst))
    return Workload("c5_qwen7b_2p1d", g, n_pages * g.page_bytes(), seg_pages * g.page_bytes(),
                    reqs, sigma=1.0, meta={"n_pages": n_pages, "segment_pages": seg_pages})


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


def small(seed: int = 0, layers: int = 3, kv_heads: int = 2, head_dim: int = 64,
          n_pages: int = 64, handoff_pages: int = 17, max_run: int = 4,
          segment_pages: int = 0) -> Workload:
    """Small random workload for oracle-sized parity tests."""
    g = Geometry(layers, kv_heads, head_dim)
    rng = np.random.default_rng(seed)
    if n_pages < 4 * handoff_pages + 2 * max_run:
        raise ValueError("small(): arena too small to place the plan reliably")
    pm = _PageMap(n_pages, segment_pages=segment_pages)
    runs = _runs_uniform(rng, handoff_pages, 1, max_run)
    src, dst = _place_request(rng, pm, runs, g.stride)
    return Workload(f"small_s{seed}", g, n_pages * g.page_bytes(),
                    segment_pages * g.page_bytes(), [Request(handoff_pages * 16, src, dst)])
