"""Helpers shared by the GPU parity tests: device arenas filled with seeded
BF16 values, host snapshots, and oracle comparison."""
from __future__ import annotations

import numpy as np

import pbe_handoff as P


def stream_ptr(torch) -> int:
    return torch.cuda.current_stream().cuda_stream


def fill_bf16(torch, buf, sigma: float, seed: int, outlier_fraction: float = 0.0,
              outlier_value: float = 0.0) -> None:
    """Fills a uint8 device tensor with BF16 N(0, sigma) values (+ outliers)."""
    g = torch.Generator(device=buf.device)
    g.manual_seed(seed)
    vals = buf.view(torch.bfloat16)
    chunk = 1 << 26
    for i in range(0, vals.numel(), chunk):
        v = vals[i:i + chunk]
        v.copy_((torch.randn(v.numel(), generator=g, device=buf.device) * sigma).to(torch.bfloat16))
        if outlier_fraction:
            m = torch.rand(v.numel(), generator=g, device=buf.device) < outlier_fraction
            sgn = torch.where(torch.rand(v.numel(), generator=g, device=buf.device) < 0.5, -1.0, 1.0)
            v[m] = (sgn[m] * outlier_value).to(torch.bfloat16)


def device_arena(torch, nbytes: int, segment_bytes: int = 0):
    """Device buffers (one per segment) and the matching ArenaView."""
    seg = segment_bytes or nbytes
    bufs = []
    off = 0
    while off < nbytes:
        n = min(seg, nbytes - off)
        bufs.append(torch.empty(n, dtype=torch.uint8, device="cuda"))
        off += n
    view = P.view_of([b.data_ptr() for b in bufs], nbytes, seg)
    return bufs, view


def snapshot(bufs) -> np.ndarray:
    return np.concatenate([b.cpu().numpy() for b in bufs])


def first_diff(a: np.ndarray, b: np.ndarray) -> str:
    idx = np.nonzero(a != b)[0]
    if len(idx) == 0:
        return "identical"
    i = int(idx[0])
    return f"{len(idx)} bytes differ, first at {i}: got {a[i]:#04x} want {b[i]:#04x}"
