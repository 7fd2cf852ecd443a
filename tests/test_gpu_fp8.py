"""GPU parity of the fused BF16 -> FP8 E4M3 handoff against the CPU oracle,
bit-exact on payload bytes and scale words."""
import numpy as np
import pytest

import pbe_handoff as P
import workload as W
from oracle import oracle as O
from tests.conftest import say
from tests.gpu_util import fill_bf16, first_diff, stream_ptr

pytestmark = pytest.mark.gpu


class Fp8Pools:
    """BF16 source arena, FP8 destination arena and scale pool on the device."""

    def __init__(self, torch, g: W.Geometry, n_pages: int):
        self.g = g
        self.n_pages = n_pages
        self.src = torch.empty(n_pages * g.page_bytes(2), dtype=torch.uint8, device="cuda")
        self.dst = torch.zeros(n_pages * g.page_bytes(1), dtype=torch.uint8, device="cuda")
        self.scale_page = 2 * g.layers * g.page_tokens * g.kv_heads * 4
        self.scales = torch.zeros(n_pages * self.scale_page, dtype=torch.uint8, device="cuda")
        self.src_view = P.view_of(self.src.data_ptr(), self.src.numel())
        self.dst_view = P.view_of(self.dst.data_ptr(), self.dst.numel())
        self.kv = P.shape(g.layers, g.kv_heads, g.head_dim, g.page_tokens)

    def runlist(self, src_ids, dst_ids, with_scales=True):
        runs = P.build_runs(src_ids, dst_ids, self.kv)
        return P.RunList.fp8(self.src_view, self.dst_view,
                             self.scales.data_ptr() if with_scales else 0,
                             self.scales.numel() if with_scales else 0, runs, self.kv)


def _check(torch, pools: Fp8Pools, src_ids, dst_ids, mode, amax=None):
    g = pools.g
    src_host = pools.src.cpu().numpy()
    dst_exp = pools.dst.cpu().numpy().copy()
    sc_exp = pools.scales.cpu().numpy().copy()
    if mode == P.PBE_FP8_SCALE_TABLE:
        O.fp8_handoff_table(src_host, dst_exp, amax, src_ids, dst_ids, g.layers, g.page_tokens,
                            g.kv_heads, g.head_dim)
        table = torch.tensor(np.ascontiguousarray(amax, np.float32).ravel(), device="cuda")
        with pools.runlist(src_ids, dst_ids, with_scales=False) as rl:
            rl.copy_fp8(mode, table.data_ptr(), stream_ptr(torch))
            torch.cuda.synchronize()
    else:
        O.fp8_handoff_token_head(src_host, dst_exp, sc_exp, src_ids, dst_ids, g.layers,
                                 g.page_tokens, g.kv_heads, g.head_dim)
        with pools.runlist(src_ids, dst_ids) as rl:
            info = rl.info()
            assert info.scale_bytes == len(src_ids) * pools.scale_page
            rl.copy_fp8(mode, 0, stream_ptr(torch))
            torch.cuda.synchronize()
    dst = pools.dst.cpu().numpy()
    assert np.array_equal(dst, dst_exp), first_diff(dst, dst_exp)
    sc = pools.scales.cpu().numpy()
    assert np.array_equal(sc, sc_exp), first_diff(sc, sc_exp)


def test_conversion_covers_every_bf16_pattern(torch_cuda):
    """All 65536 BF16 bit patterns (zeros, subnormals, NaN, +-inf included) times
    a spread of multipliers, through the table-mode kernel, vs the oracle's
    OCP E4M3 rounding."""
    torch = torch_cuda
    g = W.Geometry(1, 2, 128)
    per_page = g.page_bytes(2) // 2
    n_pages = 65536 // per_page
    pools = Fp8Pools(torch, g, n_pages)
    pats = np.arange(65536, dtype=np.uint16)
    pools.src.copy_(torch.from_numpy(pats.view(np.uint8)).cuda())
    ids = np.arange(n_pages, dtype=np.int32) * g.stride
    tables = [
        [448.0, 1.0, 3.75, 1e-3],
        [448.0 * 2.0 ** -20, 5.2e3, 0.0, 2.0 ** 100],
        [1.0e-38, 7.0, 448.0 * 3, 0.15625],
    ]
    for t in tables:
        say(f"fp8 exhaustive table {t}")
        pools.dst.zero_()
        amax = np.asarray(t, np.float32).reshape(2, 2)
        _check(torch, pools, ids, ids, P.PBE_FP8_SCALE_TABLE, amax)


def test_per_token_head_special_rows(torch_cuda):
    torch = torch_cuda
    g = W.Geometry(2, 2, 64)
    pools = Fp8Pools(torch, g, 8)
    rng = np.random.default_rng(0)
    vals = (rng.standard_normal(pools.src.numel() // 2) * 2).astype(np.float32)
    rows = vals.reshape(-1, g.head_dim)
    rows[0] = 0.0                              # amax 0: scale 1, codes +0
    rows[1, 5] = np.inf                        # amax inf: inv 0
    rows[2, 7] = np.nan                        # NaN skipped by fmaxf, coded 0x7f
    rows[3] = -0.0
    rows[4] *= 1e-30                           # tiny amax
    rows[5, 3] = 3.0e38                        # huge amax
    bits = O.bf16_from_f32(vals)
    pools.src.copy_(torch.from_numpy(bits.view(np.uint8)).cuda())
    src = np.array([0, 1, 2, 3], np.int32) * g.stride
    dst = np.array([7, 6, 4, 5], np.int32) * g.stride
    say("fp8 per-token-head special rows")
    _check(torch, pools, src, dst, P.PBE_FP8_SCALE_PER_TOKEN_HEAD)


@pytest.mark.parametrize("mode", [P.PBE_FP8_SCALE_PER_TOKEN_HEAD, P.PBE_FP8_SCALE_TABLE])
@pytest.mark.parametrize("layers,kv_heads,head_dim", [
    (3, 2, 8), (3, 2, 64), (3, 2, 128), (3, 2, 256), (1, 1, 512), (28, 2, 128), (5, 3, 64),
    (2, 8, 32), (4, 1, 16)])
def test_small_random_fp8(torch_cuda, mode, layers, kv_heads, head_dim):
    torch = torch_cuda
    seed = layers * 1000 + kv_heads * 100 + head_dim
    w = W.small(seed=seed, layers=layers, kv_heads=kv_heads, head_dim=head_dim, n_pages=48,
                handoff_pages=9, max_run=3)
    g = w.geometry
    pools = Fp8Pools(torch, g, 48)
    fill_bf16(torch, pools.src, 1.0, seed, 0.01, 40.0)
    amax = np.random.default_rng(seed).uniform(2.5, 5.0, (2 * g.layers, g.kv_heads))
    say(f"fp8 small mode={mode} L={layers} H={kv_heads} D={head_dim}")
    _check(torch, pools, w.src_ids, w.dst_ids, mode, amax)


@pytest.mark.parametrize("mode", [P.PBE_FP8_SCALE_PER_TOKEN_HEAD, P.PBE_FP8_SCALE_TABLE])
def test_config4_fp8(torch_cuda, mode):
    torch = torch_cuda
    w = W.config4(0)
    g = w.geometry
    pools = Fp8Pools(torch, g, w.meta["n_pages"])
    fill_bf16(torch, pools.src, w.sigma, 4, w.outlier_fraction, w.outlier_value)
    say(f"config4 mode={mode}")
    _check(torch, pools, w.src_ids, w.dst_ids, mode, w.amax_table)


def test_fp8_rejects_misuse(torch_cuda):
    torch = torch_cuda
    g = W.Geometry(2, 2, 64)
    pools = Fp8Pools(torch, g, 4)
    ids = np.array([0], np.int32)
    with pools.runlist(ids, ids + g.stride, with_scales=False) as rl:
        with pytest.raises(P.PbeError):
            rl.copy_fp8(P.PBE_FP8_SCALE_PER_TOKEN_HEAD)   # no scale pool
        with pytest.raises(P.PbeError):
            rl.copy_fp8(P.PBE_FP8_SCALE_TABLE)            # no table
        with pytest.raises(P.PbeError):
            rl.copy()                                     # FP8 list on the BF16 copy
    bad = W.Geometry(2, 2, 24)
    kv = P.shape(bad.layers, bad.kv_heads, bad.head_dim)
    with pytest.raises(P.PbeError) as e:
        P.RunList.fp8(pools.src_view, pools.dst_view, 0, 0, [(0, 4, 1)], kv)
    assert e.value.code == P.PBE_ERR_UNSUPPORTED


def test_fp8_destination_beyond_4_gib(torch_cuda):
    """Destination pages above the 4 GiB offset of one 6 GiB FP8 arena:
    payload and per-token-head scales bit-exact (oracle run on the gathered
    pages)."""
    torch = torch_cuda
    g = W.Geometry(28, 2, 128)
    src_pages_n, n_dst = 64, (6 << 30) // g.page_bytes(1)
    say(f"fp8 handoff into a 6 GiB FP8 arena ({n_dst} pages)")
    src = torch.empty(src_pages_n * g.page_bytes(2), dtype=torch.uint8, device="cuda")
    fill_bf16(torch, src, 1.0, 44, 0.01, 40.0)
    dst = torch.zeros(n_dst * g.page_bytes(1), dtype=torch.uint8, device="cuda")
    scale_page = 2 * g.layers * g.page_tokens * g.kv_heads * 4
    scales = torch.zeros(n_dst * scale_page, dtype=torch.uint8, device="cuda")
    kv = P.shape(g.layers, g.kv_heads, g.head_dim, g.page_tokens)
    hi = ((4 << 30) + g.page_bytes(1) - 1) // g.page_bytes(1)
    rng = np.random.default_rng(44)
    sp = rng.permutation(src_pages_n)[:40]
    dp = rng.permutation(n_dst - hi)[:40] + hi
    runs = P.build_runs(sp.astype(np.int32) * g.stride, dp.astype(np.int32) * g.stride, kv)
    with P.RunList.fp8(P.view_of(src.data_ptr(), src.numel()), P.view_of(dst.data_ptr(), dst.numel()),
                       scales.data_ptr(), scales.numel(), runs, kv) as rl:
        rl.copy_fp8(P.PBE_FP8_SCALE_PER_TOKEN_HEAD, 0, stream_ptr(torch))
    torch.cuda.synchronize()
    # oracle on compact copies: source pages as they are, destination slot k for dp[k]
    src_host = src.cpu().numpy()
    dst_exp = np.zeros(len(dp) * g.page_bytes(1), np.uint8)
    sc_exp = np.zeros(len(dp) * scale_page, np.uint8)
    O.fp8_handoff_token_head(src_host, dst_exp, sc_exp, sp.astype(np.int32) * g.stride,
                             np.arange(len(dp), dtype=np.int32) * g.stride, g.layers,
                             g.page_tokens, g.kv_heads, g.head_dim)
    idx = torch.from_numpy(dp.astype(np.int64)).cuda()
    got = dst.view(n_dst, g.page_bytes(1))[idx].cpu().numpy().reshape(-1)
    got_sc = scales.view(n_dst, scale_page)[idx].cpu().numpy().reshape(-1)
    assert np.array_equal(got, dst_exp), first_diff(got, dst_exp)
    assert np.array_equal(got_sc, sc_exp), first_diff(got_sc, sc_exp)


@pytest.mark.parametrize("mode", [P.PBE_FP8_SCALE_PER_TOKEN_HEAD, P.PBE_FP8_SCALE_TABLE])
@pytest.mark.parametrize("layers,kv_heads,head_dim,n_runs,n_pages", [
    (4, 2, 8, 40, 200),        # one lane per row: rows per slice exceed the wave
    (2, 2, 64, 3, 30),
    (3, 2, 128, 100, 400),
    (1, 1, 512, 20, 60),       # 64 lanes per row
    (2, 2, 64, 512, 1100),     # the contiguous-source path's run limit
    (2, 2, 64, 513, 1100),     # one run past it: the general path
    (1, 1, 8, 30, 120),        # 512-byte source pages: not whole slices, general path
])
def test_fp8_contiguous_sources(torch_cuda, mode, layers, kv_heads, head_dim, n_runs, n_pages):
    """One prefill's pages in one source region, cut into runs whose
    destinations are shuffled one page apart: the FP8 kernel's contiguous-
    source path (a slice's loads before its run) where the pages hold whole
    slices and the list has at most 512 runs, the general path otherwise."""
    torch = torch_cuda
    g = W.Geometry(layers, kv_heads, head_dim)
    rng = np.random.default_rng(n_runs * 7 + head_dim)
    cuts = np.sort(rng.choice(np.arange(1, n_pages), n_runs - 1, replace=False))
    lengths = np.diff(np.concatenate(([0], cuts, [n_pages])))
    starts = np.empty(n_runs, np.int64)
    at = 0
    for r in rng.permutation(n_runs):
        starts[r] = at
        at += lengths[r] + 1
    dst_pages = np.concatenate([np.arange(s, s + n) for s, n in zip(starts, lengths)])
    pools = Fp8Pools(torch, g, max(n_pages, at))
    fill_bf16(torch, pools.src, 1.0, n_runs, 0.01, 40.0)
    src = (np.arange(n_pages) * g.stride).astype(np.int32)
    dst = (dst_pages * g.stride).astype(np.int32)
    assert len(P.build_runs(src, dst, pools.kv)) == n_runs
    amax = rng.uniform(2.5, 5.0, (2 * g.layers, g.kv_heads))
    say(f"fp8 contiguous sources mode={mode} L={layers} H={kv_heads} D={head_dim} runs={n_runs}")
    _check(torch, pools, src, dst, mode, amax)


@pytest.mark.parametrize("mode", [P.PBE_FP8_SCALE_PER_TOKEN_HEAD, P.PBE_FP8_SCALE_TABLE])
def test_fp8_scattered_sources_many_runs(torch_cuda, mode):
    """The general path at the 1.5B geometry: 200 pages in runs of 1-4 on
    scattered sources, which the run list reorders by destination address;
    destinations, scales and every other byte against the oracle."""
    torch = torch_cuda
    n_pages = 4 * 200 + 16
    w = W.small(seed=77, layers=28, kv_heads=2, head_dim=128, n_pages=n_pages, handoff_pages=200,
                max_run=4)
    g = w.geometry
    kv = P.shape(g.layers, g.kv_heads, g.head_dim, g.page_tokens)
    runs = P.build_runs(w.src_ids, w.dst_ids, kv)
    assert len(runs) > 50
    assert any(runs[i][1] > runs[i + 1][1] for i in range(len(runs) - 1))  # not already in dst order
    pools = Fp8Pools(torch, g, n_pages)
    fill_bf16(torch, pools.src, 1.0, 77, 0.001, 40.0)
    amax = np.random.default_rng(77).uniform(2.5, 5.0, (2 * g.layers, g.kv_heads))
    say(f"fp8 scattered many runs mode={mode} runs={len(runs)}")
    _check(torch, pools, w.src_ids, w.dst_ids, mode, amax)
