"""GPU parity of pbe_paged_decode_pools: the decode reader over per-layer K/V
pools, the calling convention of the reference's decode kernels
(paged_kv_runtime.cpp:293-357 passes a KVPoolView's key/value pools).

- A shared arena's layer views (key = arena + 2l*half, value = key + half,
  page-major ids) read the same bytes as pbe_paged_decode over the arena, so
  the outputs must be bit-identical at the same split count.
- Separate local K and V pools (and scale pools), into which every used block
  was copied under a new id with the tables renumbered: bit-identical again,
  and within the reader's tolerance of the float64 pool-addressed oracle.
- A block id whose rows or scales end past the pools gives NaN for its
  sequence only; argument errors are rejected before any launch.
"""
import numpy as np
import pytest

import pbe_handoff as P
from oracle import oracle as O
from tests.conftest import say
from tests.gpu_util import stream_ptr
from tests.test_gpu_decode import DecodeCase, bf16_to_f64, close

pytestmark = pytest.mark.gpu


def _run_pools(case, key, value, pool_bytes, ks, vs, scale_bytes, tables, splits, seq_lens=None):
    torch = case.torch
    ws_bytes = P.decode_workspace_bytes(case.batch, case.H * case.kvm, case.D, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    case.out.fill_(0)
    sl = case.s_dev if seq_lens is None else seq_lens
    P.paged_decode_pools(key, value, pool_bytes, ks, vs, scale_bytes,
                         P.PBE_KV_FP8_E4M3 if case.fp8 else P.PBE_KV_BF16, case.H, case.D,
                         case.q.data_ptr(), case.out.data_ptr(), case.batch, case.H * case.kvm,
                         tables.data_ptr(), sl.data_ptr(), case.max_blocks, splits, ws.data_ptr(),
                         ws_bytes, stream_ptr(torch))
    torch.cuda.synchronize()
    return case.out.cpu().numpy().view(np.uint16).copy()


@pytest.mark.parametrize("fp8", [True, False])
def test_layer_views_of_the_arena_equal_the_arena_reader(torch_cuda, fp8):
    say(f"decode pools fp8={fp8}: layer views of one arena")
    case = DecodeCase(torch_cuda, fp8=fp8, layers=3, H=2, D=128, kvm=6,
                      seq_lens=[0, 1, 17, 300, 129, 64], seed=51, layer=1)
    assert len(case.bufs) == 1
    splits = P.decode_splits(case.batch, case.H, case.max_blocks,
                             P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16)
    case.run(splits=splits)
    want_bits = case.out.cpu().numpy().view(np.uint16).copy()
    base, total = case.bufs[0].data_ptr(), case.bufs[0].numel()
    k_off = 2 * case.layer * case.half
    plane = 16 * case.H
    ks = case.scales.data_ptr() + 4 * 2 * case.layer * plane if fp8 else 0
    vs = ks + 4 * plane if fp8 else 0
    s_bytes = case.scales.numel() * 4 - 4 * (2 * case.layer + 1) * plane if fp8 else 0
    got = _run_pools(case, base + k_off, base + k_off + case.half, total - k_off - case.half, ks, vs,
                     s_bytes, case.t_dev, splits)
    assert np.array_equal(got, want_bits)
    assert close(bf16_to_f64(got), case.oracle()).all()


@pytest.mark.parametrize("fp8", [True, False])
@pytest.mark.parametrize("D", [128, 64])
def test_local_pools_with_renumbered_blocks(torch_cuda, fp8, D):
    torch = torch_cuda
    say(f"decode pools fp8={fp8} D={D}: separate local pools")
    case = DecodeCase(torch, fp8=fp8, layers=2, H=2, D=D, kvm=4,
                      seq_lens=[33, 200, 1, 64, 0, 150], seed=52 + D, layer=0)
    splits = P.decode_splits(case.batch, case.H, case.max_blocks,
                             P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16)
    case.run(splits=splits)
    want_bits = case.out.cpu().numpy().view(np.uint16).copy()
    rng = np.random.default_rng(D)
    used = sorted({int(x) for x in case.tables.ravel() if x >= 0})
    n = len(used) + 3
    new_id = dict(zip(used, (rng.permutation(n)[: len(used)]).tolist()))
    half, plane = case.half, 16 * case.H
    kp = rng.integers(0, 256, n * half, dtype=np.uint8)  # unused blocks hold noise
    vp = rng.integers(0, 256, n * half, dtype=np.uint8)
    ks = np.zeros(n * plane, np.float32)
    vs = np.zeros(n * plane, np.float32)
    for old, new in new_id.items():
        k_plane, v_plane = old + 2 * case.layer, old + 2 * case.layer + 1
        kp[new * half:(new + 1) * half] = case.host[k_plane * half:(k_plane + 1) * half]
        vp[new * half:(new + 1) * half] = case.host[v_plane * half:(v_plane + 1) * half]
        if fp8:
            ks[new * plane:(new + 1) * plane] = case.host_scales[k_plane * plane:(k_plane + 1) * plane]
            vs[new * plane:(new + 1) * plane] = case.host_scales[v_plane * plane:(v_plane + 1) * plane]
    tables = np.vectorize(lambda x: new_id.get(int(x), -1))(case.tables).astype(np.int32)
    # V before K in memory: the reader must not assume an order between the pools
    dv = torch.from_numpy(vp).cuda()
    dk = torch.from_numpy(kp).cuda()
    dks = torch.from_numpy(ks).cuda()
    dvs = torch.from_numpy(vs).cuda()
    dt = torch.from_numpy(tables).cuda()
    got = _run_pools(case, dk.data_ptr(), dv.data_ptr(), n * half,
                     dks.data_ptr() if fp8 else 0, dvs.data_ptr() if fp8 else 0,
                     n * plane * 4 if fp8 else 0, dt, splits)
    assert np.array_equal(got, want_bits)
    want = O.paged_decode_pools(kp, vp, fp8, ks if fp8 else None, vs if fp8 else None, case.H,
                                case.D, case.q_host, tables, case.seq_lens)
    assert close(bf16_to_f64(got), want).all()
    # a block id just past the pools: NaN for that sequence only
    bad = tables.copy()
    bad[1, 3] = n
    got_bad = bf16_to_f64(_run_pools(case, dk.data_ptr(), dv.data_ptr(), n * half,
                                     dks.data_ptr() if fp8 else 0, dvs.data_ptr() if fp8 else 0,
                                     n * plane * 4 if fp8 else 0, torch.from_numpy(bad).cuda(),
                                     splits))
    assert np.isnan(got_bad[1]).all()
    others = [b for b in range(case.batch) if b != 1]
    assert close(got_bad[others], want[others]).all()


def test_pool_argument_errors_are_rejected(torch_cuda):
    torch = torch_cuda
    say("decode pools misuse")
    case = DecodeCase(torch, fp8=True, layers=1, H=2, D=128, kvm=6, seq_lens=[20], seed=53, layer=0)
    base = case.bufs[0].data_ptr()
    sc = case.scales.data_ptr()
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    args = dict(key_pool=base, value_pool=base + case.half, pool_bytes=case.bufs[0].numel() - case.half,
                key_scales=sc, value_scales=sc + 4 * 32, scale_pool_bytes=case.scales.numel() * 4 - 128,
                kv_dtype=P.PBE_KV_FP8_E4M3, kv_heads=2, head_dim=128, queries=case.q.data_ptr(),
                outputs=case.out.data_ptr(), batch=1, q_heads=12, tables=case.t_dev.data_ptr(),
                seq_lens=case.s_dev.data_ptr(), max_blocks=case.max_blocks, splits=0,
                workspace=ws.data_ptr(), workspace_bytes=ws.numel())
    P.paged_decode_pools(**args)  # the valid call
    torch.cuda.synchronize()
    for change in [dict(key_pool=base + 8), dict(value_scales=0), dict(key_scales=sc + 2),
                   dict(pool_bytes=case.half - 1), dict(head_dim=96), dict(value_pool=0),
                   dict(pool_bytes=1 << 40)]:  # beyond any allocation (the caching
        # allocator's segments make a small overshoot indistinguishable from valid memory)
        a = dict(args)
        a.update(change)
        try:
            P.paged_decode_pools(**a)
        except P.PbeError:
            continue
        torch.cuda.synchronize()
        pytest.fail(f"accepted {change}")
