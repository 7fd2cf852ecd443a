"""End to end on the GPU: a finished prefill's BF16 pages are handed off into
decode-owned FP8 pages (fused quantisation, per-token-head scales), and the
decode reader then attends over exactly those pages. Checked against the
oracle chain: the FP8 handoff restated on the host, then the float64 decode."""
import numpy as np
import pytest

import pbe_handoff as P
import workload as W
from oracle import oracle as O
from tests.conftest import say
from tests.gpu_util import fill_bf16, stream_ptr
from tests.test_gpu_decode import bf16_to_f64, close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fp8", [True, False])
def test_prefill_pages_handed_off_then_decoded(torch_cuda, fp8):
    torch = torch_cuda
    g = W.Geometry(layers=4, kv_heads=2, head_dim=128)
    kvm, layer, n_pages = 6, 3, 48
    seq_lens = [150, 160, 1, 0]
    need = [(n + 15) // 16 for n in seq_lens]
    say(f"handoff (fp8={fp8}) then decode, L{g.layers} H{g.kv_heads} D{g.head_dim}")
    rng = np.random.default_rng(21 + fp8)
    kv = P.shape(g.layers, g.kv_heads, g.head_dim, g.page_tokens)
    E = 1 if fp8 else 2
    src = torch.empty(n_pages * g.page_bytes(2), dtype=torch.uint8, device="cuda")
    fill_bf16(torch, src, 1.0, 5, outlier_fraction=0.001)
    dst = torch.zeros(n_pages * g.page_bytes(E), dtype=torch.uint8, device="cuda")
    scale_page = 2 * g.layers * g.page_tokens * g.kv_heads * 4
    scales = torch.zeros(n_pages * scale_page, dtype=torch.uint8, device="cuda")
    # the prefill's pages (scattered) and the decode pages reserved for them
    total = sum(need)
    src_pages = rng.permutation(n_pages)[:total]
    dst_pages = rng.permutation(n_pages)[:total]
    src_ids = (src_pages * g.stride).astype(np.int32)
    dst_ids = (dst_pages * g.stride).astype(np.int32)
    src_view = P.view_of(src.data_ptr(), src.numel())
    dst_view = P.view_of(dst.data_ptr(), dst.numel())
    runs = P.build_runs(src_ids, dst_ids, kv)
    src_host = src.cpu().numpy()
    dst_exp = dst.cpu().numpy().copy()
    sc_exp = scales.cpu().numpy().copy().view(np.uint8)
    if fp8:
        with P.RunList.fp8(src_view, dst_view, scales.data_ptr(), scales.numel(), runs, kv) as rl:
            rl.copy_fp8(P.PBE_FP8_SCALE_PER_TOKEN_HEAD, 0, stream_ptr(torch))
        O.fp8_handoff_token_head(src_host, dst_exp, sc_exp, src_ids, dst_ids, g.layers,
                                 g.page_tokens, g.kv_heads, g.head_dim)
    else:
        with P.RunList.bf16(src_view, dst_view, runs, kv) as rl:
            rl.copy(stream_ptr(torch))
        # a BF16 handoff between two arenas: the destination pages take the source bytes
        page = g.page_bytes(2)
        for s, d in zip(src_pages, dst_pages):
            dst_exp[d * page:(d + 1) * page] = src_host[s * page:(s + 1) * page]
    torch.cuda.synchronize()
    dst_host = dst.cpu().numpy()
    assert np.array_equal(dst_host, dst_exp)
    if fp8:
        assert np.array_equal(scales.cpu().numpy(), sc_exp)

    # decode over the destination pages, in sequence order
    batch = len(seq_lens)
    max_blocks = max(need)
    tables = np.zeros((batch, max_blocks), np.int32)
    k = 0
    for b, nb in enumerate(need):
        tables[b, :nb] = dst_ids[k:k + nb]
        k += nb
    qf = rng.standard_normal((batch, g.kv_heads * kvm, g.head_dim)).astype(np.float32)
    q_host = O.bf16_from_f32(qf)
    q = torch.from_numpy(q_host.view(np.int16)).cuda()
    out = torch.empty_like(q)
    t_dev = torch.from_numpy(tables).cuda()
    s_dev = torch.tensor(seq_lens, dtype=torch.int32, device="cuda")
    splits = P.decode_splits(batch, g.kv_heads, max_blocks, P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16)
    ws_bytes = P.decode_workspace_bytes(batch, g.kv_heads * kvm, g.head_dim, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    P.paged_decode(dst_view, P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16,
                   scales.data_ptr() if fp8 else 0, scales.numel() if fp8 else 0, kv, layer,
                   q.data_ptr(), out.data_ptr(), batch, g.kv_heads * kvm, t_dev.data_ptr(),
                   s_dev.data_ptr(), max_blocks, splits, ws.data_ptr(), ws_bytes, stream_ptr(torch))
    torch.cuda.synchronize()
    got = bf16_to_f64(out.cpu().numpy().view(np.uint16))
    want = O.paged_decode(dst_exp, fp8, sc_exp.view(np.float32) if fp8 else None, g.layers,
                          g.kv_heads, g.head_dim, layer, q_host, tables, seq_lens)
    assert close(got, want).all()
    assert not got[3].any()  # the empty sequence
    if fp8:
        # the quantised pages stay close to the prefill's BF16 values: decoding
        # the source pages directly differs by the FP8 rounding only
        src_tables = np.zeros_like(tables)
        k = 0
        for b, nb in enumerate(need):
            src_tables[b, :nb] = src_ids[k:k + nb]
            k += nb
        ref = O.paged_decode(src_host, False, None, g.layers, g.kv_heads, g.head_dim, layer,
                             q_host, src_tables, seq_lens)
        assert np.abs(got - ref).max() <= 0.1 * np.abs(ref).max()
