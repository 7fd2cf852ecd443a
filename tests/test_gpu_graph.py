"""The launches can be captured into a HIP graph (one kernel node each, no
memset nodes) and replayed: a prebuilt run list's handoff copy and a decode
step. Every replay is checked against the oracle, with the program's own eager
work (fresh fills) and synchronisations between replays."""
import numpy as np
import pytest

import pbe_handoff as P
import workload as W
from oracle import oracle as O
from tests.conftest import say
from tests.gpu_util import fill_bf16, first_diff

pytestmark = pytest.mark.gpu


def test_handoff_copy_replays_from_a_graph(torch_cuda):
    torch = torch_cuda
    w = W.small(seed=5, layers=3, kv_heads=2, head_dim=64, n_pages=96, handoff_pages=21, max_run=4)
    g = w.geometry
    kv = P.shape(g.layers, g.kv_heads, g.head_dim, g.page_tokens)
    say(f"graph replay of the handoff copy, {w.pages} pages")
    arena = torch.empty(w.arena_bytes, dtype=torch.uint8, device="cuda")
    view = P.view_of(arena.data_ptr(), arena.numel())
    rl = P.RunList.bf16(view, view, P.build_runs(w.src_ids, w.dst_ids, kv), kv)
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    fill_bf16(torch, arena, 1.0, 1)
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rl.copy(side.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(4):
        fill_bf16(torch, arena, 1.0, 100 + rep)  # eager work between replays
        torch.cuda.synchronize()
        expected = arena.cpu().numpy().copy()
        O.copy_handoff(expected, w.src_ids, w.dst_ids, g.half(), g.layers)
        graph.replay()
        torch.cuda.synchronize()
        got = arena.cpu().numpy()
        assert np.array_equal(got, expected), (rep, first_diff(got, expected))
    rl.close()


def test_decode_step_replays_from_a_graph(torch_cuda):
    from tests.test_gpu_decode import DecodeCase, close
    torch = torch_cuda
    say("graph replay of a decode step (FP8 pages)")
    case = DecodeCase(torch, fp8=True, layers=2, H=2, D=128, kvm=6, seq_lens=[300, 17, 0, 129],
                      seed=12)
    want = case.oracle()
    ws_bytes = P.decode_workspace_bytes(case.batch, case.H * case.kvm, case.D, 8)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            P.paged_decode(case.view, P.PBE_KV_FP8_E4M3, case.scales.data_ptr(),
                           case.scales.numel() * 4, case.kv, case.layer, case.q.data_ptr(),
                           case.out.data_ptr(), case.batch, case.H * case.kvm,
                           case.t_dev.data_ptr(), case.s_dev.data_ptr(), case.max_blocks, 8,
                           ws.data_ptr(), ws_bytes, side.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(4):
        case.out.fill_(rep + 1)  # eager work between replays: the output is overwritten
        ws.fill_(0xA5 + rep)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = (case.out.cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        assert close(got.astype(np.float64), want).all(), rep


def test_staged_calls_refuse_capture(torch_cuda):
    """pbe_copy_ops with more than 112 spans and pbe_copy_shared_kv with more
    than 112 runs whose sources are scattered stage their lists in a reused ring, so under capture they return
    PBE_ERR_UNSUPPORTED before queueing anything; the prebuilt run list
    captured in the same graph still replays correctly. A short op list rides
    in the kernel arguments and is captured like a prebuilt run list."""
    torch = torch_cuda
    w = W.small(seed=9, layers=2, kv_heads=2, head_dim=64, n_pages=640, handoff_pages=150,
                max_run=1)
    g = w.geometry
    kv = P.shape(g.layers, g.kv_heads, g.head_dim, g.page_tokens)
    say("staged calls under graph capture are refused")
    arena = torch.empty(w.arena_bytes, dtype=torch.uint8, device="cuda")
    view = P.view_of(arena.data_ptr(), arena.numel())
    runs = P.build_runs(w.src_ids, w.dst_ids, kv)
    assert len(runs) > 112
    rl = P.RunList.bf16(view, view, runs, kv)
    half = g.half()
    base = arena.data_ptr()
    # every page's first plane only: 150 spans that do not merge
    ops = P.op_array([(base + int(s) * half, base + int(d) * half, half)
                      for s, d in zip(w.src_ids.tolist(), w.dst_ids.tolist())])
    assert ops[1] > 112
    # source plane s of four pages onto plane d+1 of their destination pages,
    # which the handoff in the same graph first fills with plane s+1
    few = [(base + int(s) * half, base + (int(d) + 1) * half, half)
           for s, d in zip(w.src_ids[:4].tolist(), w.dst_ids[:4].tolist())]
    fill_bf16(torch, arena, 1.0, 3)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            with pytest.raises(P.PbeError, match="captured"):
                P.copy_ops(ops, 0, side.cuda_stream)
            with pytest.raises(P.PbeError, match="captured"):
                P.copy_shared_kv(view, w.src_ids, w.dst_ids, kv, 0, side.cuda_stream)
            rl.copy(side.cuda_stream)
            P.copy_ops(few, 0, side.cuda_stream)  # kernel-argument form: captured
    torch.cuda.synchronize()
    for rep in range(3):
        fill_bf16(torch, arena, 1.0, 40 + rep)
        torch.cuda.synchronize()
        expected = arena.cpu().numpy().copy()
        O.copy_handoff(expected, w.src_ids, w.dst_ids, g.half(), g.layers)
        for s_, d_, n_ in few:
            expected[d_ - base:d_ - base + n_] = expected[s_ - base:s_ - base + n_]
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(arena.cpu().numpy(), expected), rep
    # outside capture the same calls work
    P.copy_ops(ops, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    rl.close()


@pytest.mark.parametrize("fused", [False, True])
def test_decode_loop_step_replays_from_a_graph(torch_cuda, fused):
    """One decode step of a serving loop, captured once: the new token's K/V
    written to its page slot (pbe_scatter_kv, FP8 local pools) and attention
    over the pools (pbe_paged_decode_pools), or both in the reader's launch
    (pbe_paged_decode_append, fused). Between replays the host writes the
    next token's K/V, slots, lengths and queries into the captured buffers, as a
    loop would. Each replay's pools equal the oracle's bit for bit and its output
    is within the reader's tolerance of the float64 oracle."""
    from tests.test_gpu_decode import bf16_to_f64, close
    torch = torch_cuda
    say(f"graph replay of scatter + decode over FP8 pools, fused={fused}")
    rng = np.random.default_rng(61)
    H, D, kvm, B, n_blocks = 2, 128, 6, 16, 24
    half, plane = B * H * D, B * H
    lens = [30, 15, 47]                       # two of them cross a block boundary below
    batch = len(lens)
    tables = rng.permutation(n_blocks)[: batch * 4].reshape(batch, 4).astype(np.int32)
    kp = rng.integers(0, 0x7F, n_blocks * half, dtype=np.uint8)   # no NaN codes
    vp = rng.integers(0, 0x7F, n_blocks * half, dtype=np.uint8)
    ks = rng.uniform(1e-3, 0.05, n_blocks * plane).astype(np.float32)
    vs = rng.uniform(1e-3, 0.05, n_blocks * plane).astype(np.float32)
    d = {k: torch.from_numpy(v.copy()).cuda() for k, v in
         dict(kp=kp, vp=vp, ks=ks, vs=vs, tab=tables).items()}
    new_k = torch.zeros((batch, H * D), dtype=torch.int16, device="cuda")
    new_v = torch.zeros_like(new_k)
    slots = torch.zeros(batch, dtype=torch.int32, device="cuda")
    seq = torch.zeros(batch, dtype=torch.int32, device="cuda")
    q = torch.zeros((batch, H * kvm, D), dtype=torch.int16, device="cuda")
    out = torch.zeros_like(q)
    splits = 2
    ws_bytes = P.decode_workspace_bytes(batch, H * kvm, D, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            if fused:
                P.paged_decode_append(d["kp"].data_ptr(), d["vp"].data_ptr(), n_blocks * half,
                                      d["ks"].data_ptr(), d["vs"].data_ptr(), n_blocks * plane * 4,
                                      P.PBE_KV_FP8_E4M3, H, D, new_k.data_ptr(), new_v.data_ptr(),
                                      q.data_ptr(), out.data_ptr(), batch, H * kvm, d["tab"].data_ptr(),
                                      seq.data_ptr(), 4, splits, ws.data_ptr(), ws_bytes, side.cuda_stream)
            else:
                P.scatter_kv(new_k.data_ptr(), new_v.data_ptr(), P.PBE_IN_BF16, batch, slots.data_ptr(),
                             B, H, D, P.PBE_KV_FP8_E4M3, d["kp"].data_ptr(), n_blocks * half,
                             d["vp"].data_ptr(), n_blocks * half, d["ks"].data_ptr(), n_blocks * plane * 4,
                             d["vs"].data_ptr(), n_blocks * plane * 4, stream=side.cuda_stream)
                P.paged_decode_pools(d["kp"].data_ptr(), d["vp"].data_ptr(), n_blocks * half,
                                     d["ks"].data_ptr(), d["vs"].data_ptr(), n_blocks * plane * 4,
                                     P.PBE_KV_FP8_E4M3, H, D, q.data_ptr(), out.data_ptr(), batch,
                                     H * kvm, d["tab"].data_ptr(), seq.data_ptr(), 4, splits,
                                     ws.data_ptr(), ws_bytes, side.cuda_stream)
    torch.cuda.synchronize()
    for step in range(4):
        K = O.bf16_from_f32(rng.standard_normal((batch, H * D)).astype(np.float32))
        V = O.bf16_from_f32(rng.standard_normal((batch, H * D)).astype(np.float32))
        qh = O.bf16_from_f32(rng.standard_normal((batch, H * kvm, D)).astype(np.float32))
        s = np.array([tables[b, lens[b] // B] * B + lens[b] % B for b in range(batch)], np.int32)
        lens = [n + 1 for n in lens]
        new_k.copy_(torch.from_numpy(K.view(np.int16)))
        new_v.copy_(torch.from_numpy(V.view(np.int16)))
        slots.copy_(torch.from_numpy(s))
        seq.copy_(torch.tensor(lens, dtype=torch.int32))
        q.copy_(torch.from_numpy(qh.view(np.int16)))
        out.fill_(step + 1)
        torch.cuda.synchronize()
        O.scatter_kv(K, V, s, B, H, D, True, kp, vp, ks, vs)
        graph.replay()
        torch.cuda.synchronize()
        for name, host in (("kp", kp), ("vp", vp), ("ks", ks), ("vs", vs)):
            assert np.array_equal(d[name].cpu().numpy().view(np.uint8), host.view(np.uint8)), (step, name)
        want = O.paged_decode_pools(kp, vp, True, ks, vs, H, D, qh, tables, lens)
        got = bf16_to_f64(out.cpu().numpy().view(np.uint16))
        assert close(got, want).all(), step


def test_one_region_plan_of_150_runs_is_captured(torch_cuda):
    """A one-region plan (one prefill's pages) of 150 runs travels in the
    kernel arguments as run starts and destinations, so pbe_copy_shared_kv is
    captured (more than the 112 runs the record form holds) and every replay
    matches the oracle."""
    from tests.test_gpu_handoff import _contiguous_source_plan, _kv
    torch = torch_cuda
    g = W.Geometry(2, 2, 64)
    kv = _kv(g)
    src, dst, total = _contiguous_source_plan(g, 150, 400, 77)
    assert len(P.build_runs(src, dst, kv)) == 150
    say("graph capture of a one-region 150-run pbe_copy_shared_kv")
    arena = torch.empty((total + 3) * g.page_bytes(), dtype=torch.uint8, device="cuda")
    view = P.view_of(arena.data_ptr(), arena.numel())
    fill_bf16(torch, arena, 1.0, 5)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            P.copy_shared_kv(view, src, dst, kv, 0, side.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(3):
        fill_bf16(torch, arena, 1.0, 60 + rep)
        torch.cuda.synchronize()
        expected = arena.cpu().numpy().copy()
        O.copy_handoff(expected, src, dst, g.half(), g.layers)
        graph.replay()
        torch.cuda.synchronize()
        got = arena.cpu().numpy()
        assert np.array_equal(got, expected), (rep, first_diff(got, expected))
