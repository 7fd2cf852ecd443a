"""GPU parity of the BF16 handoff copy against the CPU oracle.

Every case fills a device arena with seeded BF16 values, snapshots it, runs the
HIP kernel through the C ABI, and compares the WHOLE arena with the oracle
applied to the snapshot: copied pages must be bit-identical and every byte
outside the destination pages must be unchanged (canary check).
"""
import numpy as np
import pytest

import pbe_handoff as P
import workload as W
from oracle import oracle as O
from tests.conftest import say
from tests.gpu_util import device_arena, fill_bf16, first_diff, snapshot, stream_ptr

pytestmark = pytest.mark.gpu


def _kv(g: W.Geometry) -> P.KvShape:
    return P.shape(g.layers, g.kv_heads, g.head_dim, g.page_tokens)


def _run_runlist_case(torch, w: W.Workload, seed: int, batched: bool = True):
    g = w.geometry
    kv = _kv(g)
    bufs, view = device_arena(torch, w.arena_bytes, w.segment_bytes)
    for i, b in enumerate(bufs):
        fill_bf16(torch, b, w.sigma, seed + i)
    torch.cuda.synchronize()
    before = snapshot(bufs)
    expected = before.copy()
    O.copy_handoff(expected, w.src_ids, w.dst_ids, g.half(), g.layers)
    reqs = [w] if batched else [W.Workload(w.name, g, w.arena_bytes, w.segment_bytes, [r])
                                for r in w.requests]
    for part in reqs:
        runs = P.build_runs(part.src_ids, part.dst_ids, kv, 2, w.segment_bytes)
        with P.RunList.bf16(view, view, runs, kv) as rl:
            info = rl.info()
            assert info.pages == part.pages
            assert info.src_bytes == part.pages * g.page_bytes()
            rl.copy(stream_ptr(torch))
            torch.cuda.synchronize()
    after = snapshot(bufs)
    assert np.array_equal(after, expected), first_diff(after, expected)


@pytest.mark.parametrize("seed", range(16))
def test_small_random_plans(torch_cuda, seed):
    shapes = [(3, 2, 64), (1, 1, 8), (5, 4, 128), (2, 2, 16), (7, 1, 32), (4, 8, 64),
              (28, 2, 128), (24, 2, 64), (1, 3, 24), (9, 5, 40), (2, 1, 256), (6, 6, 8),
              (11, 2, 96), (4, 16, 16), (1, 1, 1024), (3, 7, 56)]
    L, H, D = shapes[seed]
    n = 13 + seed
    w = W.small(seed=seed, layers=L, kv_heads=H, head_dim=D, n_pages=max(96, 4 * n + 12),
                handoff_pages=n, max_run=1 + seed % 6)
    say(f"small seed={seed} L={L} H={H} D={D} pages={w.pages}")
    _run_runlist_case(torch_cuda, w, seed)


def test_small_segmented_arena(torch_cuda):
    w = W.small(seed=11, layers=2, kv_heads=2, head_dim=64, n_pages=120, handoff_pages=20,
                max_run=6, segment_pages=40)
    say(f"segmented small pages={w.pages} segs={w.arena_bytes // w.segment_bytes}")
    _run_runlist_case(torch_cuda, w, 11)


def test_config1_qwen05b(torch_cuda):
    w = W.config1(0)
    say("config1")
    _run_runlist_case(torch_cuda, w, 1)


def test_config2_qwen15b_5040(torch_cuda):
    w = W.config2(0)
    say("config2")
    _run_runlist_case(torch_cuda, w, 2)


@pytest.mark.parametrize("batched", [True, False])
def test_config3_multi_request(torch_cuda, batched):
    w = W.config3(0)
    say(f"config3 batched={batched}")
    _run_runlist_case(torch_cuda, w, 3, batched=batched)


def test_config5_segmented_7b(torch_cuda):
    w = W.config5(0)
    say("config5 in-process, 3 segments")
    _run_runlist_case(torch_cuda, w, 5)


def test_copy_shared_kv_one_call(torch_cuda):
    torch = torch_cuda
    w = W.config2(1)
    g = w.geometry
    kv = _kv(g)
    say("pbe_copy_shared_kv config2 seed1")
    bufs, view = device_arena(torch, w.arena_bytes)
    fill_bf16(torch, bufs[0], w.sigma, 7)
    torch.cuda.synchronize()
    before = snapshot(bufs)
    expected = before.copy()
    ref_bytes = O.copy_handoff(expected, w.src_ids, w.dst_ids, g.half(), g.layers)
    copied = P.copy_shared_kv(view, w.src_ids, w.dst_ids, kv, 0, stream_ptr(torch))
    torch.cuda.synchronize()
    assert copied == ref_bytes == w.copied_bytes()
    after = snapshot(bufs)
    assert np.array_equal(after, expected), first_diff(after, expected)
    # a second call reuses the staging buffer
    w2 = W.config2(2)
    expected2 = after.copy()
    O.copy_handoff(expected2, w2.src_ids, w2.dst_ids, g.half(), g.layers)
    P.copy_shared_kv(view, w2.src_ids, w2.dst_ids, kv, 0, stream_ptr(torch))
    torch.cuda.synchronize()
    after2 = snapshot(bufs)
    assert np.array_equal(after2, expected2), first_diff(after2, expected2)


def test_copy_shared_kv_back_to_back_without_sync(torch_cuda):
    """More one-call handoffs in flight than staging slots: the ring wraps onto
    slots whose launch may still run, and slot buffers grow between calls."""
    torch = torch_cuda
    w = W.config3(0)
    g = w.geometry
    kv = _kv(g)
    say(f"pbe_copy_shared_kv back-to-back config3 requests={len(w.requests)}")
    bufs, view = device_arena(torch, w.arena_bytes, w.segment_bytes)
    for i, b in enumerate(bufs):
        fill_bf16(torch, b, w.sigma, 40 + i)
    torch.cuda.synchronize()
    expected = snapshot(bufs)
    # chunks of 1, 2, 4, ... pages: more calls than slots, each larger than the last
    src, dst = w.src_ids, w.dst_ids
    total, start, k, calls = 0, 0, 1, 0
    while start < len(src):
        s, d = src[start:start + k], dst[start:start + k]
        total += O.copy_handoff(expected, s, d, g.half(), g.layers)
        total -= P.copy_shared_kv(view, s, d, kv, 0, stream_ptr(torch))
        start, k, calls = start + k, 2 * k, calls + 1
    assert calls > 8
    # both launch forms ran: short run lists travel in the kernel arguments,
    # long ones through the staging ring
    sizes = [len(P.build_runs(src[a:a + k], dst[a:a + k], kv))
             for a, k in ((2 ** i - 1, 2 ** i) for i in range(calls)) if a < len(src)]
    assert min(sizes) <= 112 < max(sizes), sizes
    torch.cuda.synchronize()
    assert total == 0
    after = snapshot(bufs)
    assert np.array_equal(after, expected), first_diff(after, expected)


def test_copy_shared_kv_rejects_bad_ids_before_any_write(torch_cuda):
    torch = torch_cuda
    w = W.small(seed=3, n_pages=32, handoff_pages=5)
    g = w.geometry
    kv = _kv(g)
    bufs, view = device_arena(torch, w.arena_bytes)
    fill_bf16(torch, bufs[0], 1.0, 3)
    torch.cuda.synchronize()
    before = snapshot(bufs)
    bad = [
        (w.src_ids + 1, w.dst_ids),                                   # not a page id
        (w.src_ids, np.where(np.arange(w.pages) == 2, -g.stride, w.dst_ids)),  # negative
        (w.src_ids, np.full(w.pages, 32 * g.stride)),                 # past the arena
        (w.src_ids, w.src_ids),                                       # overwrite own source
        (w.src_ids, np.full(w.pages, w.dst_ids[0])),                  # dst written twice
    ]
    for i, (s, d) in enumerate(bad):
        say(f"bad ids case {i}")
        with pytest.raises(P.PbeError) as e:
            P.copy_shared_kv(view, s, d, kv, 0, stream_ptr(torch))
        assert e.value.code == P.PBE_ERR_INVALID
    torch.cuda.synchronize()
    assert np.array_equal(snapshot(bufs), before)


def test_runlist_rejects_foreign_memory(torch_cuda):
    torch = torch_cuda
    kv = P.shape(2, 2, 64)
    host = np.zeros(8 * kv.page_bytes(), np.uint8)
    view = P.view_of(host.ctypes.data, host.nbytes)
    with pytest.raises(P.PbeError) as e:
        P.RunList.bf16(view, view, [(0, 4 * kv.layers * 2, 1)], kv)
    assert e.value.code == P.PBE_ERR_INVALID


def test_component_ops_match_generic_plan(torch_cuda):
    """The generic plan form (2*layers component copies per page,
    pd_handoff.cpp:192-213) through pbe_copy_ops equals the run copy."""
    torch = torch_cuda
    w = W.small(seed=5, layers=3, kv_heads=2, head_dim=64, n_pages=64, handoff_pages=11)
    g = w.geometry
    say("copy_ops component form")
    bufs, view = device_arena(torch, w.arena_bytes)
    fill_bf16(torch, bufs[0], 1.0, 5)
    torch.cuda.synchronize()
    before = snapshot(bufs)
    expected = before.copy()
    O.copy_components(expected, w.src_ids, w.dst_ids, g.half(), g.layers)
    base = bufs[0].data_ptr()
    half = g.half()
    ops = []
    for s, d in zip(w.src_ids.tolist(), w.dst_ids.tolist()):
        for plane in range(2 * g.layers):
            ops.append((base + (s + plane) * half, base + (d + plane) * half, half))
    P.copy_ops(ops, 0, stream_ptr(torch))
    torch.cuda.synchronize()
    after = snapshot(bufs)
    assert np.array_equal(after, expected), first_diff(after, expected)
    # unaligned byte ops take the byte path
    torch.cuda.synchronize()
    src_off, dst_off = 3, 5 * half + 7
    P.copy_ops([(base + src_off, base + dst_off, 37)], 0, stream_ptr(torch))
    torch.cuda.synchronize()
    after2 = snapshot(bufs)
    exp2 = after.copy()
    exp2[dst_off:dst_off + 37] = after[src_off:src_off + 37]
    assert np.array_equal(after2, exp2), first_diff(after2, exp2)
    # 16-byte aligned ops of ragged sizes: partial rounds, ops split into
    # several pieces, and the bytes around each destination left alone
    sizes = [16, 1040, 8192 + 16, 2 * 16384 + 48]
    ops, exp3, at = [], after2.copy(), 0
    for n in sizes:
        src_off, dst_off = at, 40 * half + at + 32
        ops.append((base + src_off, base + dst_off, n))
        exp3[dst_off:dst_off + n] = after2[src_off:src_off + n]
        at += n + 4096
    assert 40 * half + at < len(exp3)
    P.copy_ops(ops, 0, stream_ptr(torch))
    torch.cuda.synchronize()
    after3 = snapshot(bufs)
    assert np.array_equal(after3, exp3), first_diff(after3, exp3)


def test_copy_ops_beyond_one_grid(torch_cuda):
    """More op pieces than one grid holds (16,384 workgroups x 4 waves): each
    wave walks several pieces in the grid-stride loop."""
    torch = torch_cuda
    n = 70000
    say(f"copy_ops {n} ops of 32 B")
    src = torch.randint(0, 256, (n * 32,), dtype=torch.uint8, device="cuda")
    dst = torch.zeros(n * 64, dtype=torch.uint8, device="cuda")
    rng = np.random.default_rng(12)
    perm = rng.permutation(n)  # op i writes slot perm[i] of dst, every other 32 B
    sb, db = src.data_ptr(), dst.data_ptr()
    ops = [(sb + 32 * i, db + 64 * int(perm[i]), 32) for i in range(n)]
    P.copy_ops(ops, 0, stream_ptr(torch))
    torch.cuda.synchronize()
    s_host = src.cpu().numpy().reshape(n, 32)
    d_host = dst.cpu().numpy().reshape(n, 64)
    expected = np.zeros((n, 64), np.uint8)
    expected[perm, :32] = s_host
    assert np.array_equal(d_host, expected)


def test_copy_ops_merging_keeps_every_op(torch_cuda):
    """Ops that continue the previous op on both sides are merged before
    staging; the result must equal the ops applied one by one. Cases: runs of
    adjacent ops (merged), the same ops in reverse order (not merged), odd
    sizes and offsets (byte path), and a chain whose merged span would overlap
    its own source (rejected before anything is written)."""
    torch = torch_cuda
    say("copy_ops merging: adjacent, reversed, odd sizes, self-overlap")
    rng = np.random.default_rng(21)
    nbytes = 4 << 20
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda")
    dst = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    sb, db = src.data_ptr(), dst.data_ptr()
    ops, cur_s, cur_d = [], 0, 0
    for k in range(200):
        size = int(rng.choice([16, 4096, 8192, 24, 1000, 16 * 1024 + 16]))
        n = int(rng.integers(1, 6))
        chain = [(cur_s + i * size, cur_d + i * size, size) for i in range(n)]
        if k % 3 == 1:
            chain.reverse()             # adjacent in memory, listed backwards
        ops.extend(chain)
        cur_s += n * size + int(rng.integers(0, 3)) * 16 + (k % 5)   # gaps, odd offsets
        cur_d += n * size + int(rng.integers(0, 3)) * 32
        if cur_s + 6 * 20000 > nbytes or cur_d + 6 * 20000 > nbytes:
            break
    P.copy_ops([(sb + s, db + d, b) for s, d, b in ops], 0, stream_ptr(torch))
    torch.cuda.synchronize()
    s_host = src.cpu().numpy()
    expected = np.zeros(nbytes, np.uint8)
    for s, d, b in ops:
        expected[d:d + b] = s_host[s:s + b]
    assert np.array_equal(dst.cpu().numpy(), expected)
    # a chain whose merged span overlaps its own source: op 1 reads what op 0 wrote
    before = dst.cpu().numpy().copy()
    bad = [(db + 0, db + 8192, 8192), (db + 8192, db + 16384, 8192)]
    with pytest.raises(P.PbeError, match="overwrites its own source"):
        P.copy_ops(bad, 0, stream_ptr(torch))
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), before)


def test_aligned_op_lists_on_both_sides_of_the_kernel_argument_limit(torch_cuda):
    """16-byte aligned op lists run on the run-list kernel: up to 112 spans in
    the kernel arguments, more through the staging ring. Spans of any 16-byte
    multiple (a partial last 2 KiB slice is clamped by the buffer resource),
    scattered destinations, at 1, 112 and 113 spans."""
    torch = torch_cuda
    rng = np.random.default_rng(33)
    nbytes = 8 << 20
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda")
    dst = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    sb, db = src.data_ptr(), dst.data_ptr()
    for n_spans in (1, 112, 113):
        say(f"copy_ops aligned, {n_spans} spans")
        dst.zero_()
        sizes = (rng.integers(1, 2500, n_spans) * 16).tolist()
        slot = 40000  # destinations in disjoint slots, shuffled; sources back to back with gaps
        order = rng.permutation(n_spans)
        ops, s_off = [], 0
        for i, size in enumerate(sizes):
            ops.append((s_off, int(order[i]) * slot, size))
            s_off += size + 16 * int(rng.integers(1, 4))
        P.copy_ops([(sb + s, db + d, b) for s, d, b in ops], 0, stream_ptr(torch))
        torch.cuda.synchronize()
        s_host = src.cpu().numpy()
        expected = np.zeros(nbytes, np.uint8)
        for s, d, b in ops:
            expected[d:d + b] = s_host[s:s + b]
        assert np.array_equal(dst.cpu().numpy(), expected), n_spans


def test_repeated_launches_are_idempotent(torch_cuda):
    torch = torch_cuda
    w = W.config2(3)
    g = w.geometry
    kv = _kv(g)
    say("repeat launches config2 seed3")
    bufs, view = device_arena(torch, w.arena_bytes)
    fill_bf16(torch, bufs[0], w.sigma, 9)
    torch.cuda.synchronize()
    before = snapshot(bufs)
    expected = before.copy()
    O.copy_handoff(expected, w.src_ids, w.dst_ids, g.half(), g.layers)
    runs = P.build_runs(w.src_ids, w.dst_ids, kv)
    with P.RunList.bf16(view, view, runs, kv) as rl:
        for _ in range(5):
            rl.copy(stream_ptr(torch))
        torch.cuda.synchronize()
    after = snapshot(bufs)
    assert np.array_equal(after, expected), first_diff(after, expected)


def test_more_than_4096_runs_three_level_search(torch_cuda):
    """6000 single-page runs: the wave-parallel run search needs three levels
    (64 x 64 < 6000), on a geometry whose page is not a slice multiple."""
    torch = torch_cuda
    g = W.Geometry(1, 1, 24)                 # half 768 B, page 1536 B
    n_pages = 13000
    rng = np.random.default_rng(6)
    pages = rng.permutation(n_pages)[:12000]
    src = (pages[:6000] * g.stride).astype(np.int32)
    dst = (pages[6000:] * g.stride).astype(np.int32)
    kv = _kv(g)
    runs = P.build_runs(src, dst, kv)
    assert len(runs) > 4096
    say(f"three-level search: {len(runs)} runs")
    bufs, view = device_arena(torch, n_pages * g.page_bytes())
    fill_bf16(torch, bufs[0], 1.0, 66)
    torch.cuda.synchronize()
    expected = snapshot(bufs).copy()
    O.copy_handoff(expected, src, dst, g.half(), g.layers)
    with P.RunList.bf16(view, view, runs, kv) as rl:
        rl.copy(stream_ptr(torch))
        torch.cuda.synchronize()
    after = snapshot(bufs)
    assert np.array_equal(after, expected), first_diff(after, expected)


def test_empty_and_degenerate_inputs_are_rejected(torch_cuda):
    torch = torch_cuda
    kv = P.shape(2, 2, 64)
    bufs, view = device_arena(torch, 8 * kv.page_bytes())
    with pytest.raises(P.PbeError):
        P.copy_shared_kv(view, [], [], kv, 0, stream_ptr(torch))
    with pytest.raises(P.PbeError):
        P.RunList.bf16(view, view, [(0, 4, 0)], kv)           # zero-page run
    with pytest.raises(P.PbeError):
        P.RunList.bf16(view, view, [(0, 6, 1)], kv)           # 6 is not a page id (stride 4)
    with pytest.raises(P.PbeError):
        P.RunList.bf16(view, view, [(0, 0, 1)], kv)           # destination is its own source
    with pytest.raises(P.PbeError):
        P.RunList.bf16(view, view, [(0, 28, 2)], kv)          # runs past the arena


def test_timed_launch_copies_and_brackets_the_kernel(torch_cuda):
    """pbe_handoff_copy_timed: same bytes as the plain launch; its events time
    the kernel alone, so they read no more than events recorded around it."""
    torch = torch_cuda
    w = W.config2(3)
    g = w.geometry
    kv = _kv(g)
    say("timed launch config2")
    bufs, view = device_arena(torch, w.arena_bytes)
    fill_bf16(torch, bufs[0], w.sigma, 9)
    torch.cuda.synchronize()
    expected = snapshot(bufs)
    O.copy_handoff(expected, w.src_ids, w.dst_ids, g.half(), g.layers)
    runs = P.build_runs(w.src_ids, w.dst_ids, kv)
    with P.RunList.bf16(view, view, runs, kv) as rl:
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        e.record()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        rl.copy_timed(stream_ptr(torch), s.cuda_event, e.cuda_event)
        b.record()
        torch.cuda.synchronize()
        inner, outer = s.elapsed_time(e), a.elapsed_time(b)
    assert 0 < inner <= outer, (inner, outer)
    after = snapshot(bufs)
    assert np.array_equal(after, expected), first_diff(after, expected)


def test_concurrent_one_call_handoffs_from_host_threads(torch_cuda):
    """Several host threads drive one-call handoffs at once, each on its own
    stream, through both launch forms (run lists in the kernel arguments and
    the shared staging ring): every request lands bit-exact."""
    import threading
    torch = torch_cuda
    w = W.config3(0)
    g = w.geometry
    kv = _kv(g)
    say(f"concurrent one-call handoffs: {len(w.requests)} threads x 8 repeats")
    bufs, view = device_arena(torch, w.arena_bytes, w.segment_bytes)
    for i, b in enumerate(bufs):
        fill_bf16(torch, b, w.sigma, 70 + i)
    torch.cuda.synchronize()
    expected = snapshot(bufs)
    O.copy_handoff(expected, w.src_ids, w.dst_ids, g.half(), g.layers)
    sizes = [len(P.build_runs(r.src_ids, r.dst_ids, kv, 2, w.segment_bytes)) for r in w.requests]
    assert min(sizes) <= 112 < max(sizes), sizes
    streams = [torch.cuda.Stream() for _ in w.requests]
    errors = []

    def worker(r, st):
        try:
            for _ in range(8):  # idempotent: the same pages again
                P.copy_shared_kv(view, r.src_ids, r.dst_ids, kv, 0, st.cuda_stream)
        except Exception as e:  # surfaced below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(r, st)) for r, st in zip(w.requests, streams)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    after = snapshot(bufs)
    assert np.array_equal(after, expected), first_diff(after, expected)


def test_single_allocation_beyond_4_gib(torch_cuda):
    """A 6 GiB single-segment arena: pages above the 4 GiB offset are copied
    from and to correctly (no 32-bit truncation of ids, offsets or addresses),
    by a prebuilt run list and by the one-call form."""
    torch = torch_cuda
    g = W.Geometry(layers=28, kv_heads=2, head_dim=128)
    kv = _kv(g)
    page = g.page_bytes()
    n_pages = (6 << 30) // page
    say(f"6 GiB single arena, {n_pages} pages of {page} B")
    arena = torch.empty(n_pages * page, dtype=torch.uint8, device="cuda")
    fill_bf16(torch, arena, 1.0, 90)
    view = P.view_of(arena.data_ptr(), arena.numel())
    hi = ((4 << 30) + page - 1) // page  # first page at or above 4 GiB
    rng = np.random.default_rng(90)
    src_pages = np.concatenate([rng.permutation(2000)[:60] + 100, rng.permutation(n_pages - hi - 200)[:60] + hi + 100])
    dst_pages = rng.permutation(np.setdiff1d(np.arange(hi - 50, n_pages - 1), src_pages))[:120]
    src_ids = (src_pages * g.stride).astype(np.int32)
    dst_ids = (dst_pages * g.stride).astype(np.int32)
    saved = {int(s): arena[int(s) * page:(int(s) + 1) * page].clone() for s in src_pages}
    canary = [int(p) for p in rng.permutation(np.setdiff1d(np.arange(n_pages),
                                                        np.concatenate([dst_pages])))[:40]]
    canary_before = {p: arena[p * page:(p + 1) * page].clone() for p in canary}
    half = len(src_ids) // 2
    with P.RunList.bf16(view, view, P.build_runs(src_ids[:half], dst_ids[:half], kv), kv) as rl:
        rl.copy(stream_ptr(torch))
    P.copy_shared_kv(view, src_ids[half:], dst_ids[half:], kv, 0, stream_ptr(torch))
    torch.cuda.synchronize()
    for s, d in zip(src_pages, dst_pages):
        assert torch.equal(arena[int(d) * page:(int(d) + 1) * page], saved[int(s)]), (s, d)
    for p in canary:
        assert torch.equal(arena[p * page:(p + 1) * page], canary_before[p]), p


def _contiguous_source_plan(g: W.Geometry, n_runs: int, n_pages: int, seed: int):
    """n_pages source pages in one region (pages 0..n_pages-1, in order) cut
    into n_runs runs whose destinations lie, shuffled and one page apart,
    above it: the shape of a single prefill's handoff into a fragmented
    decode group."""
    rng = np.random.default_rng(seed)
    cuts = np.sort(rng.choice(np.arange(1, n_pages), n_runs - 1, replace=False))
    lengths = np.diff(np.concatenate(([0], cuts, [n_pages])))
    order = rng.permutation(n_runs)
    dst_start = np.empty(n_runs, np.int64)
    at = n_pages + 1
    for r in order:                        # shuffled, with a one-page gap after each
        dst_start[r] = at
        at += lengths[r] + 1
    dst_pages = np.concatenate([np.arange(s, s + n) for s, n in zip(dst_start, lengths)])
    src = (np.arange(n_pages) * g.stride).astype(np.int32)
    dst = (dst_pages * g.stride).astype(np.int32)
    return src, dst, at


@pytest.mark.parametrize("n_runs,n_pages,head_dim", [
    (1, 40, 64), (37, 300, 64), (64, 64, 64), (65, 400, 64), (200, 700, 64),
    (256, 600, 64), (257, 600, 64),        # the one-call kernel-argument list's limit
    (511, 900, 64), (512, 1024, 64), (513, 1100, 64), (900, 1500, 64),
    (60, 300, 24),                         # 3 KiB pages: three 1 KiB slices
    (60, 300, 12),                         # pages of 1.5 KiB slices: no contiguous-source path
])
def test_contiguous_sources_across_run_counts(torch_cuda, n_runs, n_pages, head_dim):
    """Sources in one region take the kernel's contiguous-source path (the
    source of slice s is known before its run); run counts on both sides of
    each search-width step and of that path's 512-run limit, through a run
    list and through the one-call entry point (kernel-argument list up to
    112 runs, staged list above)."""
    torch = torch_cuda
    g = W.Geometry(2, 2 if head_dim == 64 else 1, head_dim)
    kv = _kv(g)
    src, dst, total = _contiguous_source_plan(g, n_runs, n_pages, 1000 + n_runs)
    runs = P.build_runs(src, dst, kv)
    assert len(runs) == n_runs
    say(f"contiguous sources runs={n_runs} pages={n_pages} page_bytes={g.page_bytes()}")
    bufs, view = device_arena(torch, (total + 3) * g.page_bytes())
    fill_bf16(torch, bufs[0], 1.0, n_runs)
    torch.cuda.synchronize()
    expected = snapshot(bufs).copy()
    O.copy_handoff(expected, src, dst, g.half(), g.layers)
    with P.RunList.bf16(view, view, runs, kv) as rl:
        # the path shows in the slice count: 1 KiB slices on the contiguous-
        # source path (pages of whole KiB, at most 512 runs), else 2 KiB per run
        page = g.page_bytes()
        if page % 1024 == 0 and n_runs <= 512:
            assert rl.info().slices == n_pages * page // 1024
        else:
            assert rl.info().slices == sum(-(-int(r[2]) * page // 2048) for r in runs)
        rl.copy(stream_ptr(torch))
        torch.cuda.synchronize()
    after = snapshot(bufs)
    assert np.array_equal(after, expected), first_diff(after, expected)
    # the same plan again through the one-call entry point, over fresh values
    fill_bf16(torch, bufs[0], 1.0, n_runs + 7)
    torch.cuda.synchronize()
    expected = snapshot(bufs).copy()
    O.copy_handoff(expected, src, dst, g.half(), g.layers)
    P.copy_shared_kv(view, src, dst, kv, 0, stream_ptr(torch))
    torch.cuda.synchronize()
    after = snapshot(bufs)
    assert np.array_equal(after, expected), first_diff(after, expected)


# Workgroup rounds of the copy kernels' XCD grouping: 8 XCDs x 24 workgroups
# of 512 threads (1 KiB slices) on the contiguous-source path, 8 x 48 of 256
# threads (2 KiB slices) on the general path. A 16 KiB page is two workgroups
# on either path, so a round is 96 pages there and 192 pages here.
@pytest.mark.parametrize("path,n_pages", [
    ("contiguous", 95), ("contiguous", 96), ("contiguous", 97), ("contiguous", 200),
    ("general", 191), ("general", 192), ("general", 193), ("general", 400),
])
def test_grids_at_xcd_group_round_boundaries(torch_cuda, path, n_pages):
    """Grids below one round of XCD groups (dispatch order kept), of exactly
    whole rounds, and of whole rounds plus a partial one: every slice is
    copied exactly once, through a run list and through the one-call entry
    point, the whole arena compared with the oracle."""
    torch = torch_cuda
    g = W.Geometry(2, 2, 64)
    assert g.page_bytes() == 16384
    kv = _kv(g)
    if path == "contiguous":
        src, dst, total = _contiguous_source_plan(g, max(1, n_pages // 3), n_pages, 2000 + n_pages)
        arena_pages = total + 3
        slices = n_pages * 16
    else:
        w = W.small(seed=n_pages, layers=2, kv_heads=2, head_dim=64, n_pages=4 * n_pages + 16,
                    handoff_pages=n_pages)
        src, dst = w.src_ids, w.dst_ids
        arena_pages = 4 * n_pages + 16
        slices = n_pages * 8
    runs = P.build_runs(src, dst, kv)
    say(f"xcd rounds path={path} pages={n_pages} runs={len(runs)}")
    bufs, view = device_arena(torch, arena_pages * g.page_bytes())
    for rep, seed in enumerate((n_pages, n_pages + 1)):
        fill_bf16(torch, bufs[0], 1.0, seed)
        torch.cuda.synchronize()
        expected = snapshot(bufs).copy()
        O.copy_handoff(expected, src, dst, g.half(), g.layers)
        if rep == 0:
            with P.RunList.bf16(view, view, runs, kv) as rl:
                assert rl.info().slices == slices
                rl.copy(stream_ptr(torch))
                torch.cuda.synchronize()
        else:
            P.copy_shared_kv(view, src, dst, kv, 0, stream_ptr(torch))
            torch.cuda.synchronize()
        after = snapshot(bufs)
        assert np.array_equal(after, expected), first_diff(after, expected)
