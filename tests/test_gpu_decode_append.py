"""GPU parity of pbe_paged_decode_append: one decode step that writes each
sequence's new token at its last position and reads the pages in the same
launch, against the two launches it replaces, pbe_scatter_kv (BF16 input)
then pbe_paged_decode_pools, on copies of the same pools.

- The K and V pools and both scale pools (every byte, written or not) and the
  outputs (every bit) are identical between the two forms.
- The written pools equal the oracle's page writer (orc_scatter_kv) applied
  to the original pools, and the outputs are within the reader's tolerance of
  the float64 pool-addressed oracle over those pools.
- Split counts from 1 to more splits than blocks move the last block into
  every position of a split; zero-length sequences, a length beyond the
  table, a bad id mid-table and a bad last id are covered (NaN for that
  sequence, and the last two write nothing exactly where scatter does not).
- Argument errors are rejected before any launch.
"""
import numpy as np
import pytest

import pbe_handoff as P
from oracle import oracle as O
from tests.conftest import say
from tests.gpu_util import stream_ptr
from tests.test_gpu_decode import bf16_to_f64, close

pytestmark = pytest.mark.gpu

B = 16


class Step:
    """Local K/V pools (noise in every block), block tables, queries and the
    step's new K/V rows, on the host and the device."""

    def __init__(self, torch, fp8, H, D, kvm, seq_lens, seed, spare=5):
        self.torch, self.fp8, self.H, self.D, self.kvm = torch, fp8, H, D, kvm
        rng = np.random.default_rng(seed)
        self.seq_lens = np.array(seq_lens, np.int32)
        self.batch = len(seq_lens)
        e = 1 if fp8 else 2
        self.half = B * H * D * e
        need = [max(0, (n + B - 1) // B) for n in seq_lens]
        self.max_blocks = max(1, max(need)) + 1
        used = sum(min(n, self.max_blocks) for n in need)
        self.n = used + spare
        perm = rng.permutation(self.n).astype(np.int32)
        self.tables = np.full((self.batch, self.max_blocks), -1, np.int32)
        k = 0
        for b, n in enumerate(need):
            n = min(n, self.max_blocks)
            self.tables[b, :n] = perm[k:k + n]
            k += n
        if fp8:
            codes = rng.integers(0, 256, 2 * self.n * self.half, dtype=np.uint8)
            codes[(codes & 0x7F) == 0x7F] = 0  # no NaN codes in the noise
            self.kp, self.vp = codes[: self.n * self.half].copy(), codes[self.n * self.half:].copy()
            planes = self.n * B * H
            self.ks = rng.uniform(0.002, 0.02, planes).astype(np.float32)
            self.vs = rng.uniform(0.002, 0.02, planes).astype(np.float32)
        else:
            vals = O.bf16_from_f32(rng.standard_normal(2 * self.n * self.half // 2).astype(np.float32))
            self.kp = vals[: self.n * self.half // 2].view(np.uint8).copy()
            self.vp = vals[self.n * self.half // 2:].view(np.uint8).copy()
            self.ks = self.vs = None
        x = (rng.standard_normal((2, self.batch, H * D)) * 1.5).astype(np.float32)
        if self.batch > 3:
            x[0, 1, :D] = 0.0             # zero key row of head 0: scale 1, codes 0
            x[1, 2, D:] *= 300.0          # a large value row
            x[0, 3, :D] = 1e-38           # 448/amax overflows
        self.new_k, self.new_v = O.bf16_from_f32(x[0]), O.bf16_from_f32(x[1])
        self.q = O.bf16_from_f32(rng.standard_normal((self.batch, H * kvm, D)).astype(np.float32))

    def slots(self):
        """The slot of each sequence's new token, as the scatter form takes it."""
        s = np.full(self.batch, -1, np.int32)
        for b, n in enumerate(self.seq_lens):
            if 0 < n <= self.max_blocks * B:
                s[b] = self.tables[b, (n - 1) // B] * B + (n - 1) % B
        return s

    def device(self):
        t = self.torch
        d = dict(kp=t.from_numpy(self.kp).cuda(), vp=t.from_numpy(self.vp).cuda(),
                 tab=t.from_numpy(self.tables).cuda(), sl=t.from_numpy(self.seq_lens).cuda(),
                 nk=t.from_numpy(self.new_k).cuda(), nv=t.from_numpy(self.new_v).cuda(),
                 q=t.from_numpy(self.q).cuda(),
                 out=t.zeros((self.batch, self.H * self.kvm, self.D), dtype=t.int16, device="cuda"))
        if self.fp8:
            d["ks"] = t.from_numpy(self.ks).cuda()
            d["vs"] = t.from_numpy(self.vs).cuda()
        return d

    def _ws(self, splits):
        if splits == 0:  # the automatic count
            splits = P.decode_splits(self.batch, self.H, self.max_blocks,
                                     P.PBE_KV_FP8_E4M3 if self.fp8 else P.PBE_KV_BF16)
        n = P.decode_workspace_bytes(self.batch, self.H * self.kvm, self.D, splits)
        return self.torch.empty(n, dtype=self.torch.uint8, device="cuda"), n

    def _pool_args(self, d):
        sc = 4 * self.n * B * self.H if self.fp8 else 0
        return (d["kp"].data_ptr(), d["vp"].data_ptr(), self.n * self.half,
                d["ks"].data_ptr() if self.fp8 else 0, d["vs"].data_ptr() if self.fp8 else 0, sc,
                P.PBE_KV_FP8_E4M3 if self.fp8 else P.PBE_KV_BF16, self.H, self.D)

    def two_step(self, splits):
        d = self.device()
        slots = self.torch.from_numpy(self.slots()).cuda()
        kp, vp, pb, ks, vs, sb, dt, H, D = self._pool_args(d)
        P.scatter_kv(d["nk"].data_ptr(), d["nv"].data_ptr(), P.PBE_IN_BF16, self.batch,
                     slots.data_ptr(), B, H, D, dt, kp, pb, vp, pb, ks, sb, vs, sb,
                     stream=stream_ptr(self.torch))
        ws, n = self._ws(splits)
        P.paged_decode_pools(kp, vp, pb, ks, vs, sb, dt, H, D, d["q"].data_ptr(),
                             d["out"].data_ptr(), self.batch, H * self.kvm, d["tab"].data_ptr(),
                             d["sl"].data_ptr(), self.max_blocks, splits, ws.data_ptr(), n,
                             stream_ptr(self.torch))
        self.torch.cuda.synchronize()
        return self._host(d)

    def fused(self, splits, **change):
        d = self.device()
        ws, n = self._ws(splits)
        a = dict(zip(["key_pool", "value_pool", "pool_bytes", "key_scales", "value_scales",
                      "scale_pool_bytes", "kv_dtype", "kv_heads", "head_dim"], self._pool_args(d)))
        a.update(new_keys=d["nk"].data_ptr(), new_values=d["nv"].data_ptr(), queries=d["q"].data_ptr(),
                 outputs=d["out"].data_ptr(), batch=self.batch, q_heads=self.H * self.kvm,
                 tables=d["tab"].data_ptr(), seq_lens=d["sl"].data_ptr(),
                 max_blocks=self.max_blocks, splits=splits, workspace=ws.data_ptr(),
                 workspace_bytes=n, stream=stream_ptr(self.torch))
        a.update(change)
        P.paged_decode_append(**a)
        self.torch.cuda.synchronize()
        return self._host(d)

    def _host(self, d):
        h = dict(kp=d["kp"].cpu().numpy(), vp=d["vp"].cpu().numpy(),
                 out=d["out"].cpu().numpy().view(np.uint16))
        if self.fp8:
            h["ks"] = d["ks"].cpu().numpy()
            h["vs"] = d["vs"].cpu().numpy()
        return h


def _same(a, b):
    for key in a:
        x, y = a[key], b[key]
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), key


def _oracle_pools(step):
    """The original pools with the oracle's page writer applied."""
    kp, vp = step.kp.copy(), step.vp.copy()
    ks = step.ks.copy() if step.fp8 else None
    vs = step.vs.copy() if step.fp8 else None
    O.scatter_kv(step.new_k, step.new_v, step.slots(), B, step.H, step.D, step.fp8, kp, vp, ks, vs)
    return kp, vp, ks, vs


GEOMETRIES = [  # fp8, H, D, kvm, sequence lengths
    (True, 2, 128, 6, [5040, 1, 16, 17, 0, 300, 33, 64]),
    (False, 2, 128, 6, [5040, 1, 16, 17, 0, 300, 33, 64]),
    (True, 4, 64, 2, [1, 15, 16, 31, 32, 129, 700]),
    (False, 1, 64, 8, [200, 0, 16, 2]),
    (True, 1, 128, 1, [48, 49, 7, 1024]),
]


@pytest.mark.parametrize("geo", range(len(GEOMETRIES)))
def test_append_equals_scatter_then_decode(torch_cuda, geo):
    fp8, H, D, kvm, lens = GEOMETRIES[geo]
    step = Step(torch_cuda, fp8, H, D, kvm, lens, seed=100 + geo)
    auto = P.decode_splits(step.batch, H, step.max_blocks,
                           P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16)
    want_pools = _oracle_pools(step)
    for splits in sorted({1, 3, auto, step.max_blocks + 2}):
        say(f"decode append fp8={fp8} H={H} D={D} kvm={kvm} splits={splits}")
        a = step.two_step(splits)
        b = step.fused(splits)
        _same(a, b)
        assert np.array_equal(b["kp"], want_pools[0]) and np.array_equal(b["vp"], want_pools[1])
        if fp8:
            assert np.array_equal(b["ks"].view(np.uint32), want_pools[2].view(np.uint32))
            assert np.array_equal(b["vs"].view(np.uint32), want_pools[3].view(np.uint32))
    want = O.paged_decode_pools(b["kp"], b["vp"], fp8, b.get("ks"), b.get("vs"), H, D, step.q,
                                step.tables, step.seq_lens)
    assert close(bf16_to_f64(b["out"]), want).all()
    assert not (b["kp"] == step.kp).all()  # something was written


def test_arena_layer_views(torch_cuda):
    """The shared page-major arena through its layer views (key = arena +
    2*layer*half, value = key + half, page-major ids): the same equality."""
    torch = torch_cuda
    say("decode append over an arena layer view")
    layers, layer, H, D, kvm = 3, 1, 2, 128, 6
    step = Step(torch, True, H, D, kvm, [100, 17, 1, 250], seed=7)
    # renumber the blocks as page-major ids of a 3-layer arena and lay the
    # per-layer pools into it
    pages = step.n
    half, plane = step.half, B * H
    arena = np.random.default_rng(1).integers(0, 128, pages * 2 * layers * half, dtype=np.uint8)
    arena[(arena & 0x7F) == 0x7F] = 0
    sc = np.random.default_rng(2).uniform(0.002, 0.02, pages * 2 * layers * plane).astype(np.float32)
    for blk in range(pages):
        k_plane = blk * 2 * layers + 2 * layer
        arena[k_plane * half:(k_plane + 1) * half] = step.kp[blk * half:(blk + 1) * half]
        arena[(k_plane + 1) * half:(k_plane + 2) * half] = step.vp[blk * half:(blk + 1) * half]
        sc[k_plane * plane:(k_plane + 1) * plane] = step.ks[blk * plane:(blk + 1) * plane]
        sc[(k_plane + 1) * plane:(k_plane + 2) * plane] = step.vs[blk * plane:(blk + 1) * plane]
    tables = np.where(step.tables >= 0, step.tables * 2 * layers, -1).astype(np.int32)
    results = []
    for fused in (False, True):
        d_arena = torch.from_numpy(arena.copy()).cuda()
        d_sc = torch.from_numpy(sc.copy()).cuda()
        d = step.device()
        d["tab"] = torch.from_numpy(tables).cuda()
        base, sb = d_arena.data_ptr(), d_sc.data_ptr()
        kp, vp = base + 2 * layer * half, base + (2 * layer + 1) * half
        pb = arena.size - (2 * layer + 1) * half
        ks, vs = sb + 4 * 2 * layer * plane, sb + 4 * (2 * layer + 1) * plane
        sbytes = sc.size * 4 - 4 * (2 * layer + 1) * plane
        splits = P.decode_splits(step.batch, H, step.max_blocks, P.PBE_KV_FP8_E4M3)
        n = P.decode_workspace_bytes(step.batch, H * kvm, D, splits)
        ws = torch.empty(n, dtype=torch.uint8, device="cuda")
        if fused:
            P.paged_decode_append(kp, vp, pb, ks, vs, sbytes, P.PBE_KV_FP8_E4M3, H, D,
                                  d["nk"].data_ptr(), d["nv"].data_ptr(), d["q"].data_ptr(),
                                  d["out"].data_ptr(), step.batch, H * kvm, d["tab"].data_ptr(),
                                  d["sl"].data_ptr(), step.max_blocks, splits, ws.data_ptr(), n,
                                  stream_ptr(torch))
        else:
            s = np.array([tables[b, (m - 1) // B] * B + (m - 1) % B for b, m in enumerate(step.seq_lens)],
                         np.int32)
            slots = torch.from_numpy(s).cuda()
            P.scatter_kv(d["nk"].data_ptr(), d["nv"].data_ptr(), P.PBE_IN_BF16, step.batch,
                         slots.data_ptr(), B, H, D, P.PBE_KV_FP8_E4M3, kp, pb, vp, pb, ks, sbytes,
                         vs, sbytes, stream=stream_ptr(torch))
            P.paged_decode_pools(kp, vp, pb, ks, vs, sbytes, P.PBE_KV_FP8_E4M3, H, D,
                                 d["q"].data_ptr(), d["out"].data_ptr(), step.batch, H * kvm,
                                 d["tab"].data_ptr(), d["sl"].data_ptr(), step.max_blocks, splits,
                                 ws.data_ptr(), n, stream_ptr(torch))
        torch.cuda.synchronize()
        results.append((d_arena.cpu().numpy(), d_sc.cpu().numpy(), d["out"].cpu().numpy()))
    for x, y in zip(*results):
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8))
    assert not np.array_equal(results[1][0], arena)


@pytest.mark.parametrize("fp8", [True, False])
def test_bad_ids_and_lengths(torch_cuda, fp8):
    step = Step(torch_cuda, fp8, 2, 128, 6, [40, 70, 33, 17, 50], seed=9 + fp8)
    step.tables[1, 4] = step.n              # bad last id: nothing written, NaN
    step.tables[2, 0] = -7                  # bad id mid-table: the token is written, NaN
    step.seq_lens[3] = step.max_blocks * B + 1  # longer than the table: nothing written, NaN
    splits = 2
    say(f"decode append bad ids fp8={fp8}")
    a = step.two_step(splits)
    b = step.fused(splits)
    _same(a, b)
    out = bf16_to_f64(b["out"])
    for s in (1, 2, 3):
        assert np.isnan(out[s]).all()
    assert not np.isnan(out[[0, 4]]).any()
    want = _oracle_pools(step)
    assert np.array_equal(b["kp"], want[0]) and np.array_equal(b["vp"], want[1])


def test_append_argument_errors_are_rejected(torch_cuda):
    step = Step(torch_cuda, True, 2, 128, 6, [20, 5], seed=3)
    say("decode append misuse")
    step.fused(0)  # the valid call
    for change in [dict(new_keys=0), dict(new_values=0), dict(new_keys=None),
                   dict(head_dim=96), dict(value_scales=0), dict(pool_bytes=1 << 40)]:
        try:
            step.fused(0, **change)
        except P.PbeError:
            continue
        pytest.fail(f"accepted {change}")
    d = step.device()
    ws = step.torch.empty(1 << 20, dtype=step.torch.uint8, device="cuda")
    with pytest.raises(P.PbeError):  # unaligned new keys
        P.paged_decode_append(d["kp"].data_ptr(), d["vp"].data_ptr(), step.n * step.half,
                              d["ks"].data_ptr(), d["vs"].data_ptr(), 4 * step.n * B * 2,
                              P.PBE_KV_FP8_E4M3, 2, 128, d["nk"].data_ptr() + 2, d["nv"].data_ptr(),
                              d["q"].data_ptr(), d["out"].data_ptr(), step.batch, 12,
                              d["tab"].data_ptr(), d["sl"].data_ptr(), step.max_blocks, 0,
                              ws.data_ptr(), ws.numel())


@pytest.mark.parametrize("seed", range(12))
def test_random_geometries_equal_scatter_then_decode(torch_cuda, seed):
    """Seeded random shapes: page dtype, KV heads, head_dim, query heads per KV
    head, ragged lengths (zeros included) and split counts."""
    rng = np.random.default_rng(1000 + seed)
    fp8 = bool(rng.integers(0, 2))
    H = int(rng.choice([1, 2, 4]))
    D = int(rng.choice([64, 128]))
    kvm = int(rng.integers(1, 9))
    lens = [int(x) for x in rng.integers(0, 700, int(rng.integers(1, 9)))]
    if not any(lens):
        lens[0] = 1
    step = Step(torch_cuda, fp8, H, D, kvm, lens, seed=2000 + seed)
    splits = int(rng.choice([0, 1, 2, 5, step.max_blocks + 1]))
    say(f"decode append random seed={seed} fp8={fp8} H={H} D={D} kvm={kvm} lens={lens} splits={splits}")
    a = step.two_step(splits)
    b = step.fused(splits)
    _same(a, b)


@pytest.mark.parametrize("fp8", [True, False])
def test_arena_form_on_a_segmented_arena(torch_cuda, fp8):
    """pbe_paged_decode_append_arena over a 4-segment page-major arena: the arena
    afterwards equals the oracle's page writer applied to it (scales included),
    and the outputs equal pbe_paged_decode over that arena, bit for bit."""
    from tests.test_gpu_decode import DecodeCase
    torch = torch_cuda
    say(f"decode append, arena form over a segmented arena, fp8={fp8}")
    layers, layer, H, D, kvm = 3, 1, 2, 128, 6
    case = DecodeCase(torch, fp8=fp8, layers=layers, H=H, D=D, kvm=kvm,
                      seq_lens=[40, 1, 16, 33, 0, 97], seed=61 + fp8, segment_pages=4, layer=layer)
    assert len(case.bufs) > 1
    rng = np.random.default_rng(62)
    kv_rows = O.bf16_from_f32((rng.standard_normal((2, case.batch, H * D)) * 1.5).astype(np.float32))
    nk = torch.from_numpy(kv_rows[0].view(np.int16)).cuda()
    nv = torch.from_numpy(kv_rows[1].view(np.int16)).cuda()
    dt = P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16
    splits = P.decode_splits(case.batch, H, case.max_blocks, dt)
    n = P.decode_workspace_bytes(case.batch, H * kvm, D, splits)
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    P.paged_decode_append_arena(case.view, dt, case.scales.data_ptr() if fp8 else 0,
                                case.scales.numel() * 4 if fp8 else 0, case.kv, layer,
                                nk.data_ptr(), nv.data_ptr(), case.q.data_ptr(), case.out.data_ptr(),
                                case.batch, H * kvm, case.t_dev.data_ptr(), case.s_dev.data_ptr(),
                                case.max_blocks, splits, ws.data_ptr(), n, stream_ptr(torch))
    torch.cuda.synchronize()
    fused = case.out.cpu().numpy().view(np.uint16).copy()
    # expected pages: the oracle's page writer on the host arena (layer planes)
    want = case.host.copy()
    want_sc = case.host_scales.copy() if fp8 else None
    half, plane = case.half, 16 * H
    slots = np.array([case.tables[b, (m - 1) // 16] * 16 + (m - 1) % 16 if m > 0 else -1
                      for b, m in enumerate(case.seq_lens)], np.int32)
    O.scatter_kv(kv_rows[0], kv_rows[1], slots, 16, H, D, fp8, want[2 * layer * half:],
                 want[(2 * layer + 1) * half:],
                 want_sc[2 * layer * plane:] if fp8 else None,
                 want_sc[(2 * layer + 1) * plane:] if fp8 else None)
    got = np.concatenate([x.cpu().numpy() for x in case.bufs])
    assert np.array_equal(got, want)
    if fp8:
        assert np.array_equal(case.scales.cpu().numpy().view(np.uint32), want_sc.view(np.uint32))
    case.run(splits=splits)  # the reader over the written arena
    assert np.array_equal(fused, case.out.cpu().numpy().view(np.uint16))
    # and both against the float64 oracle over the written pages (the oracle's
    # page writer output above), so a reader fault on segmented arenas shows
    want_out = O.paged_decode(want, fp8, want_sc, layers, H, D, layer, case.q_host, case.tables,
                              case.seq_lens)
    assert close(bf16_to_f64(fused), want_out).all()
