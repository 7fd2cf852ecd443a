"""GPU numerics of the decode-side reader (pbe_paged_decode) against the
float64 oracle and a plain torch fp32 attention of the same op.

FP8 pages come from the library's own fused handoff (BF16 pages -> FP8 E4M3 +
per-token-head scales), so these tests run the whole path a decode step sees:
handoff output -> paged attention. Tail token slots of every last block hold
NaN bytes, which the reader must not touch.

Tolerance (written out in `close()`): the output is rounded to BF16 (2^-9
relative), fp32 accumulation and exp2 add ~1e-6; the bound is 2^-8 of the
value plus 2^-11 of the row's largest magnitude.
"""
import numpy as np
import pytest

import pbe_handoff as P
from oracle import oracle as O
from tests.conftest import say
from tests.gpu_util import device_arena, fill_bf16, stream_ptr

pytestmark = pytest.mark.gpu


def close(got, want):
    rowmax = np.abs(want).max(axis=-1, keepdims=True)
    return np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 2.0 ** -11 * rowmax + 1e-30


def bf16_to_f64(u16):
    return (np.asarray(u16, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


class DecodeCase:
    def __init__(self, torch, *, fp8, layers, H, D, kvm, seq_lens, seed, n_pages=None,
                 segment_pages=0, layer=None, raw_codes=False):
        self.torch = torch
        self.fp8, self.layers, self.H, self.D, self.kvm = fp8, layers, H, D, kvm
        self.layer = layers - 1 if layer is None else layer
        self.seq_lens = list(seq_lens)
        self.batch = len(seq_lens)
        self.max_blocks = max(1, max((n + 15) // 16 for n in seq_lens))
        need = sum((n + 15) // 16 for n in seq_lens)
        self.n_pages = n_pages or max(8, need + 3)
        self.kv = P.shape(layers, H, D)
        rng = np.random.default_rng(seed)
        E = 1 if fp8 else 2
        self.half = 16 * H * D * E
        self.page = 2 * layers * self.half
        seg = segment_pages * self.page if segment_pages else 0
        # BF16 pages (the prefill's KV)
        self.bf_bufs, self.bf_view = device_arena(torch, self.n_pages * 2 * layers * 16 * H * D * 2,
                                                  segment_pages * 2 * layers * 16 * H * D * 2)
        for i, b in enumerate(self.bf_bufs):
            fill_bf16(torch, b, 1.0, seed * 7 + i)
        if fp8:
            self.bufs, self.view = device_arena(torch, self.n_pages * self.page, seg)
            self.scales = torch.zeros(self.n_pages * 2 * layers * 16 * H, dtype=torch.float32,
                                      device="cuda")
            ids = np.arange(self.n_pages, dtype=np.int32) * 2 * layers
            runs = P.build_runs(ids, ids, self.kv, 1, seg)
            with P.RunList.fp8(self.bf_view, self.view, self.scales.data_ptr(),
                               self.scales.numel() * 4, runs, self.kv) as rl:
                rl.copy_fp8(P.PBE_FP8_SCALE_PER_TOKEN_HEAD, 0, stream_ptr(torch))
            torch.cuda.synchronize()
            if raw_codes:  # every non-NaN E4M3 code (subnormals, +-448) and random scales
                for x in self.bufs:
                    codes = rng.integers(0, 254, x.numel(), dtype=np.uint8)
                    codes[codes >= 0x7F] += 1  # skip 0x7f; 0xff is out of range
                    x.copy_(torch.from_numpy(codes).cuda())
                self.scales.copy_(torch.from_numpy(
                    rng.uniform(1e-3, 0.05, self.scales.numel()).astype(np.float32)).cuda())
        else:
            self.bufs, self.view = self.bf_bufs, self.bf_view
            self.scales = None
        # page tables: distinct pages in random order
        perm = rng.permutation(self.n_pages)
        self.tables = np.full((self.batch, self.max_blocks), -1, np.int32)
        k = 0
        for b, n in enumerate(seq_lens):
            for i in range((n + 15) // 16):
                self.tables[b, i] = perm[k] * 2 * layers
                k += 1
        # NaN bytes in the tail slots of every last block (every layer)
        host = np.concatenate([x.cpu().numpy() for x in self.bufs])
        nan_byte = 0xFF
        for b, n in enumerate(seq_lens):
            if n % 16 == 0:
                continue
            pid = int(self.tables[b, (n - 1) // 16])
            for plane in range(2 * layers):
                start = (pid + plane) * self.half + (n % 16) * H * D * E
                host[start:(pid + plane + 1) * self.half] = nan_byte
        off = 0
        for x in self.bufs:
            x.copy_(torch.from_numpy(host[off:off + x.numel()].copy()).cuda())
            off += x.numel()
        self.host = host
        self.host_scales = self.scales.cpu().numpy() if fp8 else None
        qf = rng.standard_normal((self.batch, H * kvm, D)).astype(np.float32)
        self.q_host = O.bf16_from_f32(qf)
        self.q = torch.from_numpy(self.q_host.view(np.int16)).cuda()
        self.out = torch.empty_like(self.q)
        self.t_dev = torch.from_numpy(self.tables.copy()).cuda()
        self.s_dev = torch.tensor(self.seq_lens, dtype=torch.int32, device="cuda")

    def run(self, splits=0, tables=None, seq_lens=None, ws=None):
        torch = self.torch
        s = splits or P.decode_splits(self.batch, self.H, self.max_blocks,
                                      P.PBE_KV_FP8_E4M3 if self.fp8 else P.PBE_KV_BF16)
        ws_bytes = P.decode_workspace_bytes(self.batch, self.H * self.kvm, self.D, s)
        if ws is None:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        assert ws.numel() >= ws_bytes
        t = self.t_dev if tables is None else tables
        sl = self.s_dev if seq_lens is None else seq_lens
        P.paged_decode(self.view, P.PBE_KV_FP8_E4M3 if self.fp8 else P.PBE_KV_BF16,
                       self.scales.data_ptr() if self.fp8 else 0,
                       self.scales.numel() * 4 if self.fp8 else 0, self.kv, self.layer,
                       self.q.data_ptr(), self.out.data_ptr(), self.batch, self.H * self.kvm,
                       t.data_ptr(), sl.data_ptr(), self.max_blocks, splits, ws.data_ptr(),
                       ws_bytes, stream_ptr(torch))
        torch.cuda.synchronize()
        return bf16_to_f64(self.out.cpu().numpy().view(np.uint16))

    def oracle(self):
        return O.paged_decode(self.host, self.fp8, self.host_scales, self.layers, self.H, self.D,
                              self.layer, self.q_host, self.tables, self.seq_lens)

    def torch_fp32(self):
        """Plain torch fp32 attention over gathered, dequantized pages."""
        import torch
        H, D, L, E = self.H, self.D, self.layers, 1 if self.fp8 else 2
        pages = torch.from_numpy(self.host).view(-1, L, 2, 16, H, D * E)
        lut = torch.tensor(O.e4m3_table(), dtype=torch.float32)
        sc = torch.from_numpy(self.host_scales).view(-1, L, 2, 16, H) if self.fp8 else None

        def dequant(raw):  # gathered bytes [n, D*E] -> fp32 [n, D]
            if self.fp8:
                return lut[raw.long()]
            return (raw.contiguous().view(torch.int16).int() << 16).view(torch.float32)
        q = torch.from_numpy(bf16_to_f64(self.q_host).astype(np.float32))
        out = torch.zeros(self.batch, H * self.kvm, D)
        for b, n in enumerate(self.seq_lens):
            if n == 0:
                continue
            t = torch.arange(n)
            pg = torch.from_numpy(self.tables[b].astype(np.int64))[t // 16] // (2 * L)
            tok = t % 16
            for h in range(H):
                K = dequant(pages[pg, self.layer, 0, tok, h])
                V = dequant(pages[pg, self.layer, 1, tok, h])
                ks = sc[pg, self.layer, 0, tok, h] if sc is not None else torch.ones(n)
                vs = sc[pg, self.layer, 1, tok, h] if sc is not None else torch.ones(n)
                qh = q[b, h * self.kvm:(h + 1) * self.kvm]
                s = (qh @ K.T) / float(np.sqrt(D)) * ks
                p = torch.softmax(s, dim=-1) * vs
                out[b, h * self.kvm:(h + 1) * self.kvm] = p @ V
        return out.double().numpy()


def _check(case, got):
    want = case.oracle()
    ok = close(got, want)
    assert ok.all(), f"{(~ok).sum()} of {ok.size} outside tolerance; worst at " \
        f"{np.unravel_index(np.argmax(np.abs(got - want)), got.shape)}"
    ref = case.torch_fp32()
    assert close(got, ref).all()
    return want


@pytest.mark.parametrize("fp8", [True, False])
def test_qwen15b_geometry_ragged_lengths(torch_cuda, fp8):
    say(f"decode fp8={fp8} L4 H2 D128 kvm6 ragged")
    case = DecodeCase(torch_cuda, fp8=fp8, layers=4, H=2, D=128, kvm=6,
                      seq_lens=[0, 1, 15, 16, 17, 33, 300, 511], seed=1)
    got = case.run()
    want = _check(case, got)
    assert not got[0].any()  # empty sequence: zeros
    for splits in (1, 64):
        say(f"decode fp8={fp8} splits={splits}")
        assert close(case.run(splits), want).all()


@pytest.mark.parametrize("fp8", [True, False])
def test_qwen05b_geometry_head_dim_64(torch_cuda, fp8):
    say(f"decode fp8={fp8} L3 H2 D64 kvm7")
    case = DecodeCase(torch_cuda, fp8=fp8, layers=3, H=2, D=64, kvm=7,
                      seq_lens=[5, 64, 65, 200, 1], seed=2, layer=1)
    _check(case, case.run())


def test_every_e4m3_code_dequantizes_exactly(torch_cuda):
    say("decode fp8 raw codes")
    case = DecodeCase(torch_cuda, fp8=True, layers=2, H=2, D=128, kvm=4,
                      seq_lens=[200, 3, 64, 129], seed=7, raw_codes=True)
    _check(case, case.run())


def test_segmented_arena_and_one_query_head_per_kv_head(torch_cuda):
    say("decode fp8 segmented kvm1 H4")
    case = DecodeCase(torch_cuda, fp8=True, layers=2, H=4, D=128, kvm=1,
                      seq_lens=[40, 100, 7, 160], seed=3, segment_pages=5, n_pages=25)
    assert case.view.nseg == 5
    _check(case, case.run())


@pytest.mark.parametrize("fp8", [True, False])
@pytest.mark.parametrize("H,kvm,D", [(3, 2, 128), (1, 8, 64), (3, 5, 64)])
def test_odd_kv_head_counts_and_eight_query_heads(torch_cuda, fp8, H, kvm, D):
    """Odd KV head counts and the largest group (8 query heads per KV head)."""
    say(f"decode fp8={fp8} H{H} kvm{kvm} D{D}")
    case = DecodeCase(torch_cuda, fp8=fp8, layers=2, H=H, D=D, kvm=kvm,
                      seq_lens=[33, 1, 160, 17], seed=8 + H + kvm)
    _check(case, case.run())


def test_workspace_contents_do_not_matter_and_reuse_is_safe(torch_cuda):
    """The workspace may hold anything (all ones, random bytes, the previous
    launch's partials): the output is the same, bit for bit."""
    torch = torch_cuda
    say("decode fp8 workspace garbage + reuse")
    case = DecodeCase(torch, fp8=True, layers=2, H=2, D=128, kvm=6,
                      seq_lens=[300, 17, 0, 129, 64], seed=9)
    want = _check(case, case.run())
    for splits in (1, 2, 8, 64):
        n = P.decode_workspace_bytes(case.batch, case.H * case.kvm, case.D, splits)
        first = case.run(splits, ws=torch.zeros(n, dtype=torch.uint8, device="cuda"))
        assert close(first, want).all(), splits
        ws = torch.full((n,), 0xFF, dtype=torch.uint8, device="cuda")
        for rep in range(3):  # the same workspace three times in a row
            assert np.array_equal(case.run(splits, ws=ws), first), (splits, rep)
        ws.copy_(torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda"))
        assert np.array_equal(case.run(splits, ws=ws), first), splits


def test_5040_token_prefix_batch(torch_cuda):
    say("decode fp8 5040-token prefixes x3, 28 layers")
    case = DecodeCase(torch_cuda, fp8=True, layers=28, H=2, D=128, kvm=6,
                      seq_lens=[5040, 5040, 5041], seed=4, layer=27)
    want = _check(case, case.run())
    # FP8 waves keep one block in flight up to 48 blocks per split and three
    # beyond: 316 blocks in 1, 4 (79 each), 6 (53) and 7 (46) splits.
    for splits in (1, 4, 6, 7):
        say(f"decode fp8 5040-token prefixes splits={splits}")
        assert close(case.run(splits), want).all(), splits


def test_bad_tables_give_nan_only_for_their_sequence(torch_cuda):
    torch = torch_cuda
    say("decode fp8 invalid ids")
    case = DecodeCase(torch, fp8=True, layers=2, H=2, D=128, kvm=6,
                      seq_lens=[40, 40, 40, 40], seed=5)
    want = case.oracle()
    t = case.tables.copy()
    t[1, 1] = 5                        # not a page id
    t[2, 2] = case.n_pages * 4 + 4     # past the arena
    sl = list(case.seq_lens)
    sl[3] = 16 * case.max_blocks + 1   # needs more blocks than the table holds
    got = case.run(tables=torch.from_numpy(t).cuda(),
                   seq_lens=torch.tensor(sl, dtype=torch.int32, device="cuda"))
    assert close(got[0], want[0]).all()
    assert np.isnan(got[1:]).all()


def test_argument_errors_are_rejected_before_launch(torch_cuda):
    torch = torch_cuda
    case = DecodeCase(torch, fp8=True, layers=2, H=2, D=128, kvm=6, seq_lens=[20], seed=6)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    base = dict(view=case.view, kv_dtype=P.PBE_KV_FP8_E4M3, scales=case.scales.data_ptr(),
                scale_bytes=case.scales.numel() * 4, kv=case.kv, layer=1,
                queries=case.q.data_ptr(), outputs=case.out.data_ptr(), batch=1, q_heads=12,
                tables=case.t_dev.data_ptr(), seq_lens=case.s_dev.data_ptr(),
                max_blocks=case.max_blocks, splits=0, workspace=ws.data_ptr(),
                workspace_bytes=ws.numel())
    bad = [dict(layer=2), dict(q_heads=13), dict(q_heads=18), dict(splits=1025), dict(kv_dtype=7),
           dict(scales=0), dict(workspace_bytes=16), dict(queries=case.q.data_ptr() + 2),
           dict(kv=P.shape(2, 2, 96)), dict(tables=0)]
    for change in bad:
        args = dict(base)
        args.update(change)
        with pytest.raises(P.PbeError):
            P.paged_decode(**args)


@pytest.mark.parametrize("fp8", [True, False])
def test_pages_beyond_4_gib_of_a_single_arena(torch_cuda, fp8):
    """The blocks of every sequence lie above the 4 GiB offset of one 6 GiB
    allocation (and of a 100-200 MB scale pool): addresses, page indices and
    scale offsets are computed without 32-bit truncation. The oracle runs on
    the used pages gathered into a compact host arena."""
    torch = torch_cuda
    L, H, D, kvm, layer = 2, 2, 128, 6, 1
    E = 1 if fp8 else 2
    half = 16 * H * D * E
    page = 2 * L * half
    n_pages = (6 << 30) // page
    say(f"decode fp8={fp8} over a 6 GiB arena, {n_pages} pages")
    arena = torch.empty(n_pages * page, dtype=torch.uint8, device="cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(31 + fp8)
    if fp8:  # E4M3 codes without the NaN codes
        arena.copy_(torch.randint(0, 0x7F, arena.shape, generator=g, device="cuda", dtype=torch.uint8)
                    | (torch.randint(0, 2, arena.shape, generator=g, device="cuda", dtype=torch.uint8) << 7))
        scales = torch.rand(n_pages * 2 * L * 16 * H, generator=g, device="cuda") * 0.05 + 1e-3
    else:
        fill_bf16(torch, arena, 1.0, 31)
        scales = None
    seq_lens = [200, 77, 300]
    need = [(n + 15) // 16 for n in seq_lens]
    hi = ((4 << 30) + page - 1) // page
    rng = np.random.default_rng(31)
    pages = rng.permutation(n_pages - hi)[:sum(need)] + hi
    batch, max_blocks = len(seq_lens), max(need)
    tables = np.zeros((batch, max_blocks), np.int32)
    compact = np.zeros((batch, max_blocks), np.int32)
    k = 0
    for b, nb in enumerate(need):
        tables[b, :nb] = pages[k:k + nb] * 2 * L
        compact[b, :nb] = np.arange(k, k + nb) * 2 * L
        k += nb
    view = P.view_of(arena.data_ptr(), arena.numel())
    kv = P.shape(L, H, D)
    qf = rng.standard_normal((batch, H * kvm, D)).astype(np.float32)
    q_host = O.bf16_from_f32(qf)
    q = torch.from_numpy(q_host.view(np.int16)).cuda()
    out = torch.empty_like(q)
    t_dev = torch.from_numpy(tables).cuda()
    s_dev = torch.tensor(seq_lens, dtype=torch.int32, device="cuda")
    splits = P.decode_splits(batch, H, max_blocks, P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16)
    ws_bytes = P.decode_workspace_bytes(batch, H * kvm, D, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    P.paged_decode(view, P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16,
                   scales.data_ptr() if fp8 else 0, scales.numel() * 4 if fp8 else 0, kv, layer,
                   q.data_ptr(), out.data_ptr(), batch, H * kvm, t_dev.data_ptr(), s_dev.data_ptr(),
                   max_blocks, splits, ws.data_ptr(), ws_bytes, stream_ptr(torch))
    torch.cuda.synchronize()
    got = bf16_to_f64(out.cpu().numpy().view(np.uint16))
    idx = torch.from_numpy(pages.astype(np.int64)).cuda()
    host = arena.view(n_pages, page)[idx].cpu().numpy().reshape(-1)
    host_scales = scales.view(n_pages, -1)[idx].cpu().numpy().reshape(-1) if fp8 else None
    want = O.paged_decode(host, fp8, host_scales, L, H, D, layer, q_host, compact, seq_lens)
    assert close(got, want).all()


@pytest.mark.parametrize("fp8", [True, False])
def test_one_long_sequence_uses_hundreds_of_splits(torch_cuda, fp8):
    """A small batch of long sequences takes hundreds of splits (one wave per
    SIMD, at least 4 blocks each) and the column-grouped combine; 1024 explicit
    splits leave most of them empty. Both against the float64 oracle."""
    say(f"decode fp8={fp8} one 20000-token sequence + a short one, many splits")
    case = DecodeCase(torch_cuda, fp8=fp8, layers=2, H=2, D=128, kvm=6, seq_lens=[20000, 37],
                      seed=71, layer=1)
    dtype = P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16
    auto = P.decode_splits(case.batch, case.H, case.max_blocks, dtype)
    assert auto > 64
    want = _check(case, case.run())
    say(f"decode fp8={fp8} splits=1024")
    assert close(case.run(1024), want).all()
