"""GPU parity of the page writer (pbe_scatter_kv / pbe_scatter_kv_to_page)
against the oracle's restatement of scatter_kv_kernel.cu, through the C ABI.

Every case compares the whole K and V pools (unwritten bytes are canaries)
and the whole scale pools bit for bit. Inputs mix N(0, s) values with the
rows the FP8 rule treats specially: all-zero rows, NaN elements, rows whose
448/amax overflows, infinities. Slot lists hold sequences' page-major slots,
negative slots and slots beyond the pool, in random order. The last case is a
decode loop: prompt tokens written to FP8 pages, one decode token appended at
its slot, then the paged decode reader over those pages.
"""
import numpy as np
import pytest

import pbe_handoff as P
from oracle import oracle as O
from tests.conftest import say
from tests.gpu_util import first_diff, stream_ptr

pytestmark = pytest.mark.gpu

B = 16


def _inputs(rng, n, heads, head_dim, f32, special=True):
    x = rng.standard_normal((2, n, heads * head_dim)).astype(np.float32) * 1.5
    if special and n > 6:
        x[0, 1] = 0.0                                   # zero token (K)
        x[1, 2, :head_dim] = 0.0                        # zero row (V, head 0)
        x[0, 3, 5] = np.nan
        x[1, 4, head_dim - 1] = np.inf
        x[0, 5, :head_dim] = 1e-38                      # 448/amax overflows
        x[1, 6, head_dim:] *= 300.0                     # large row (other heads)
    if f32:
        return x[0].copy(), x[1].copy()
    return O.bf16_from_f32(x[0]), O.bf16_from_f32(x[1])


def _slots(rng, n, pages, layers, blocks_in_pool):
    """n slots: mostly distinct page-major slots, a few negative or beyond the pool."""
    ids = rng.permutation(pages)[: (n + B - 1) // B + 1] * 2 * layers
    slots = np.array([ids[t // B] * B + t % B for t in range(n)], np.int64)
    rng.shuffle(slots)
    if n > 8:
        slots[0] = -1
        slots[1] = blocks_in_pool * B + 5           # beyond the pool
        slots[2] = -(2 ** 31)
    return slots.astype(np.int32)


class Pools:
    """A page-major arena of `layers` layers on the device plus scale planes,
    with layer `layer`'s K / V planes as the writer's pools."""

    def __init__(self, torch, layers, heads, head_dim, pages, fp8, f32, layer):
        self.torch = torch
        e = 1 if fp8 else (4 if f32 else 2)
        self.half = B * heads * head_dim * e
        self.plane = B * heads
        total = pages * 2 * layers * self.half
        rng = np.random.default_rng(pages)
        self.host = rng.integers(0, 256, total, dtype=np.uint8)          # canaries
        self.arena = torch.from_numpy(self.host.copy()).cuda()
        n_sc = pages * 2 * layers * self.plane
        self.host_sc = np.full(n_sc, -3.0, np.float32)
        self.sc = torch.from_numpy(self.host_sc.copy()).cuda()
        self.k_off, self.v_off = 2 * layer * self.half, (2 * layer + 1) * self.half
        self.ks_off, self.vs_off = 2 * layer * self.plane, (2 * layer + 1) * self.plane
        self.fp8 = fp8

    def args(self):
        base, sc = self.arena.data_ptr(), self.sc.data_ptr()
        n, m = self.arena.numel(), self.sc.numel() * 4
        a = [base + self.k_off, n - self.k_off, base + self.v_off, n - self.v_off]
        if self.fp8:
            a += [sc + 4 * self.ks_off, m - 4 * self.ks_off, sc + 4 * self.vs_off, m - 4 * self.vs_off]
        else:
            a += [0, 0, 0, 0]
        return a

    def oracle(self, K, V, slots, heads, head_dim):
        host, sc = self.host.copy(), self.host_sc.copy()
        O.scatter_kv(K, V, slots, B, heads, head_dim, self.fp8, host[self.k_off:], host[self.v_off:],
                     sc[self.ks_off:], sc[self.vs_off:])
        return host, sc

    def check(self, want_host, want_sc):
        self.torch.cuda.synchronize()
        got = self.arena.cpu().numpy()
        assert np.array_equal(got, want_host), first_diff(got, want_host)
        got_sc = self.sc.cpu().numpy()
        assert np.array_equal(got_sc.view(np.uint32), want_sc.view(np.uint32)), \
            first_diff(got_sc.view(np.uint8), want_sc.view(np.uint8))


CASES = [(2, 128), (2, 64), (4, 128), (1, 256), (3, 64), (8, 16)]


@pytest.mark.parametrize("heads,head_dim", CASES)
@pytest.mark.parametrize("in_dtype", ["bf16", "f32"])
@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_scatter_matches_the_oracle(torch_cuda, heads, head_dim, in_dtype, kv):
    torch = torch_cuda
    f32, fp8 = in_dtype == "f32", kv == "fp8"
    if fp8 and f32 and head_dim * 4 // 16 > 64:
        pytest.skip("one amax group spans more than a wave")
    rng = np.random.default_rng(heads * 1000 + head_dim + 7 * f32 + 3 * fp8)
    layers, layer, pages = 3, 2, 40
    n = 301
    say(f"scatter in={in_dtype} kv={kv} H={heads} D={head_dim} n={n}")
    pools = Pools(torch, layers, heads, head_dim, pages, fp8, f32, layer)
    K, V = _inputs(rng, n, heads, head_dim, f32)
    slots = _slots(rng, n, pages, layers, (pools.arena.numel() - pools.k_off) // pools.half)
    want_host, want_sc = pools.oracle(K, V, slots, heads, head_dim)
    dK = torch.from_numpy(K.view(np.uint8).copy()).cuda()
    dV = torch.from_numpy(V.view(np.uint8).copy()).cuda()
    dS = torch.from_numpy(slots).cuda()
    P.scatter_kv(dK.data_ptr(), dV.data_ptr(), P.PBE_IN_F32 if f32 else P.PBE_IN_BF16, n,
                 dS.data_ptr(), B, heads, head_dim, P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16,
                 *pools.args(), stream=stream_ptr(torch))
    pools.check(want_host, want_sc)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_single_token_at_a_slot_equals_the_batched_form(torch_cuda, kv):
    torch = torch_cuda
    fp8 = kv == "fp8"
    heads, head_dim, layers, layer, pages = 2, 128, 2, 1, 8
    rng = np.random.default_rng(5)
    pools = Pools(torch, layers, heads, head_dim, pages, fp8, False, layer)
    K, V = _inputs(rng, 1, heads, head_dim, False)
    block, offset = 3 * 2 * layers, 13
    say(f"scatter_kv_to_page kv={kv}")
    want_host, want_sc = pools.oracle(K, V, np.array([block * B + offset], np.int32), heads, head_dim)
    dK = torch.from_numpy(K.view(np.uint8).copy()).cuda()
    dV = torch.from_numpy(V.view(np.uint8).copy()).cuda()
    P.scatter_kv_to_page(dK.data_ptr(), dV.data_ptr(), P.PBE_IN_BF16, block, offset, B, heads,
                         head_dim, P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16, *pools.args(),
                         stream=stream_ptr(torch))
    pools.check(want_host, want_sc)
    with pytest.raises(P.PbeError) as e:
        P.scatter_kv_to_page(dK.data_ptr(), dV.data_ptr(), P.PBE_IN_BF16, block, B, B, heads,
                             head_dim, P.PBE_KV_BF16, *pools.args()[:4])
    assert e.value.code == P.PBE_ERR_INVALID


def test_scatter_rejects_misuse_before_any_write(torch_cuda):
    torch = torch_cuda
    heads, head_dim = 2, 64
    pools = Pools(torch, 1, heads, head_dim, 4, True, False, 0)
    K = torch.zeros((4, heads * head_dim), dtype=torch.bfloat16, device="cuda")
    S = torch.zeros(4, dtype=torch.int32, device="cuda")
    a = pools.args()
    say("scatter misuse")

    def call(keys=K.data_ptr(), values=K.data_ptr(), in_dtype=P.PBE_IN_BF16, n=4, slots=S.data_ptr(),
             hd=head_dim, kv=P.PBE_KV_FP8_E4M3, pool_args=a):
        P.scatter_kv(keys, values, in_dtype, n, slots, B, heads, hd, kv, *pool_args,
                     stream=stream_ptr(torch))

    bad = [
        dict(in_dtype=7), dict(kv=9), dict(n=-1), dict(slots=0),
        dict(keys=K.data_ptr() + 2),                         # misaligned input
        dict(pool_args=a[:4] + [0, 0, 0, 0]),                # FP8 without scales
        dict(pool_args=[a[0] + 1] + a[1:]),                  # misaligned FP8 pool
        dict(values=pools.host.ctypes.data),                 # host memory
    ]
    for kw in bad:
        with pytest.raises(P.PbeError) as e:
            call(**kw)
        assert e.value.code == P.PBE_ERR_INVALID, kw
    with pytest.raises(P.PbeError) as e:
        call(hd=48)  # 48 BF16 = 6 lanes: not a power of two
    assert e.value.code == P.PBE_ERR_UNSUPPORTED
    call(n=0)  # no-op
    pools.check(pools.host, pools.host_sc)


@pytest.mark.parametrize("fp8", [True, False])
def test_prompt_and_decode_token_written_then_decoded(torch_cuda, fp8):
    """The producer side of the decode reader: a batch's prompt K/V written to
    pages with slot mappings, each sequence's next token appended at its slot,
    then one decode step. Pages equal the oracle's bit for bit; the attention
    equals the float64 oracle over the oracle's pages within the reader's
    tolerance."""
    from tests.test_gpu_decode import close, bf16_to_f64
    torch = torch_cuda
    rng = np.random.default_rng(31 + fp8)
    heads, head_dim, kvm, layers, layer, pages = 2, 128, 6, 4, 3, 64
    prompt = [300, 17, 64, 129]
    say(f"scatter then decode fp8={fp8}")
    pools = Pools(torch, layers, heads, head_dim, pages, fp8, False, layer)
    perm = rng.permutation(pages)
    tables, k = [], 0
    for n in prompt:
        need = (n + 1 + B - 1) // B
        tables.append([int(perm[k + i]) * 2 * layers for i in range(need)])
        k += need
    width = max(len(t) for t in tables)
    tab = np.full((len(prompt), width), -1, np.int32)
    for b, t in enumerate(tables):
        tab[b, :len(t)] = t
    slots = np.array([tables[b][t // B] * B + t % B for b, n in enumerate(prompt) for t in range(n)],
                     np.int32)
    K, V = _inputs(rng, len(slots), heads, head_dim, False, special=False)
    host, sc = pools.oracle(K, V, slots, heads, head_dim)
    dK = torch.from_numpy(K.view(np.uint8).copy()).cuda()
    dV = torch.from_numpy(V.view(np.uint8).copy()).cuda()
    dS = torch.from_numpy(slots).cuda()
    kv_dtype = P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16
    P.scatter_kv(dK.data_ptr(), dV.data_ptr(), P.PBE_IN_BF16, len(slots), dS.data_ptr(), B, heads,
                 head_dim, kv_dtype, *pools.args(), stream=stream_ptr(torch))
    # decode tokens: one per sequence at position prompt[b]
    Kd, Vd = _inputs(rng, len(prompt), heads, head_dim, False)
    for b, n in enumerate(prompt):
        blk, off = tables[b][n // B], n % B
        one = np.array([blk * B + off], np.int32)
        O.scatter_kv(Kd[b:b + 1], Vd[b:b + 1], one, B, heads, head_dim, fp8, host[pools.k_off:],
                     host[pools.v_off:], sc[pools.ks_off:], sc[pools.vs_off:])
        dk = torch.from_numpy(Kd[b:b + 1].view(np.uint8).copy()).cuda()
        dv = torch.from_numpy(Vd[b:b + 1].view(np.uint8).copy()).cuda()
        P.scatter_kv_to_page(dk.data_ptr(), dv.data_ptr(), P.PBE_IN_BF16, blk, off, B, heads,
                             head_dim, kv_dtype, *pools.args(), stream=stream_ptr(torch))
    pools.check(host, sc)
    lens = [n + 1 for n in prompt]
    q = O.bf16_from_f32(rng.standard_normal((len(prompt), heads * kvm, head_dim)).astype(np.float32))
    dq = torch.from_numpy(q.view(np.int16).copy()).cuda()
    out = torch.empty_like(dq)
    view = P.view_of([pools.arena.data_ptr()], pools.arena.numel())
    kv = P.shape(layers, heads, head_dim)
    dtab = torch.from_numpy(tab).cuda()
    dlen = torch.tensor(lens, dtype=torch.int32, device="cuda")
    splits = P.decode_splits(len(prompt), heads, width, kv_dtype)
    ws_bytes = P.decode_workspace_bytes(len(prompt), heads * kvm, head_dim, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    P.paged_decode(view, kv_dtype, pools.sc.data_ptr() if fp8 else 0, pools.sc.numel() * 4 if fp8 else 0,
                   kv, layer, dq.data_ptr(), out.data_ptr(), len(prompt), heads * kvm, dtab.data_ptr(),
                   dlen.data_ptr(), width, splits, ws.data_ptr(), ws_bytes, stream_ptr(torch))
    torch.cuda.synchronize()
    got = bf16_to_f64(out.cpu().numpy().view(np.uint16))
    want = O.paged_decode(host, fp8, sc if fp8 else None, layers, heads, head_dim, layer, q, tab, lens)
    assert close(got, want).all()
