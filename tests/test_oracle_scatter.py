"""Pins of the oracle's page writer (orc_scatter_kv, the restatement of
scatter_kv_kernel.cu:99-216), each through something other than its own
formula:

- plain BF16: the pages it writes, read back by the pinned paged-decode oracle,
  give the attention numpy computes directly on the unpaged token-major K/V;
- FP8 from BF16: byte-identical (codes and scales) to the pinned FP8 handoff
  of the plain pages it would have written: same rows, same per-(token, head)
  rule, the same page-major scale layout;
- FP8 from FP32: element-wise numpy amax / (448/amax) / x*inv in float32 fed to
  the pinned E4M3 conversion, with zero and NaN rows;
- plain FP32: the same bytes as the BF16 form with head_dim doubled;
- skipped slots (negative, beyond the pool) leave every byte as it was.
"""
import numpy as np
import pytest

from oracle import oracle as O

B = 16  # tokens per page


def _layout(layers, heads, head_dim, pages, elem):
    half = B * heads * head_dim * elem
    return half, pages * 2 * layers * half


def _plan(rng, seq_lens, pages, layers):
    """Distinct random pages per sequence; page-major block ids and slots."""
    perm = rng.permutation(pages)
    tables, slots, k = [], [], 0
    for n in seq_lens:
        ids = [int(perm[k + i]) * 2 * layers for i in range((n + B - 1) // B)]
        k += len(ids)
        tables.append(ids)
        slots += [ids[t // B] * B + t % B for t in range(n)]
    width = max(len(t) for t in tables)
    tab = np.full((len(seq_lens), width), -1, np.int32)
    for b, t in enumerate(tables):
        tab[b, :len(t)] = t
    return tab, np.array(slots, np.int32)


def _planes(arena, half, layer):
    return arena[2 * layer * half:], arena[(2 * layer + 1) * half:]


def _bf16(rng, shape, scale=1.0):
    return O.bf16_from_f32((rng.standard_normal(shape) * scale).astype(np.float32))


@pytest.mark.parametrize("heads,head_dim,layers,layer", [(2, 64, 3, 1), (1, 128, 2, 0), (3, 32, 2, 1)])
def test_plain_pages_read_back_as_the_unpaged_attention(heads, head_dim, layers, layer):
    rng = np.random.default_rng(heads * 100 + head_dim)
    seq_lens = [37, 16, 1, 70]
    pages = 16
    half, total = _layout(layers, heads, head_dim, pages, 2)
    tab, slots = _plan(rng, seq_lens, pages, layers)
    n = len(slots)
    K, V = _bf16(rng, (n, heads * head_dim)), _bf16(rng, (n, heads * head_dim))
    arena = np.zeros(total, np.uint8)
    kp, vp = _planes(arena, half, layer)
    O.scatter_kv(K, V, slots, B, heads, head_dim, False, kp, vp)
    kvm = 2
    q = _bf16(rng, (len(seq_lens), heads * kvm, head_dim))
    got = O.paged_decode(arena, False, None, layers, heads, head_dim, layer, q, tab, seq_lens)
    f = lambda u: (u.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    Kf, Vf, qf = f(K), f(V), f(q)
    start = 0
    for b, L in enumerate(seq_lens):
        for qh in range(heads * kvm):
            h = qh // kvm
            k = Kf[start:start + L, h * head_dim:(h + 1) * head_dim]
            v = Vf[start:start + L, h * head_dim:(h + 1) * head_dim]
            s = k @ qf[b, qh] / np.sqrt(head_dim)
            p = np.exp(s - s.max())
            want = p @ v / p.sum()
            assert np.allclose(got[b, qh], want, rtol=1e-6, atol=1e-6), (b, qh)
        start += L


@pytest.mark.parametrize("heads,head_dim", [(2, 128), (4, 64), (1, 8)])
def test_fp8_rows_equal_the_fp8_handoff_of_the_plain_pages(heads, head_dim):
    rng = np.random.default_rng(7 + head_dim)
    layers, layer, pages = 2, 1, 12
    seq_lens = [33, 48, 5]
    tab, slots = _plan(rng, seq_lens, pages, layers)
    n = len(slots)
    K = _bf16(rng, (n, heads * head_dim), 2.0)
    V = _bf16(rng, (n, heads * head_dim), 0.5)
    K[3] = 0                               # an all-zero token: scale 1, codes 0
    K[5, 1] = 0x7FC0                       # a NaN element (BF16 quiet NaN)
    V[9, :head_dim] = O.bf16_from_f32(np.full(head_dim, 1e-38, np.float32))  # 448/amax overflows
    half16, total16 = _layout(layers, heads, head_dim, pages, 2)
    half8, total8 = _layout(layers, heads, head_dim, pages, 1)
    bf = np.zeros(total16, np.uint8)
    O.scatter_kv(K, V, slots, B, heads, head_dim, False, *_planes(bf, half16, layer))
    # reference path: the pinned FP8 handoff of every page
    hand = np.zeros(total8, np.uint8)
    hand_sc = np.zeros(pages * 2 * layers * B * heads, np.float32)
    ids = np.arange(pages, dtype=np.int32) * 2 * layers
    O.fp8_handoff_token_head(bf, hand, hand_sc, ids, ids, layers, B, heads, head_dim)
    # the page writer straight to FP8 (untouched slots hold the handoff's zero-row result)
    got = np.zeros(total8, np.uint8)
    sc = np.ones(pages * 2 * layers * B * heads, np.float32)
    plane = B * heads
    O.scatter_kv(K, V, slots, B, heads, head_dim, True, *_planes(got, half8, layer),
                 sc[2 * layer * plane:], sc[(2 * layer + 1) * plane:])
    for p in range(pages):
        for kv in range(2):
            pl = p * 2 * layers + 2 * layer + kv
            assert np.array_equal(got[pl * half8:(pl + 1) * half8], hand[pl * half8:(pl + 1) * half8])
            a, b = sc[pl * plane:(pl + 1) * plane], hand_sc[pl * plane:(pl + 1) * plane]
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # the special rows did what the rule says
    r0 = slots[3] % B * heads
    blk0 = (slots[3] // B + 2 * layer) * plane
    assert np.all(sc[blk0 + r0:blk0 + r0 + heads] == 1.0)
    assert 0x7F in got  # the NaN element and the 0 * inf products of the tiny row


def test_fp32_input_matches_elementwise_numpy():
    rng = np.random.default_rng(3)
    heads, head_dim, layers, layer, pages = 2, 64, 1, 0, 6
    seq_lens = [20, 9]
    tab, slots = _plan(rng, seq_lens, pages, layers)
    n = len(slots)
    K = (rng.standard_normal((n, heads * head_dim)) * 3).astype(np.float32)
    V = (rng.standard_normal((n, heads * head_dim)) * 0.01).astype(np.float32)
    K[0] = 0.0
    K[2, 7] = np.nan
    V[4, 70] = -np.inf                     # amax inf: inv 0, scale inf, codes 0
    half8, total8 = _layout(layers, heads, head_dim, pages, 1)
    got = np.full(total8, 0xA5, np.uint8)
    plane = B * heads
    sc = np.full(pages * 2 * layers * plane, -1.0, np.float32)
    O.scatter_kv(K, V, slots, B, heads, head_dim, True, *_planes(got, half8, layer),
                 sc[2 * layer * plane:], sc[(2 * layer + 1) * plane:])
    for t in range(n):
        blk, off = divmod(int(slots[t]), B)
        for kv, X in ((0, K), (1, V)):
            for h in range(heads):
                x = X[t, h * head_dim:(h + 1) * head_dim]
                amax = np.float32(np.nanmax(np.abs(x))) if not np.all(np.isnan(x)) else np.float32(0)
                inv = np.float32(448) / amax if amax > 0 else np.float32(0)
                with np.errstate(invalid="ignore", over="ignore"):
                    prod = (x * inv).astype(np.float32) if inv > 0 else np.zeros_like(x)
                want = O.e4m3_from_f32(prod)
                pl = blk + 2 * layer + kv
                start = pl * half8 + (off * heads + h) * head_dim
                assert np.array_equal(got[start:start + head_dim], want), (t, kv, h)
                want_scale = amax / np.float32(448) if amax > 0 else np.float32(1)
                assert sc[pl * plane + off * heads + h] == want_scale


def test_plain_fp32_is_the_bf16_form_on_the_same_bytes():
    rng = np.random.default_rng(5)
    heads, head_dim, layers, pages = 2, 32, 2, 5
    tab, slots = _plan(rng, [30, 17], pages, layers)
    n = len(slots)
    K = rng.standard_normal((n, heads * head_dim)).astype(np.float32)
    V = rng.standard_normal((n, heads * head_dim)).astype(np.float32)
    half32, total32 = _layout(layers, heads, head_dim, pages, 4)
    a = np.zeros(total32, np.uint8)
    O.scatter_kv(K, V, slots, B, heads, head_dim, False, *_planes(a, half32, 1))
    b = np.zeros(total32, np.uint8)
    O.scatter_kv(K.view(np.uint16), V.view(np.uint16), slots, B, heads, 2 * head_dim, False,
                 *_planes(b, half32, 1))
    assert np.array_equal(a, b)
    assert a.any()


@pytest.mark.parametrize("fp8", [False, True])
def test_negative_and_out_of_pool_slots_write_nothing(fp8):
    rng = np.random.default_rng(11)
    heads, head_dim = 2, 16
    E = 1 if fp8 else 2
    row = heads * head_dim * E
    blocks = 4
    kp = np.full(blocks * B * row, 0xA5, np.uint8)
    vp = np.full(blocks * B * row, 0x5A, np.uint8)
    ks = np.full(blocks * B * heads, 7.0, np.float32)
    vs = np.full(blocks * B * heads, 7.0, np.float32)
    K, V = _bf16(rng, (4, heads * head_dim)), _bf16(rng, (4, heads * head_dim))
    slots = np.array([-1, blocks * B, blocks * B + 3, -(2 ** 31)], np.int32)
    O.scatter_kv(K, V, slots, B, heads, head_dim, fp8, kp, vp, ks, vs)
    assert np.all(kp == 0xA5) and np.all(vp == 0x5A)
    assert np.all(ks == 7.0) and np.all(vs == 7.0)
    # the last in-range slot writes
    O.scatter_kv(K[:1], V[:1], np.array([blocks * B - 1], np.int32), B, heads, head_dim, fp8, kp,
                 vp, ks, vs)
    assert not np.all(kp[-row:] == 0xA5) and np.all(kp[:-row] == 0xA5)
