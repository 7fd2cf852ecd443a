"""Pins the decode-reader oracle (oracle.paged_decode) on the CPU.

The oracle walks byte offsets the way the reference kernels do. The checks
here recompute attention from a reshaped view of the page-major arena
([page][layer][K|V][token][kv_head][D]) with natural-base softmax
exp(q.k / sqrt(D)), so a wrong offset, plane, head mapping or base-2 scale
fails them; plus closed forms (one token, no tokens, identical keys).
"""
import numpy as np
import pytest

from oracle import oracle as O


def make_case(rng, fp8, layers, H, D, kvm, seq_lens, n_pages=40):
    E = 1 if fp8 else 2
    half = 16 * H * D * E
    page = 2 * layers * half
    arena = rng.integers(0, 256, n_pages * page, dtype=np.uint8)
    if fp8:
        arena[(arena & 0x7F) == 0x7F] = 0x11  # no NaN codes in used slots
    else:
        vals = (rng.standard_normal(n_pages * page // 2) * 0.7).astype(np.float32)
        arena = O.bf16_from_f32(vals).view(np.uint8)
    scales = rng.uniform(0.01, 0.2, n_pages * 2 * layers * 16 * H).astype(np.float32) if fp8 else None
    batch = len(seq_lens)
    max_blocks = max(1, max((n + 15) // 16 for n in seq_lens))
    perm = rng.permutation(n_pages)
    tables = np.zeros((batch, max_blocks), np.int32)
    k = 0
    for b in range(batch):
        for i in range(max_blocks):
            tables[b, i] = perm[k % n_pages] * 2 * layers
            k += 1
    q = O.bf16_from_f32(rng.standard_normal((batch, H * kvm, D)).astype(np.float32))
    return arena, scales, tables, q


def natural_attention(arena, fp8, scales, layers, H, D, layer, q, tables, seq_lens):
    E = 1 if fp8 else 2
    n_pages = arena.size // (2 * layers * 16 * H * D * E)
    if fp8:
        vals = O.e4m3_table()[arena].reshape(n_pages, layers, 2, 16, H, D)
        sc = scales.astype(np.float64).reshape(n_pages, layers, 2, 16, H)
    else:
        vals = (arena.view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        vals = vals.reshape(n_pages, layers, 2, 16, H, D)
        sc = np.ones((n_pages, layers, 2, 16, H))
    qf = (q.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    batch, q_heads, _ = q.shape
    kvm = q_heads // H
    out = np.zeros((batch, q_heads, D))
    for b in range(batch):
        n = seq_lens[b]
        if n == 0:
            continue
        pages = tables[b] // (2 * layers)
        t = np.arange(n)
        pg, tok = pages[t // 16], t % 16
        for qh in range(q_heads):
            h = qh // kvm
            K = vals[pg, layer, 0, tok, h]
            V = vals[pg, layer, 1, tok, h]
            s = (K @ qf[b, qh]) / np.sqrt(D) * sc[pg, layer, 0, tok, h]
            w = np.exp(s - s.max())
            out[b, qh] = (w * sc[pg, layer, 1, tok, h]) @ V / w.sum()
    return out


@pytest.mark.parametrize("fp8,D,kvm", [(True, 128, 6), (False, 128, 6), (True, 64, 7), (False, 64, 1)])
def test_oracle_matches_natural_base_attention_on_reshaped_pages(fp8, D, kvm):
    rng = np.random.default_rng(D + kvm + fp8)
    layers, H, layer = 3, 2, 2
    seq_lens = [0, 1, 15, 16, 17, 70]
    arena, scales, tables, q = make_case(rng, fp8, layers, H, D, kvm, seq_lens)
    got = O.paged_decode(arena, fp8, scales, layers, H, D, layer, q, tables, seq_lens)
    want = natural_attention(arena, fp8, scales, layers, H, D, layer, q, tables, seq_lens)
    # the only difference: the fp32 scale constant 1/sqrt(D)*log2(e) (relative ~1e-7)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-7)


def test_closed_forms_single_token_empty_and_identical_keys():
    rng = np.random.default_rng(3)
    layers, H, D, kvm = 2, 1, 64, 2
    arena, scales, tables, q = make_case(rng, True, layers, H, D, kvm, [1, 0, 32])
    lut = O.e4m3_table()
    half = 16 * H * D
    out = O.paged_decode(arena, True, scales, layers, H, D, 1, q, tables, [1, 0, 32])
    # one token: the output is its value row times its value scale
    vid = tables[0, 0] + 2 * 1 + 1
    v0 = lut[arena[vid * half: vid * half + D]] * scales[vid * 16 * H]
    assert np.allclose(out[0, 0], v0, rtol=1e-12) and np.allclose(out[0, 1], v0, rtol=1e-12)
    assert not out[1].any()  # no tokens: zeros
    # identical keys and key scales in both blocks of sequence 2: the mean of the scaled values
    k0 = (tables[2, 0] + 2) * half
    row = arena[k0: k0 + D].copy()
    for blk in range(2):
        kid = tables[2, blk] + 2
        arena[kid * half:(kid + 1) * half] = np.tile(row, 16)
        scales[kid * 16: kid * 16 + 16] = 0.05
    out = O.paged_decode(arena, True, scales, layers, H, D, 1, q, tables, [1, 0, 32])
    vals = []
    for blk in range(2):
        vid = tables[2, blk] + 3
        for tok in range(16):
            off = vid * half + tok * D
            vals.append(lut[arena[off: off + D]] * scales[vid * 16 + tok])
    assert np.allclose(out[2, 0], np.mean(vals, axis=0), rtol=1e-9)


@pytest.mark.parametrize("fp8", [True, False])
def test_pool_addressing_equals_page_major_on_layer_views_and_moved_blocks(fp8):
    """oracle.paged_decode_pools (per-layer pools, the reference kernels'
    addressing) against the pinned page-major form: (1) over a shared arena's
    layer views (key = arena + 2l*half, value = key + half) with the same ids;
    (2) over separate local K and V pools into which every used block was moved
    to a new id, with the tables renumbered. Both must be exactly equal."""
    rng = np.random.default_rng(41 + fp8)
    layers, H, D, kvm, layer = 3, 2, 64, 3, 1
    seq_lens = [40, 17, 0, 33]
    arena, scales, tables, q = make_case(rng, fp8, layers, H, D, kvm, seq_lens)
    E = 1 if fp8 else 2
    half = 16 * H * D * E
    plane = 16 * H
    want = O.paged_decode(arena, fp8, scales, layers, H, D, layer, q, tables, seq_lens)
    views = O.paged_decode_pools(arena[2 * layer * half:], arena[(2 * layer + 1) * half:], fp8,
                                 scales[2 * layer * plane:] if fp8 else None,
                                 scales[(2 * layer + 1) * plane:] if fp8 else None, H, D, q, tables,
                                 seq_lens)
    assert np.array_equal(views, want)
    # local pools: block ids renumbered 0..n-1 in a shuffled order
    used = sorted(set(tables.ravel().tolist()))
    new_id = dict(zip(used, rng.permutation(len(used)).tolist()))
    kp = np.zeros(len(used) * half, np.uint8)
    vp = np.zeros(len(used) * half, np.uint8)
    ks = np.zeros(len(used) * plane, np.float32)
    vs = np.zeros(len(used) * plane, np.float32)
    for old, new in new_id.items():
        k_plane, v_plane = old + 2 * layer, old + 2 * layer + 1
        kp[new * half:(new + 1) * half] = arena[k_plane * half:(k_plane + 1) * half]
        vp[new * half:(new + 1) * half] = arena[v_plane * half:(v_plane + 1) * half]
        if fp8:
            ks[new * plane:(new + 1) * plane] = scales[k_plane * plane:(k_plane + 1) * plane]
            vs[new * plane:(new + 1) * plane] = scales[v_plane * plane:(v_plane + 1) * plane]
    local_tables = np.vectorize(new_id.get)(tables).astype(np.int32)
    moved = O.paged_decode_pools(kp, vp, fp8, ks if fp8 else None, vs if fp8 else None, H, D, q,
                                 local_tables, seq_lens)
    assert np.array_equal(moved, want)
