"""Pins the CPU oracle (oracle/pbe_oracle.c) against golden vectors, closed
forms, brute force and third-party conversions, so that it can serve as the
checker of the HIP kernels. CPU only."""
import json
import math
from pathlib import Path

import numpy as np
import pytest

import workload as W
from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def _f(x):
    return float(x) if not isinstance(x, str) else float(x.replace("inf", "inf"))


# ------------------------------------------------------------------ FP8 E4M3

def test_e4m3_golden_cases():
    cases = json.loads((GOLDEN / "e4m3_cases.json").read_text())["cases"]
    xs = np.array([_f(c["x"]) for c in cases], np.float32)
    got = O.e4m3_from_f32(xs)
    for c, g in zip(cases, got.tolist()):
        assert g == c["code"], f"{c} -> {g:#04x}"


def _brute_e4m3(x: float) -> int:
    """Nearest representable value by exhaustive search over the 256 codes,
    ties to the even code; values whose magnitude exceeds 448 saturate."""
    if math.isnan(x):
        return 0x7F
    vals = []
    for code in range(256):
        e, m, s = (code >> 3) & 15, code & 7, -1.0 if code & 0x80 else 1.0
        if (code & 0x7F) == 0x7F:
            continue
        v = s * (m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
        vals.append((v, code))
    if abs(x) >= 448:
        return 0xFE if x < 0 else 0x7E
    best = min(abs(v - x) for v, _ in vals)
    cands = [c for v, c in vals if abs(v - x) == best]
    if len(cands) > 1:  # a tie, or +0/-0
        if x == 0 or all((c & 0x7F) == 0 for c in cands):
            return 0x80 if math.copysign(1, x) < 0 else 0x00
        cands = [c for c in cands if (c & 1) == 0]
    c = cands[0]
    if (c & 0x7F) == 0:  # zero result keeps the input's sign
        return 0x80 if math.copysign(1, x) < 0 else 0x00
    return c


def test_e4m3_matches_brute_force_search():
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(3000).astype(np.float32) * 50,
        rng.standard_normal(1000).astype(np.float32) * 0.01,
        (rng.uniform(-1, 1, 1000) * 2.0 ** -8).astype(np.float32),
        np.float32([0.0, -0.0, 448, -448, 447.99, 464.0, 480.0, 1e-40, -1e-40]),
    ])
    got = O.e4m3_from_f32(xs)
    for x, g in zip(xs.tolist(), got.tolist()):
        assert g == _brute_e4m3(x), (x, hex(g), hex(_brute_e4m3(x)))


def test_e4m3_matches_torch_in_range():
    """Third-party check: torch's float8_e4m3fn cast (round to nearest even,
    no saturation) on every BF16 value times a spread of multipliers, where
    the product stays within +-448."""
    torch = pytest.importorskip("torch")
    bits = np.arange(65536, dtype=np.uint32) << 16
    base = bits.view(np.float32)
    for inv in (1.0, 448.0 / 3.7, 448.0 / 0.013, 448.0 / 250.0, 0.5):
        with np.errstate(over="ignore", invalid="ignore"):
            x = (base * np.float32(inv)).astype(np.float32)
        keep = np.isfinite(x) & (np.abs(x) <= 448)
        x = x[keep]
        want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        got = O.e4m3_from_f32(x)
        bad = np.nonzero(got != want)[0]
        assert len(bad) == 0, f"inv={inv}: {x[bad[:5]]} -> {got[bad[:5]]} vs {want[bad[:5]]}"


def test_e4m3_decode_round_trip():
    for code in range(256):
        if (code & 0x7F) == 0x7F:
            assert math.isnan(O.e4m3_to_f32(code))
            continue
        v = O.e4m3_to_f32(code)
        back = int(O.e4m3_from_f32(np.float32([v]))[0])
        assert back == code or (v == 0 and (back & 0x7F) == 0), (code, v, back)


def test_e4m3_decode_matches_torch_float8_e4m3fn():
    """Every one of the 256 codes decodes to torch's float8_e4m3fn value (the
    OCP E4M3 'fn' format: no infinities, 0x7F/0xFF NaN)."""
    torch = pytest.importorskip("torch")
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    want = codes.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    got = O.e4m3_table()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])


# ------------------------------------------------------------------ BF16

def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 1.5,
                        np.float32([0, -0.0, 1e-40, 3.4e38, -3.4e38, 1.00390625, 1.01171875])])
    got = O.bf16_from_f32(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ coalescing

def test_coalesce_golden_runs():
    for c in json.loads((GOLDEN / "handoff_runs.json").read_text())["cases"]:
        runs = O.coalesce(c["src"], c["dst"], c["layers"])
        assert [list(r) for r in runs] == c["runs"], c


@pytest.mark.parametrize("seed", range(20))
def test_coalesce_runs_are_maximal_and_cover_the_plan(seed):
    rng = np.random.default_rng(seed)
    L = int(rng.integers(1, 6))
    stride = 2 * L
    n = int(rng.integers(1, 40))
    # random plan with deliberate contiguous stretches
    src, dst = [], []
    s, d = int(rng.integers(0, 50)), int(rng.integers(100, 150))
    for _ in range(n):
        if rng.random() < 0.4:
            s, d = int(rng.integers(0, 500)), int(rng.integers(600, 1100))
        else:
            s, d = s + 1, d + (1 if rng.random() < 0.8 else 3)
        src.append(s * stride)
        dst.append(d * stride)
    runs = O.coalesce(src, dst, L)
    # concatenation of the runs reproduces the plan
    flat_s = [r[0] + k * stride for r in runs for k in range(r[2])]
    flat_d = [r[1] + k * stride for r in runs for k in range(r[2])]
    assert flat_s == src and flat_d == dst
    # maximality: consecutive runs could not have been merged
    for a, b in zip(runs, runs[1:]):
        assert not (b[0] == a[0] + a[2] * stride and b[1] == a[1] + a[2] * stride)


# ------------------------------------------------------------------ copies

def _page_pattern_arena(g: W.Geometry, n_pages: int) -> np.ndarray:
    """Every plane of page p filled with the byte (p*7 + 64*plane + layer) & 0xff,
    the page-major layout pinned by demo/shared_kv_reuse_probe.cpp:76-83
    (byte at offset + (2l + plane)*half == pattern + 64*plane + l)."""
    half = g.half()
    a = np.zeros(n_pages * g.page_bytes(), np.uint8)
    for p in range(n_pages):
        for l in range(g.layers):
            for plane in range(2):
                off = p * g.page_bytes() + (2 * l + plane) * half
                a[off:off + half] = (p * 7 + 64 * plane + l) & 0xFF
    return a


@pytest.mark.parametrize("seed", range(4))
def test_copy_handoff_closed_form_and_canaries(seed):
    w = W.small(seed=seed, layers=3, kv_heads=2, head_dim=16, n_pages=80, handoff_pages=11,
                max_run=4)
    g = w.geometry
    n_pages = w.arena_bytes // g.page_bytes()
    arena = _page_pattern_arena(g, n_pages)
    before = arena.copy()
    copied = O.copy_handoff(arena, w.src_ids, w.dst_ids, g.half(), g.layers)
    assert copied == w.pages * g.page_bytes()
    dst_pages = set((w.dst_ids // g.stride).tolist())
    for sp, dp in zip((w.src_ids // g.stride).tolist(), (w.dst_ids // g.stride).tolist()):
        for l in range(g.layers):
            for plane in range(2):
                off = dp * g.page_bytes() + (2 * l + plane) * g.half()
                assert np.all(arena[off:off + g.half()] == ((sp * 7 + 64 * plane + l) & 0xFF))
    for p in range(n_pages):
        if p not in dst_pages:
            s = slice(p * g.page_bytes(), (p + 1) * g.page_bytes())
            assert np.array_equal(arena[s], before[s]), f"canary page {p} changed"


@pytest.mark.parametrize("seed", range(4))
def test_run_and_component_forms_agree(seed):
    """The reference's two decompositions of the same copy (one memcpy per run,
    split_pd_engine.cpp:96-108, and 2*layers memcpys per page,
    pd_handoff.cpp:192-213) give identical arenas."""
    w = W.small(seed=10 + seed, layers=4, kv_heads=2, head_dim=32, n_pages=96, handoff_pages=20,
                max_run=5)
    g = w.geometry
    rng = np.random.default_rng(seed)
    a = rng.integers(0, 256, w.arena_bytes, dtype=np.uint8)
    b = a.copy()
    O.copy_handoff(a, w.src_ids, w.dst_ids, g.half(), g.layers)
    O.copy_components(b, w.src_ids, w.dst_ids, g.half(), g.layers)
    assert np.array_equal(a, b)


def test_validate_ids_golden():
    for c in json.loads((GOLDEN / "validate_ids.json").read_text())["cases"]:
        assert O.validate_ids(c["ids"], c["layers"], c["half"], c["arena_bytes"]) == c["bad"], c


# ------------------------------------------------------------------ FP8 handoff

def _fp8_pools(g: W.Geometry, n_pages: int, seed: int, outliers: bool):
    rng = np.random.default_rng(seed)
    vals = rng.standard_normal(n_pages * g.page_bytes(2) // 2).astype(np.float32)
    if outliers:
        m = rng.random(vals.size) < 0.01
        vals[m] = np.where(rng.random(m.sum()) < 0.5, -40.0, 40.0)
    src = O.bf16_from_f32(vals).view(np.uint8)
    dst = np.zeros(n_pages * g.page_bytes(1), np.uint8)
    scale_page = 2 * g.layers * g.page_tokens * g.kv_heads * 4
    scales = np.zeros(n_pages * scale_page, np.uint8)
    return src, dst, scales


def _rows(buf: np.ndarray, g: W.Geometry, page: int, elem: int, dtype):
    """View of one page as [2L][tokens][heads][head_dim]."""
    n = g.page_bytes(elem)
    return buf[page * n:(page + 1) * n].view(dtype).reshape(
        2 * g.layers, g.page_tokens, g.kv_heads, g.head_dim)


@pytest.mark.parametrize("head_dim", [8, 64, 128])
def test_fp8_token_head_properties(head_dim):
    """Per-row closed forms of scatter_kv_kernel.cu:166-211: the row's scale is
    amax/448 in the slot [page][layer][K|V][token][head]; the amax element maps
    to +-448 (code 0x7E/0xFE); every element decodes to within half an E4M3
    ulp of x/scale; rows land at the destination page's FP8 offset."""
    g = W.Geometry(3, 2, head_dim)
    w = W.small(seed=head_dim, layers=3, kv_heads=2, head_dim=head_dim, n_pages=48,
                handoff_pages=7, max_run=3)
    src, dst, scales = _fp8_pools(g, 48, head_dim, outliers=True)
    O.fp8_handoff_token_head(src, dst, scales, w.src_ids, w.dst_ids, g.layers, g.page_tokens,
                             g.kv_heads, g.head_dim)
    table = np.array([O.e4m3_to_f32(c) for c in range(256)], np.float32)
    sc_page = 2 * g.layers * g.page_tokens * g.kv_heads
    written = set()
    divided = []
    for sp, dp in zip((w.src_ids // g.stride).tolist(), (w.dst_ids // g.stride).tolist()):
        x = _rows(src, g, sp, 2, np.uint16).astype(np.uint32) << 16
        x = x.view(np.float32)
        q = _rows(dst, g, dp, 1, np.uint8)
        s = scales.view(np.float32)[dp * sc_page:(dp + 1) * sc_page].reshape(
            2 * g.layers, g.page_tokens, g.kv_heads)
        amax = np.abs(x).max(axis=-1)
        assert np.array_equal(s, np.where(amax > 0, amax / np.float32(448), np.float32(1)))
        deq = table[q] * s[..., None]
        err = np.abs(deq - x)
        # half an ulp of E4M3 relative to the value (3 mantissa bits) plus the
        # subnormal step, both in units of the row scale
        bound = (np.abs(x) * 2.0 ** -4 + 2.0 ** -10 * s[..., None]) * 1.0001
        assert np.all(err <= bound)
        peak = q[np.abs(x) == amax[..., None]]
        assert np.all((peak & 0x7F) == 0x7E)
        # element by element, in the reference's order (scatter_kv_kernel.cu:
        # 205-206): inv = 448/amax once per row in fp32, then e4m3(x * inv)
        # through the independently pinned scalar conversion
        inv = np.where(amax > 0, np.float32(448) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
        prod = (x * inv[..., None]).astype(np.float32)
        assert np.array_equal(q, O.e4m3_from_f32(prod))
        # dividing by the stored scale instead rounds some elements differently
        by_scale = (x / s[..., None]).astype(np.float32)
        divided.append(O.e4m3_from_f32(by_scale) != q)
        written.add(dp)
    untouched = [p for p in range(48) if p not in written]
    for p in untouched:
        assert not _rows(dst, g, p, 1, np.uint8).any()
    # the element-wise check above tells the two orders apart on this data
    assert any(d.any() for d in divided)


def test_fp8_table_mode_matches_elementwise_conversion():
    """Table mode: q = e4m3(x * 448/amax[layer, K|V, head]) element by element;
    checked through the (independently pinned) scalar conversion."""
    g = W.Geometry(2, 2, 64)
    w = W.small(seed=3, layers=2, kv_heads=2, head_dim=64, n_pages=40, handoff_pages=6)
    src, dst, _ = _fp8_pools(g, 40, 3, outliers=True)
    amax = np.random.default_rng(3).uniform(2.5, 5.0, (2 * g.layers, g.kv_heads)).astype(np.float32)
    O.fp8_handoff_table(src, dst, amax, w.src_ids, w.dst_ids, g.layers, g.page_tokens, g.kv_heads,
                        g.head_dim)
    inv = (np.float32(448) / amax).astype(np.float32)
    for sp, dp in zip((w.src_ids // g.stride).tolist(), (w.dst_ids // g.stride).tolist()):
        x = (_rows(src, g, sp, 2, np.uint16).astype(np.uint32) << 16).view(np.float32)
        prod = (x * inv[:, None, :, None]).astype(np.float32)
        want = O.e4m3_from_f32(prod)
        assert np.array_equal(_rows(dst, g, dp, 1, np.uint8), want)
    assert np.allclose(O.table_scales(amax), amax / 448)
