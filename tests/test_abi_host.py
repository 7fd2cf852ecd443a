"""The C-ABI library: it loads, exports every entry point include/pbe_handoff.h
declares, and its host-side planning matches the oracle. No GPU needed."""
import re
from pathlib import Path

import numpy as np
import pytest

import pbe_handoff as P
import workload as W
from oracle import oracle as O

HEADER = Path(__file__).resolve().parent.parent / "include" / "pbe_handoff.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(pbe_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = P.lib()
    declared = _declared()
    assert len(declared) >= 30
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in pbe_handoff.h but not exported"
    # the Python binding covers the header except the C++-facing stream helpers
    cxx_only = {"pbe_stream_create", "pbe_stream_destroy", "pbe_stream_synchronize",
                "pbe_stream_wait_raw_event", "pbe_pointer_kind"}
    assert set(declared) - cxx_only <= set(P.EXPORTED)
    assert P.lib().pbe_version().decode().startswith("pbe-handoff")


@pytest.mark.parametrize("seed", range(12))
def test_build_runs_matches_oracle(seed):
    w = W.small(seed=seed, layers=1 + seed % 5, kv_heads=2, head_dim=64, n_pages=120,
                handoff_pages=25, max_run=1 + seed % 6)
    g = w.geometry
    kv = P.shape(g.layers, g.kv_heads, g.head_dim)
    assert P.build_runs(w.src_ids, w.dst_ids, kv) == O.coalesce(w.src_ids, w.dst_ids, g.layers)


def test_build_runs_breaks_at_segment_boundaries():
    kv = P.shape(2, 2, 64)
    page = kv.page_bytes()
    stride = 4
    src = np.arange(0, 8) * stride            # pages 0..7, contiguous
    dst = (np.arange(0, 8) + 20) * stride     # pages 20..27, contiguous
    assert P.build_runs(src, dst, kv) == [(0, 20 * stride, 8)]
    # segments of 6 pages: src breaks after page 5, dst pages 20..23 | 24..27
    runs = P.build_runs(src, dst, kv, 2, 6 * page)
    assert runs == [(0, 80, 4), (16, 96, 2), (24, 104, 2)]
    flat = [(s + k * stride, d + k * stride) for s, d, n in runs for k in range(n)]
    assert flat == list(zip(src.tolist(), dst.tolist()))


def test_validate_ids_matches_oracle_and_golden():
    import json
    cases = json.loads((Path(__file__).parent / "golden" / "validate_ids.json").read_text())["cases"]
    for c in cases:
        kv = P.KvShape(c["layers"], 1, c["half"] // 32, 16)  # 16*1*(half/32)*2 = half
        assert kv.half_bytes() == c["half"]
        assert P.validate_ids(c["ids"], kv, c["arena_bytes"]) == c["bad"], c
        assert O.validate_ids(c["ids"], c["layers"], c["half"], c["arena_bytes"]) == c["bad"]


def test_device_calls_fail_loudly_without_gpu():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(P.PbeError) as e:
        P.Arena.create(1 << 20)
    assert e.value.code == P.PBE_ERR_HIP


def test_invalid_arguments_are_rejected_on_the_host():
    kv = P.shape(2, 2, 64)
    with pytest.raises(ValueError):
        P.build_runs([0, 4], [8], kv)
    bad = P.KvShape(0, 2, 64, 16)
    with pytest.raises(P.PbeError) as e:
        P.build_runs([0], [4], bad)
    assert e.value.code == P.PBE_ERR_INVALID


def test_decode_split_count_by_page_dtype():
    """pbe_paged_decode_splits: at most 1024 waves (batch x kv_heads x splits),
    FP8 pages 2048 while every split keeps >= 8 blocks, >= 4 blocks per
    split, at most 1024 splits. The choices at 5040 tokens (315 blocks) and
    2048 tokens (128 blocks) are the ones measured fastest on MI355X."""
    fp8, bf16 = P.PBE_KV_FP8_E4M3, P.PBE_KV_BF16
    assert P.decode_splits(64, 2, 315, fp8) == 16
    assert P.decode_splits(64, 2, 315, bf16) == 8
    assert P.decode_splits(128, 2, 315, fp8) == 8
    assert P.decode_splits(128, 2, 315, bf16) == 4
    assert P.decode_splits(32, 2, 315, fp8) == 32   # 10 blocks each
    assert P.decode_splits(64, 2, 128, fp8) == 16   # 8 blocks each
    assert P.decode_splits(32, 2, 128, fp8) == 16   # 32 splits would leave 4 blocks each
    assert P.decode_splits(16, 2, 315, fp8) == 32
    assert P.decode_splits(1, 2, 10000, fp8) == 1024  # two waves per SIMD, ~10 blocks each
    assert P.decode_splits(1, 2, 2048, fp8) == 512   # a 32K-token sequence: 4 blocks per split
    assert P.decode_splits(1, 2, 315, fp8) == 79     # at least 4 blocks per split
    assert P.decode_splits(1, 1, 7, bf16) == 2      # at least 4 blocks per split
    assert P.decode_splits(4096, 8, 315, fp8) == 1
    assert P.decode_splits(0, 2, 315, fp8) == 1


def test_page_writer_and_pool_reader_reject_bad_arguments_on_the_host():
    """pbe_scatter_kv / pbe_scatter_kv_to_page / pbe_paged_decode_pools check
    dtypes, shapes and slots before any HIP call; an empty scatter is a no-op."""
    fake = 1 << 40  # never dereferenced: every case fails (or returns) first
    common = dict(keys=fake, values=fake, n_tokens=4, slots=fake, block_size=16, kv_heads=2,
                  head_dim=64, key_pool=fake, key_pool_bytes=1 << 20, value_pool=fake,
                  value_pool_bytes=1 << 20)

    def scatter(**kw):
        a = dict(common, in_dtype=P.PBE_IN_BF16, kv_dtype=P.PBE_KV_BF16)
        a.update(kw)
        P.scatter_kv(**a)

    for kw, code in [(dict(in_dtype=7), P.PBE_ERR_INVALID), (dict(kv_dtype=9), P.PBE_ERR_INVALID),
                     (dict(n_tokens=-1), P.PBE_ERR_INVALID), (dict(slots=0), P.PBE_ERR_INVALID),
                     (dict(block_size=0), P.PBE_ERR_INVALID),
                     (dict(kv_dtype=P.PBE_KV_FP8_E4M3, head_dim=48), P.PBE_ERR_UNSUPPORTED),
                     (dict(kv_dtype=P.PBE_KV_FP8_E4M3), P.PBE_ERR_INVALID),  # no scale pools
                     (dict(head_dim=3), P.PBE_ERR_INVALID)]:                  # 12-byte rows
        with pytest.raises(P.PbeError) as e:
            scatter(**kw)
        assert e.value.code == code, kw
    scatter(n_tokens=0)  # nothing to write: no device work, no error
    with pytest.raises(P.PbeError) as e:
        P.scatter_kv_to_page(fake, fake, P.PBE_IN_BF16, 3, 16, 16, 2, 64, P.PBE_KV_BF16, fake,
                             1 << 20, fake, 1 << 20)
    assert e.value.code == P.PBE_ERR_INVALID  # offset == block_size is not a slot
    with pytest.raises(P.PbeError) as e:
        P.paged_decode_pools(fake, fake, 1 << 20, 0, 0, 0, 9, 2, 128, fake, fake, 1, 12, fake,
                             fake, 4, 0, fake, 1 << 20)
    assert e.value.code == P.PBE_ERR_INVALID
    with pytest.raises(P.PbeError) as e:
        P.paged_decode_pools(fake, fake, 1 << 20, 0, 0, 0, P.PBE_KV_BF16, 2, 96, fake, fake, 1, 12,
                             fake, fake, 4, 0, fake, 1 << 20)
    assert e.value.code == P.PBE_ERR_UNSUPPORTED


def test_append_reader_rejects_bad_arguments_on_the_host():
    """pbe_paged_decode_append checks the new token's operands, and everything
    pbe_paged_decode_pools checks, before any HIP call."""
    fake = 1 << 40
    args = dict(key_pool=fake, value_pool=fake, pool_bytes=1 << 20, key_scales=0, value_scales=0,
                scale_pool_bytes=0, kv_dtype=P.PBE_KV_BF16, kv_heads=2, head_dim=128,
                new_keys=fake, new_values=fake, queries=fake, outputs=fake, batch=1, q_heads=12,
                tables=fake, seq_lens=fake, max_blocks=4, splits=0, workspace=fake,
                workspace_bytes=1 << 20)
    for kw, code in [(dict(new_keys=0), P.PBE_ERR_INVALID), (dict(new_values=0), P.PBE_ERR_INVALID),
                     (dict(new_keys=fake + 8), P.PBE_ERR_INVALID),  # not 16-byte aligned
                     (dict(kv_dtype=9), P.PBE_ERR_INVALID),
                     (dict(head_dim=96), P.PBE_ERR_UNSUPPORTED),
                     (dict(kv_dtype=P.PBE_KV_FP8_E4M3), P.PBE_ERR_INVALID),  # no scale pools
                     (dict(q_heads=13), P.PBE_ERR_UNSUPPORTED)]:
        a = dict(args)
        a.update(kw)
        with pytest.raises(P.PbeError) as e:
            P.paged_decode_append(**a)
        assert e.value.code == code, kw
