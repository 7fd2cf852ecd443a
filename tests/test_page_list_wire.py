"""Compact page-list wire form (pbe_page_list_*), host only.

The reference ships a prefill's page list as one JSON integer array per layer
(remote_prefill_result_to_json, serving_zmq_rpc.cpp:222-253) and copy_shared_kv
requires the arrays to be identical page-major lists (split_pd_engine.cpp:63-80).
The expected bytes below are written out from the format definition in
include/pbe_handoff.h (little-endian header, {first, pages} spans, FNV-1a 32),
with FNV-1a itself pinned by its published test vectors.
"""
import json
import random
import struct

import numpy as np
import pytest

import pbe_handoff as P
import workload as W


def fnv1a32(data: bytes, h: int = 0x811C9DC5) -> int:
    for b in data:
        h = ((h ^ b) * 0x01000193) & 0xFFFFFFFF
    return h


def test_fnv1a_published_vectors():
    assert fnv1a32(b"") == 0x811C9DC5
    assert fnv1a32(b"a") == 0xE40C292C
    assert fnv1a32(b"foobar") == 0xBF9CF968


def spec_bytes(spans, layers, epoch):
    n_pages = sum(k for _, k in spans)
    body = b"".join(struct.pack("<ii", f, k) for f, k in spans)
    head0 = struct.pack("<IHHiiiIQ", 0x50454250, 1, 32, layers, n_pages, len(spans), 0, epoch)
    c = fnv1a32(body, fnv1a32(head0))
    return struct.pack("<IHHiiiIQ", 0x50454250, 1, 32, layers, n_pages, len(spans), c, epoch) + body


def test_hand_worked_case_matches_format_definition():
    # L = 4: page stride 8. Spans: 0,8,16 | 64,72 | 24
    ids = [0, 8, 16, 64, 72, 24]
    wire = P.encode_page_list(ids, 4, 0x0102030405060708)
    assert wire[:4] == b"PBEP"
    assert wire == spec_bytes([(0, 3), (64, 2), (24, 1)], 4, 0x0102030405060708)
    assert len(wire) == 32 + 3 * 8
    back, layers, epoch = P.decode_page_list(wire)
    assert back.tolist() == ids and layers == 4 and epoch == 0x0102030405060708


def brute_spans(ids, layers):
    spans = []
    for i, x in enumerate(ids):
        if i and x == ids[i - 1] + 2 * layers:
            spans[-1][1] += 1
        else:
            spans.append([x, 1])
    return [tuple(s) for s in spans]


@pytest.mark.parametrize("seed", range(20))
def test_random_lists_round_trip_bit_exact(seed):
    rng = random.Random(seed)
    layers = rng.choice([1, 2, 24, 28, 80])
    stride = 2 * layers
    n = rng.choice([0, 1, 2, 7, 64, 500])
    pages = rng.sample(range(0, 20000), n)
    # splice in consecutive stretches so spans longer than one page occur
    ids = []
    for p in pages:
        ids.extend(range(p * stride, (p + rng.randint(1, 5)) * stride, stride))
    ids = ids[:max(n, 0) * 3]
    wire = P.encode_page_list(ids, layers, seed + 1)
    assert wire == spec_bytes(brute_spans(ids, layers), layers, seed + 1)
    assert P.lib().pbe_page_list_bytes(np.asarray(ids, np.int32).ctypes.data_as(P.C.c_void_p)
                                       if ids else None, len(ids), layers) == len(wire)
    back, lay, ep = P.decode_page_list(wire)
    assert back.tolist() == ids and lay == layers and ep == seed + 1


def test_largest_ids_and_long_span():
    layers = 1
    top = 2**31 - 2  # largest even int32: the last valid page id for 2L = 2
    ids = list(range(top - 2 * 999, top + 1, 2))
    wire = P.encode_page_list(ids, layers, 3)
    assert len(wire) == 40
    back, _, _ = P.decode_page_list(wire)
    assert back[-1] == top and len(back) == 1000


def test_invalid_ids_are_rejected_at_encode():
    for ids in ([0, 3], [-2], [4, 10]):  # 2L = 4: 3, -2 and 10 are not page ids
        with pytest.raises(P.PbeError):
            P.encode_page_list(ids, 2, 1)
    with pytest.raises(P.PbeError):
        P.encode_page_list([0], 0, 1)


def test_every_single_bit_flip_truncation_and_extension_is_rejected():
    wire = P.encode_page_list([0, 4, 8, 40, 44, 100 * 4], 2, 12345)
    for i in range(len(wire)):
        for bit in range(8):
            bad = bytearray(wire)
            bad[i] ^= 1 << bit
            with pytest.raises(P.PbeError):
                P.decode_page_list(bytes(bad))
    for cut in range(len(wire)):
        with pytest.raises(P.PbeError):
            P.decode_page_list(wire[:cut])
    with pytest.raises(P.PbeError):
        P.decode_page_list(wire + b"\0" * 8)


def test_short_list_claiming_millions_of_pages_is_bounded():
    """40 bytes can claim 2^22 + 1 pages: rejected before anything is
    allocated unless the caller's bound (its arena capacity) allows them."""
    wire = spec_bytes([(0, (1 << 22) + 1)], 1, 3)
    assert len(wire) == 40
    with pytest.raises(P.PbeError):
        P.decode_page_list(wire)
    with pytest.raises(P.PbeError):
        P.decode_page_list(spec_bytes([(0, 1000)], 1, 3), max_pages=999)
    ids, layers, epoch = P.decode_page_list(wire, max_pages=1 << 23)
    assert len(ids) == (1 << 22) + 1 and ids[-1] == 2 << 22 and layers == 1 and epoch == 3


def test_structurally_bad_lists_with_valid_checksums_are_rejected():
    cases = [
        [(0, 0)],                # span without pages
        [(-4, 1)],               # negative id
        [(6, 1)],                # not a multiple of 2L = 4
        [(2**31 - 4, 2)],        # second page beyond INT32_MAX
    ]
    for spans in cases:
        with pytest.raises(P.PbeError):
            P.decode_page_list(spec_bytes(spans, 2, 1))
    # span totals disagree with n_pages
    good = spec_bytes([(0, 2)], 2, 1)
    hdr = list(struct.unpack("<IHHiiiIQ", good[:32]))
    hdr[4] = 3
    hdr[6] = 0
    body = good[32:]
    hdr[6] = fnv1a32(body, fnv1a32(struct.pack("<IHHiiiIQ", *hdr)))
    with pytest.raises(P.PbeError):
        P.decode_page_list(struct.pack("<IHHiiiIQ", *hdr) + body)


def test_config2_page_list_is_far_smaller_than_per_layer_json():
    w = W.config2(0)
    g = w.geometry
    ids = w.src_ids
    wire = P.encode_page_list(ids, g.layers, 1)
    layers_json = json.dumps([{"layer_idx": l, "src_block_ids": ids.tolist(), "blocks": []}
                              for l in range(g.layers)])
    spans = brute_spans(ids.tolist(), g.layers)
    assert len(wire) == 32 + 8 * len(spans)
    assert len(wire) * 100 < len(layers_json)
    back, _, _ = P.decode_page_list(wire)
    assert np.array_equal(back, ids)


def test_fuzzed_input_is_rejected_or_round_trips():
    """Arbitrary bytes, and valid lists with random byte edits and checksums
    recomputed over the edit: decoding either raises PbeError or yields a list
    whose encoding is exactly the input (nothing else is accepted)."""
    hyp = pytest.importorskip("hypothesis")
    st = hyp.strategies

    def check(data: bytes):
        try:
            ids, layers, epoch = P.decode_page_list(data, max_pages=1 << 16)
        except P.PbeError:
            return
        assert P.encode_page_list(ids, layers, epoch) == data

    @hyp.settings(max_examples=300, deadline=None, derandomize=True)
    @hyp.given(st.binary(max_size=200))
    def raw(data):
        check(data)

    @hyp.settings(max_examples=300, deadline=None, derandomize=True)
    @hyp.given(st.lists(st.tuples(st.integers(-8, 1 << 20), st.integers(-2, 50)), max_size=6),
               st.integers(1, 64), st.integers(0, 2**64 - 1))
    def spans(sp, layers, epoch):
        check(spec_bytes(sp, layers, epoch))

    raw()
    spans()
