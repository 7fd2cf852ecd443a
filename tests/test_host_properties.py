"""Property-based checks of the C-ABI's host-side planning against the oracle,
on id lists hypothesis draws: any order, repeats, ids off the page stride,
negative and out-of-range ids. No GPU needed.

- pbe_validate_ids returns the oracle's first bad index on every list
  (split_pd_engine.cpp:61-67 checks each id in turn).
- pbe_build_runs equals the oracle's coalescing on page-major lists
  (split_pd_engine.cpp:96-101), and its runs flatten back to the input pairs,
  in order, with no two neighbours that could have been merged; with
  segments, no run crosses a segment boundary on either side.
"""
import numpy as np
from hypothesis import given, settings, strategies as st

import pbe_handoff as P
from oracle import oracle as O

I32 = st.integers(min_value=-(2 ** 31), max_value=2 ** 31 - 1)


def _flatten(runs, stride):
    return [(s + k * stride, d + k * stride) for s, d, n in runs for k in range(n)]


@settings(max_examples=300, deadline=None)
@given(layers=st.integers(1, 6), head_dim=st.sampled_from([8, 64, 128]),
       pages=st.integers(1, 64), ids=st.lists(st.one_of(I32, st.integers(-4, 400)), max_size=40))
def test_validate_ids_agrees_with_the_oracle(layers, head_dim, pages, ids):
    kv = P.shape(layers, 1, head_dim)
    half = kv.half_bytes()
    arena = pages * 2 * layers * half
    assert P.validate_ids(ids, kv, arena) == O.validate_ids(ids, layers, half, arena)


page_major = st.integers(1, 5).flatmap(lambda layers: st.tuples(
    st.just(layers),
    st.lists(st.tuples(st.integers(0, 300), st.integers(0, 300)), min_size=1, max_size=60)))


@settings(max_examples=300, deadline=None)
@given(case=page_major)
def test_build_runs_agrees_with_the_oracle_on_any_order(case):
    layers, pairs = case
    stride = 2 * layers
    src = [p * stride for p, _ in pairs]
    dst = [q * stride for _, q in pairs]
    kv = P.shape(layers, 2, 64)
    runs = P.build_runs(src, dst, kv)
    assert runs == O.coalesce(src, dst, layers)
    assert _flatten(runs, stride) == list(zip(src, dst))
    for (s0, d0, n0), (s1, d1, _) in zip(runs, runs[1:]):
        assert not (s1 == s0 + n0 * stride and d1 == d0 + n0 * stride), "mergeable neighbours"


@settings(max_examples=200, deadline=None)
@given(case=page_major, seg_pages=st.integers(1, 40))
def test_build_runs_never_crosses_a_segment(case, seg_pages):
    layers, pairs = case
    stride = 2 * layers
    kv = P.shape(layers, 2, 64)
    src = [p * stride for p, _ in pairs]
    dst = [q * stride for _, q in pairs]
    runs = P.build_runs(src, dst, kv, 2, seg_pages * kv.page_bytes())
    assert _flatten(runs, stride) == list(zip(src, dst))
    for s, d, n in runs:
        for start in (s // stride, d // stride):
            assert start // seg_pages == (start + n - 1) // seg_pages
    # merging may only stop where the unsegmented plan stops or a segment ends
    for (s0, d0, n0), (s1, d1, _) in zip(runs, runs[1:]):
        if s1 == s0 + n0 * stride and d1 == d0 + n0 * stride:
            assert (s1 // stride) % seg_pages == 0 or (d1 // stride) % seg_pages == 0


@settings(max_examples=100, deadline=None)
@given(n=st.integers(1, 50), seed=st.integers(0, 2 ** 32 - 1))
def test_build_runs_is_identity_on_repeated_input(n, seed):
    """A run list rebuilt from its own flattening is unchanged (idempotence)."""
    rng = np.random.default_rng(seed)
    layers = int(rng.integers(1, 4))
    stride = 2 * layers
    kv = P.shape(layers, 2, 64)
    src = (rng.integers(0, 40, n) * stride).tolist()
    dst = (rng.integers(0, 40, n) * stride).tolist()
    runs = P.build_runs(src, dst, kv)
    flat = _flatten(runs, stride)
    assert P.build_runs([a for a, _ in flat], [b for _, b in flat], kv) == runs
