"""The allocation-free decode entry point (pbe_paged_decode_noalloc) against
pbe_paged_decode with a caller workspace: the same kernels with the same split
count, so outputs must be bit-identical. Two calls in a row, the second with a
smaller batch, so stale partials of the first call would show; then a launch
whose partials exceed the static scratch is rejected before any device work."""
import numpy as np
import pytest

import pbe_handoff as P
from tests.conftest import say
from tests.gpu_util import stream_ptr
from tests.test_gpu_decode import DecodeCase, bf16_to_f64, close

pytestmark = pytest.mark.gpu


def _noalloc(case, splits):
    torch = case.torch
    P.paged_decode_noalloc(case.view, P.PBE_KV_FP8_E4M3 if case.fp8 else P.PBE_KV_BF16,
                           case.scales.data_ptr() if case.fp8 else 0,
                           case.scales.numel() * 4 if case.fp8 else 0, case.kv, case.layer,
                           case.q.data_ptr(), case.out.data_ptr(), case.batch, case.H * case.kvm,
                           case.t_dev.data_ptr(), case.s_dev.data_ptr(), case.max_blocks, splits,
                           stream_ptr(torch))
    torch.cuda.synchronize()
    return case.out.cpu().numpy().copy()


@pytest.mark.parametrize("fp8", [True, False])
def test_noalloc_decode_equals_workspace_decode_twice(torch_cuda, fp8):
    big = DecodeCase(torch_cuda, fp8=fp8, layers=3, H=2, D=128, kvm=6,
                     seq_lens=[700, 1, 33, 512, 0, 129, 64, 300], seed=11)
    small = DecodeCase(torch_cuda, fp8=fp8, layers=3, H=2, D=128, kvm=6,
                       seq_lens=[17, 250, 16], seed=12)
    for name, case in (("big", big), ("small", small)):
        say(f"noalloc decode fp8={fp8} {name} batch={case.batch}")
        dtype = P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16
        splits = P.decode_splits(case.batch, case.H, case.max_blocks, dtype)
        need = P.decode_workspace_bytes(case.batch, case.H * case.kvm, case.D, splits)
        assert need <= P.PBE_DECODE_SCRATCH_BYTES
        case.out.fill_(0)
        case.run(splits=splits)
        want_bits = case.out.cpu().numpy().view(np.uint16).copy()
        case.out.fill_(0)
        got_bits = _noalloc(case, splits).view(np.uint16)
        assert np.array_equal(got_bits, want_bits)  # bit-identical, NaN rows included
        assert close(bf16_to_f64(got_bits), case.oracle()).all()


def test_noalloc_decode_rejects_partials_beyond_the_scratch(torch_cuda):
    case = DecodeCase(torch_cuda, fp8=True, layers=2, H=2, D=128, kvm=8,
                      seq_lens=[64] * 4, seed=3)
    # 4 sequences x 16 query heads x 64 splits x (128 + 2) floats = 2.1 MB fits;
    # a batch claiming 64 sequences with 64 splits needs 34 MB and must be refused
    say("noalloc decode over-size rejection")
    need = P.decode_workspace_bytes(64, 16, 128, 64)
    assert need > P.PBE_DECODE_SCRATCH_BYTES
    t = torch_cuda.full((64, case.max_blocks), -1, dtype=torch_cuda.int32, device="cuda")
    s = torch_cuda.zeros(64, dtype=torch_cuda.int32, device="cuda")
    q = torch_cuda.zeros((64, 16, 128), dtype=torch_cuda.int16, device="cuda")
    out = torch_cuda.full((64, 16, 128), 7, dtype=torch_cuda.int16, device="cuda")
    with pytest.raises(P.PbeError, match="static scratch"):
        P.paged_decode_noalloc(case.view, P.PBE_KV_FP8_E4M3, case.scales.data_ptr(),
                               case.scales.numel() * 4, case.kv, case.layer, q.data_ptr(),
                               out.data_ptr(), 64, 16, t.data_ptr(), s.data_ptr(), case.max_blocks,
                               64, stream_ptr(torch_cuda))
    torch_cuda.cuda.synchronize()
    assert bool((out == 7).all())  # nothing was launched


def test_noalloc_decode_lowers_an_automatic_split_count_to_fit(torch_cuda):
    # 16 sequences x 8 KV heads x 8 query heads each: the automatic FP8 count
    # (two waves per SIMD) needs more partials than the static scratch holds,
    # so splits = 0 must run at the largest count that fits, bit-identical to
    # the workspace form at that count.
    case = DecodeCase(torch_cuda, fp8=True, layers=1, H=8, D=128, kvm=8,
                      seq_lens=[4090] * 15 + [1000], seed=21)
    q_heads = case.H * case.kvm
    auto = P.decode_splits(case.batch, case.H, case.max_blocks, P.PBE_KV_FP8_E4M3)
    per_split = P.decode_workspace_bytes(case.batch, q_heads, case.D, 1)
    fit = min(auto, P.PBE_DECODE_SCRATCH_BYTES // per_split)
    say(f"noalloc decode automatic splits: auto={auto} fit={fit}")
    assert P.decode_workspace_bytes(case.batch, q_heads, case.D, auto) > P.PBE_DECODE_SCRATCH_BYTES
    assert 1 <= fit < auto
    case.out.fill_(0)
    case.run(splits=fit)
    want_bits = case.out.cpu().numpy().view(np.uint16).copy()
    case.out.fill_(0)
    got_bits = _noalloc(case, 0).view(np.uint16)
    assert np.array_equal(got_bits, want_bits)
    assert not np.isnan(bf16_to_f64(got_bits)).any()


def test_noalloc_decode_refuses_a_second_stream_while_the_first_is_queued(torch_cuda):
    # Stream a is held by a host function (bounded: it returns after 20 s at
    # the latest, and the gate is opened in every case), so a call queued on
    # it keeps the static scratch in use; a call on stream b must then be
    # refused with PBE_ERR_BUSY before it queues anything, while a second call
    # on stream a is accepted (stream order serialises it).
    import ctypes
    import threading
    torch = torch_cuda
    case = DecodeCase(torch, fp8=True, layers=2, H=2, D=128, kvm=6,
                      seq_lens=[300, 17, 64], seed=31)
    dtype = P.PBE_KV_FP8_E4M3
    splits = P.decode_splits(case.batch, case.H, case.max_blocks, dtype)
    case.out.fill_(0)
    case.run(splits=splits)
    want_bits = case.out.cpu().numpy().view(np.uint16).copy()

    def call(out, stream):
        P.paged_decode_noalloc(case.view, dtype, case.scales.data_ptr(), case.scales.numel() * 4,
                               case.kv, case.layer, case.q.data_ptr(), out.data_ptr(), case.batch,
                               case.H * case.kvm, case.t_dev.data_ptr(), case.s_dev.data_ptr(),
                               case.max_blocks, splits, stream)

    hip = ctypes.CDLL("libamdhip64.so.7")
    hostfn = ctypes.CFUNCTYPE(None, ctypes.c_void_p)
    hip.hipLaunchHostFunc.argtypes = [ctypes.c_void_p, hostfn, ctypes.c_void_p]
    gate = threading.Event()

    def hold(_):
        gate.wait(20)

    hold_fn = hostfn(hold)  # kept alive until both streams have drained
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    out_a = torch.zeros_like(case.out)
    out_b = torch.full_like(case.out, 7)
    torch.cuda.synchronize()
    say("noalloc decode guard: stream a gated, call on a, then on b")
    refused = None
    try:
        assert hip.hipLaunchHostFunc(a.cuda_stream, hold_fn, None) == 0
        call(out_a, a.cuda_stream)  # queued behind the gate
        try:
            call(out_b, b.cuda_stream)
        except P.PbeError as e:
            refused = e
        call(out_a, a.cuda_stream)  # same stream: accepted
    finally:
        gate.set()
    a.synchronize()
    torch.cuda.synchronize()
    assert refused is not None and refused.code == P.PBE_ERR_BUSY, refused
    assert bool((out_b == 7).all())  # the refused call queued nothing
    assert np.array_equal(out_a.cpu().numpy().view(np.uint16), want_bits)
    # once stream a has drained, stream b is accepted and bit-identical
    call(out_b, b.cuda_stream)
    b.synchronize()
    assert np.array_equal(out_b.cpu().numpy().view(np.uint16), want_bits)
