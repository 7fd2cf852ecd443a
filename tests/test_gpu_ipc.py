"""Cross-process handoff on one GPU: an owner process exports a segmented
arena (hipIpcGetMemHandle per segment), prefill processes write their KV and
set IPC "KV written" signals, and the decode process's stream waits on those
signals on the GPU, copies every request with one run-list kernel and sets a
"copy done" signal that the prefill processes' streams wait on before retiring
their pages. The decode side then checks the whole arena."""
import multiprocessing as mp

import pytest

import workload as W
from tests import ipc_workers as IW
from tests.conftest import say

pytestmark = pytest.mark.gpu


def _recv(conn, what, timeout=120.0):
    if not conn.poll(timeout):
        raise TimeoutError(f"no {what}")
    return conn.recv()


def _run(kv_shape, arena_bytes, segment_bytes, requests):
    ctx = mp.get_context("spawn")
    procs, conns = [], {}

    def start(name, target, *args):
        parent, child = ctx.Pipe()
        p = ctx.Process(target=target, args=(child, *args), name=name)
        p.start()
        procs.append(p)
        conns[name] = parent

    try:
        start("owner", IW.owner, arena_bytes, segment_bytes, 77)
        for i, (src, _) in enumerate(requests):
            start(f"prefill{i}", IW.prefill, kv_shape, list(map(int, src)), 1000 + i)
        start("decode", IW.decode, kv_shape, [(list(map(int, s)), list(map(int, d))) for s, d in requests],
              len(requests))
        msg = _recv(conns["owner"], "arena export")
        assert "ipc" in msg, msg
        for name in conns:
            if name != "owner":
                conns[name].send(msg["ipc"])
        for i in range(len(requests)):
            ev = _recv(conns[f"prefill{i}"], f"prefill{i} event")
            assert "event" in ev, ev
            conns["decode"].send(ev["event"])
        done = _recv(conns["decode"], "copy-done event")
        assert "done_event" in done, done
        for i in range(len(requests)):
            conns[f"prefill{i}"].send(done["done_event"])
        for i in range(len(requests)):
            r = _recv(conns[f"prefill{i}"], f"prefill{i} result")
            assert r["ok"], r
        result = _recv(conns["decode"], "decode result")
        conns["decode"].send("exit")
        conns["owner"].send("shutdown")
        o = _recv(conns["owner"], "owner shutdown")
        assert o["ok"], o
        for p in procs:
            p.join(timeout=60)
        return result
    finally:
        for p in procs:
            if p.is_alive():
                p.terminate()
                p.join(timeout=10)


def test_ipc_handoff_small_two_segments():
    w = W.small(seed=21, layers=2, kv_heads=2, head_dim=64, n_pages=64, handoff_pages=12,
                max_run=4, segment_pages=32)
    g = w.geometry
    say("ipc small: owner + 1 prefill + decode, 2 segments")
    r = _run((g.layers, g.kv_heads, g.head_dim, g.page_tokens), w.arena_bytes, w.segment_bytes,
             [(w.src_ids, w.dst_ids)])
    assert r["ok"], r


def test_ipc_handoff_config5_two_prefills():
    w = W.config5(0)
    g = w.geometry
    say("ipc config5: owner + 2 prefills (32768 + 512 tokens) + decode, 3 segments")
    r = _run((g.layers, g.kv_heads, g.head_dim, g.page_tokens), w.arena_bytes, w.segment_bytes,
             [(q.src_ids, q.dst_ids) for q in w.requests])
    print(f"[c5 cross-process] first copy {r['kernel_ms'] * 1e3:.1f} us, repeat "
          f"{r['repeat_ms'] * 1e3:.1f} us = {r['bytes'] / (r['repeat_ms'] * 1e-3) / 1e9:.1f} GB/s, "
          f"runs {r['runs']}", flush=True)
    assert r["ok"], r
