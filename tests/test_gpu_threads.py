"""Concurrent callers: two host threads launch through the library at the same
time, each on its own stream (ctypes releases the GIL, so the library's
calls overlap).  The library keeps the tuning overrides and the launch
records per thread, and the split-KV workspace cache per (device, stream).
Thread A forces the general kernel on a Qwen3-8B S=4096 prefill, which the
shape-based dispatch sends to the ping-pong kernel. Thread B runs that
dispatch on the same shape and, in alternation, a Gemma-3-12B S=1536 launch
that splits its key ranges.  Every launch's records name the kernel its own
thread asked for, and every output equals the single-threaded result bit for
bit.
"""
import threading

import pytest
import torch

from helpers import announce
from kernelfuser_amd import GEMMA3_12B, QWEN3_8B, _lib, launch_attention, make_inputs

pytestmark = pytest.mark.gpu

ROUNDS = 12


def _launch(xs, out, kn):
    return [r["kernel"] for r in launch_attention(xs.reference7, out, causal=True, mode="query", kn=kn,
                                                    norm_style="fp32") if r["kernel"].startswith("attn_")]


def test_two_host_threads_on_two_streams(gpu):
    big = make_inputs(1, 4096, QWEN3_8B, 7171).to(gpu)
    split = make_inputs(1, 1536, GEMMA3_12B, 7272).to(gpu)
    announce("two host threads, two streams: forced general vs by-shape ping-pong and a split launch")
    refs = {}
    for name, xs, kernel in (("general", big, "general"), ("auto", big, "auto"), ("split", split, "auto")):
        out, kn = torch.empty_like(xs.q), torch.empty_like(xs.k)
        with _lib.tuning(attn_kernel=kernel):
            k = _launch(xs, out, kn)
        torch.cuda.synchronize()
        refs[name] = (out, k)
    assert refs["general"][1][0].startswith("attn_fwd_kernel") and refs["auto"][1][0].startswith("attn_pp_kernel")
    assert refs["split"][1][0].startswith("attn_fwd_kernel<256")

    errors, start = [], threading.Barrier(2)

    def worker(jobs, kernel):
        try:
            st = torch.cuda.Stream()
            st.wait_stream(torch.cuda.default_stream())
            outs = []
            with _lib.tuning(attn_kernel=kernel), torch.cuda.stream(st):
                start.wait()
                for i in range(ROUNDS):
                    name, xs = jobs[i % len(jobs)]
                    out, kn = torch.empty_like(xs.q), torch.empty_like(xs.k)
                    k = _launch(xs, out, kn)
                    assert k == refs[name][1], (name, k, refs[name][1])
                    outs.append((name, out))
            st.synchronize()
            for name, out in outs:
                assert torch.equal(out, refs[name][0]), name
        except Exception as e:  # reported by the main thread
            errors.append(repr(e))

    ths = [threading.Thread(target=worker, args=([("general", big)], "general")),
           threading.Thread(target=worker, args=([("auto", big), ("split", split)], "auto"))]
    for t in ths:
        t.start()
    for t in ths:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in ths), "a worker did not finish"
    assert not errors, errors
