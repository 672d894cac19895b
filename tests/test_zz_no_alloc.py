"""aexq_lmhead_argmax_noalloc (the LM head for callers that cannot allocate)
against aexq_lmhead_argmax on the same inputs, through the C ABI: two calls in
a row, the second smaller, each equal to the allocating entry point bit for bit
(argmax and top-2 gap), and the oracle's argmax unless near-tie.  Its first
call on a fresh context can be captured into a HIP graph (nothing grows), and
the replays match.  Sizes the fixed scratch cannot take, and the logits path,
are refused.
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _announce(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def aexq():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from aiimage_amd import aexq as mod
    return mod


def _case(ctx, aexq, orc, n, m, seed):
    from aiimage_amd import synth
    k = 1024
    words, scales, _ = synth.q8_weights(n, k, seed)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    x16 = synth.activations(m, k, seed + 1)
    x = torch.as_tensor(x16).cuda()
    am_ref = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    gap_ref = torch.full((m,), -1.0, dtype=torch.float32, device="cuda")
    ctx.lmhead_argmax(w, aexq.describe(x, m, k), None, am_ref, gap_ref)
    am = torch.full((m,), -2, dtype=torch.int32, device="cuda")
    gap = torch.full((m,), -2.0, dtype=torch.float32, device="cuda")
    ctx.lmhead_argmax_noalloc(w, aexq.describe(x, m, k), am, gap)
    torch.cuda.synchronize()
    assert torch.equal(am, am_ref), (am, am_ref)
    assert torch.equal(gap, gap_ref), (gap, gap_ref)
    deq = orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F16)
    logits = orc.gemm_gpu_semantics(x16.astype(np.float32), deq)
    got = am.cpu().numpy()
    for r in range(m):
        srt = np.sort(logits[r])
        if srt[-1] - srt[-2] >= 1e-3:
            assert got[r] == int(np.argmax(logits[r])), r
    w.release()


def test_noalloc_lmhead_matches_allocating_entry_point(aexq, orc):
    ctx = aexq.Context(0)
    try:
        _announce("noalloc LM head: 151936 x 1024, M = 8, then 20000 x 1024, M = 1")
        _case(ctx, aexq, orc, 151936, 8, 1300)
        _case(ctx, aexq, orc, 20000, 1, 1310)
    finally:
        torch.cuda.synchronize()
        ctx.close()


@pytest.mark.parametrize("m", [1, 8])
def test_noalloc_first_call_under_capture(aexq, m):
    """The entry point allocates nothing: on a fresh context (no scratch grown
    yet) its very first call is made inside HIP graph capture on a side
    stream, where any context allocation is refused.  The capture succeeds,
    and every replay -- with eager work between replays -- gives the argmax and
    gap of the allocating entry point."""
    from aiimage_amd import synth
    n, k = 151936, 1024
    _announce(f"noalloc first call under graph capture, M = {m}")
    ctx = aexq.Context(0)
    try:
        words, scales, _ = synth.q8_weights(n, k, 1330 + m)
        w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
        x = torch.as_tensor(synth.activations(m, k, 1331 + m)).cuda()
        xd = aexq.describe(x, m, k)
        am = torch.full((m,), -2, dtype=torch.int32, device="cuda")
        gap = torch.full((m,), -2.0, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        stream = torch.cuda.Stream()
        ctx.set_stream(stream)
        g = torch.cuda.CUDAGraph()
        try:
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
                ctx.lmhead_argmax_noalloc(w, xd, am, gap)
        finally:
            ctx.set_stream(torch.cuda.current_stream())
        torch.cuda.synchronize()
        am_ref = torch.full((m,), -1, dtype=torch.int32, device="cuda")
        gap_ref = torch.full((m,), -1.0, dtype=torch.float32, device="cuda")
        ctx.lmhead_argmax(w, xd, None, am_ref, gap_ref)
        torch.cuda.synchronize()
        for rep in range(3):
            am.fill_(-2)
            gap.fill_(-2.0)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(am, am_ref), (rep, am, am_ref)
            assert torch.equal(gap, gap_ref), (rep, gap, gap_ref)
            ctx.lmhead_argmax(w, xd, None, am_ref, gap_ref)   # eager work between replays
            torch.cuda.synchronize()
        del g
        w.release()
    finally:
        torch.cuda.synchronize()
        ctx.close()


def test_noalloc_lmhead_refusals(aexq):
    from aiimage_amd import _abi, synth
    ctx = aexq.Context(0)
    try:
        _announce("noalloc LM head refuses the logits pass (K = 1000) and M = 512")
        n, k = 4096, 1000
        words, scales, _ = synth.q8_weights(n, k, 1320)
        w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
        x = torch.as_tensor(synth.activations(2, k, 1321)).cuda()
        am = torch.zeros(2, dtype=torch.int32, device="cuda")
        with pytest.raises(_abi.NotSupportedError):
            ctx.lmhead_argmax_noalloc(w, aexq.describe(x, 2, k), am)
        w.release()
        n, k, m = 151936, 1024, 512
        words, scales, _ = synth.q8_weights(n, k, 1322)
        w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
        x = torch.as_tensor(synth.activations(m, k, 1323)).cuda()
        am = torch.zeros(m, dtype=torch.int32, device="cuda")
        with pytest.raises(_abi.NotSupportedError):
            ctx.lmhead_argmax_noalloc(w, aexq.describe(x, m, k), am)
        w.release()
    finally:
        torch.cuda.synchronize()
        ctx.close()
