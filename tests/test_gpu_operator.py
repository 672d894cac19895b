"""GPU checks of the operator mirror's execute path, the tied-weight alias and
the context's scratch growth around a captured graph.

  * HipGemmLayer: LoadLayer (AexisGemmLayer.cs:15-162) then the execute path
    (GL:471-601: output storage chosen by GL:515-525, the Gemm dispatched with
    the layer's alpha / beta / C) for q_proj at M = 1 (Pack4-linear output) and
    for the 151,936-row LM head (tiled output: beta*C + alpha*sum), against the
    float64 oracle.  GL = Packages/com.aexis/Runtime/Execution/Layers/
    AexisGemmLayer.cs, relative to the reference root.
  * The tied embedding / LM head (GL:91-111, Qwen35SharedTokenEmbeddingWeights
    EMB:95-120): a non-owning alias drives the embedding gather and the LM head;
    releasing it leaves the owner's device copy intact.
  * A graph captured before a call that grows the context's scratch replays to
    the same result afterwards (replaced scratch is retired, not freed), and
    growth while the stream is capturing is refused.
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _announce(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def aexq():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from aiimage_amd import aexq as mod
    return mod


@pytest.fixture(scope="module")
def ctx(aexq):
    c = aexq.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def normwise(y, r):
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.max(np.abs(y - r)) / max(np.max(np.abs(r)), 1e-30))


def test_gemm_layer_q_proj_forward(ctx, aexq, orc):
    _announce("HipGemmLayer q_proj M=1")
    from aiimage_amd import synth
    n, k = 2048, 1024
    words, scales, _ = synth.q4_weights(n, k, 1200, group=32, code=synth.NIBBLE_OFFSET8)
    qt = aexq.QuantizedTensor(n * k, 32, words, scales, bits=4, nibble_code=synth.NIBBLE_OFFSET8)
    bias = synth.activations(1, n, 1201)[0].astype(np.float32)
    layer = aexq.HipGemmLayer(ctx, "q_proj").load_layer(
        {0: 0.5, 1: 2.0, 3: 1, 5: 1, 6: 1, 8: n, 9: k, 10: 4}, qt, bias=bias)
    x16 = synth.activations(1, k, 1202)
    y, layout = layer.forward(torch.as_tensor(x16).cuda(), 1)
    torch.cuda.synchronize()
    assert layout == aexq.LAYOUT_PACK4_LINEAR
    wf = orc.dequant_q4(words, scales, n, k, 32, synth.NIBBLE_OFFSET8, orc.SCALE_F16)
    # Pack4-linear output: alpha * (beta * C + sum) (MM:1054-1057, 1101)
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), wf, alpha=0.5, beta=2.0, c=bias,
                                 broadcast_c=4)[0]
    assert normwise(y.cpu().numpy()[:n], ref) <= TOL


def test_gemm_layer_lm_head_forward_tiled(ctx, aexq, orc):
    _announce("HipGemmLayer LM head 151936 rows, tiled output")
    from aiimage_amd import synth
    n, k = synth.VOCAB, 1024
    words, scales, _ = synth.q8_weights(n, k, 1210)
    qt = aexq.QuantizedTensor(n * k, k, words, scales, bits=8)
    bias = np.full(n, 0.25, np.float32)
    layer = aexq.HipGemmLayer(ctx, "lm_head").load_layer(
        {0: 2.0, 1: 0.5, 3: 1, 5: 1, 6: 1, 8: n, 9: k, 10: 4}, qt, bias=bias)
    x16 = synth.activations(1, k, 1211)
    y, layout = layer.forward(torch.as_tensor(x16).cuda(), 1, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert layout == aexq.LAYOUT_PACK4_TILED
    wf = orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F16)
    # tiled output: beta * C + alpha * sum (MM:2301)
    ref = 0.5 * 0.25 + 2.0 * orc.gemm_gpu_semantics(x16.astype(np.float32), wf)[0]
    got = y.cpu().numpy()
    assert got.size >= n
    assert normwise(got[:n], ref) <= 1e-5


def test_tied_alias_embedding_and_lm_head(ctx, aexq, orc):
    _announce("tied alias: embedding + LM head, alias released before the owner")
    from aiimage_amd import synth
    n, k = 50000, 1024
    words, scales, _ = synth.q8_weights(n, k, 1220)
    owner = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    alias = owner.alias()
    inf_o, inf_a = owner.info(), alias.info()
    assert (inf_a.n, inf_a.k, inf_a.bits, inf_a.code_bytes) == (inf_o.n, inf_o.k, inf_o.bits,
                                                                inf_o.code_bytes)
    deq = orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F16)
    toks = np.array([0, 1, 31337, n - 1], np.int32)
    emb = torch.zeros(len(toks) * k, dtype=torch.float16, device="cuda")
    ctx.embed_q8(alias, torch.as_tensor(toks).cuda(), emb)
    x16 = synth.activations(1, k, 1221)
    am_alias = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx.lmhead_argmax(alias, aexq.describe(torch.as_tensor(x16).cuda(), 1, k), None, am_alias)
    torch.cuda.synchronize()
    assert np.array_equal(emb.cpu().numpy().reshape(len(toks), k), deq[toks].astype(np.float16))
    logits = orc.gemm_gpu_semantics(x16.astype(np.float32), deq)[0]
    srt = np.sort(logits)
    if srt[-1] - srt[-2] >= 1e-3:
        assert int(am_alias.item()) == int(np.argmax(logits))
    alias.release()
    # the owner's copy is untouched by the alias's release
    am_owner = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx.lmhead_argmax(owner, aexq.describe(torch.as_tensor(x16).cuda(), 1, k), None, am_owner)
    emb2 = torch.zeros_like(emb)
    ctx.embed_q8(owner, torch.as_tensor(toks).cuda(), emb2)
    torch.cuda.synchronize()
    assert int(am_owner.item()) == int(am_alias.item())
    assert torch.equal(emb, emb2)
    owner.release()


# the refused capture below launches nothing, so torch warns that its graph is empty
@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_graph_replays_after_scratch_growth(ctx, aexq, orc, monkeypatch):
    _announce("graph replay after the context's scratch grows; growth under capture refused")
    from aiimage_amd import _abi, synth
    c2 = aexq.Context(0)
    try:
        n, k = 40000, 1024
        words, scales, _ = synth.q8_weights(n, k, 1230)
        w = c2.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
        x1 = torch.as_tensor(synth.activations(1, k, 1231)).cuda()
        am1 = torch.zeros(1, dtype=torch.int32, device="cuda")
        stream = torch.cuda.Stream()
        c2.set_stream(stream)
        with torch.cuda.stream(stream):
            c2.lmhead_argmax(w, aexq.describe(x1, 1, k), None, am1)   # sizes the scratch
        stream.synchronize()
        want = int(am1.item())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
            c2.lmhead_argmax(w, aexq.describe(x1, 1, k), None, am1)
        # an argmax over [64][151936] logits at 32 workgroups per CU takes 149
        # partials per row, 4768 per launch of 32 rows: more than the M = 1 LM
        # head's one per workgroup (1024), so the partial buffer grows, and the
        # captured graph still names the old one
        rows, width = 64, 151936
        lg = torch.randn(rows, width, device="cuda", dtype=torch.float32)
        am64 = torch.zeros(rows, dtype=torch.int32, device="cuda")
        monkeypatch.setenv("AEXQ_ARGMAX_WG_PER_CU", "32")
        with torch.cuda.stream(stream):
            c2.argmax(aexq.describe(lg.reshape(-1), rows, width), am64)
        stream.synchronize()
        monkeypatch.delenv("AEXQ_ARGMAX_WG_PER_CU")
        assert np.array_equal(am64.cpu().numpy(), np.argmax(lg.cpu().numpy(), axis=1))
        for i in range(3):
            am1.fill_(-1)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert int(am1.item()) == want, i
        # growth while capturing is refused before anything is launched: the
        # first RMSNorm-in pre-pass of this context needs its row scratch
        wq, sq, _ = synth.q4_weights(1024, k, 1233, group=32, code=synth.NIBBLE_OFFSET8)
        w4 = c2.weight(aexq.QuantizedTensor(1024 * k, 32, wq, sq, bits=4,
                                            nibble_code=synth.NIBBLE_OFFSET8), 1024, k)
        xm = torch.as_tensor(synth.activations(64, k, 1234)).cuda()
        ym = torch.zeros(64 * 1024, dtype=torch.float16, device="cuda")
        kw = dict(rmsnorm=True, rms_eps=1e-6)
        assert "rms_prepass=1" in c2.plan_check(w4, aexq.describe(xm, 64, k),
                                                aexq.describe(ym, 64, 1024), **kw)
        g2 = torch.cuda.CUDAGraph()
        with pytest.raises(_abi.NotSupportedError):
            with torch.cuda.graph(g2, stream=stream, capture_error_mode="thread_local"):
                c2.linear(w4, aexq.describe(xm, 64, k), aexq.describe(ym, 64, 1024), **kw)
        torch.cuda.synchronize()
        # outside a capture the same call grows the scratch and runs
        with torch.cuda.stream(stream):
            c2.linear(w4, aexq.describe(xm, 64, k), aexq.describe(ym, 64, 1024), **kw)
        stream.synchronize()
        wf = orc.dequant_q4(wq, sq, 1024, k, 32, synth.NIBBLE_OFFSET8, orc.SCALE_F16)
        xn = orc.rmsnorm(xm.cpu().numpy().astype(np.float32), 1e-6).astype(np.float16)
        ref = orc.gemm_gpu_semantics(xn.astype(np.float32), wf)
        assert normwise(ym.cpu().numpy().reshape(64, 1024), ref) <= TOL
    finally:
        torch.cuda.synchronize()
        c2.close()


def test_weight_released_after_its_context(aexq):
    """A weight may outlive the context that made it: its release frees the
    device copy without touching the destroyed context (no HIP error is left
    behind for the next launch to report)."""
    _announce("weight released after its context")
    from aiimage_amd import synth
    c3 = aexq.Context(0)
    n, k = 512, 1024
    words, scales, _ = synth.q8_weights(n, k, 1240)
    w = c3.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    a = w.alias()
    c3.close()
    a.release()
    w.release()
    t = torch.zeros(1024, device="cuda") + 1.0
    torch.cuda.synchronize()
    assert float(t.sum().item()) == 1024.0
