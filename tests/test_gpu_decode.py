"""GPU parity of the decode-step operators and of a full decode step (benchmark
config 3) against compositions of the CPU oracle's functions.

The oracle rounds to fp16 at the same points the device stores fp16 (each
launch's output), so the comparison isolates accumulation order: bars are
normwise max|y - r| / max|r| <= 1e-3 per operator and <= 5e-3 for the hidden
state after two whole layers; greedy argmax equal unless the oracle's top-2
gap is below 1e-3.
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL = 1e-3
ARGMAX_TIE = 1e-3


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


def f16(a):
    return np.asarray(a, np.float64).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("hq,hkv,length,cap", [
    (16, 4, 41, 64), (16, 4, 2048, 2048), (8, 8, 5, 16), (16, 2, 97, 128),
    # merges over several chunks of split rows, more than one row of statistics per thread
    (16, 4, 8192, 8192), (16, 2, 4100, 4160), (8, 8, 9000, 9000)])
def test_rope_kv_append_attention(ctx, aexq, orc, hq, hkv, length, cap, fused):
    """RoPE + KV append + attention, as two launches or fused in one; the
    fused kernel rotates q in LDS and leaves the caller's q as it was."""
    _announce(f"rope+attention hq={hq} hkv={hkv} len={length} fused={fused}")
    d = 128
    pos = length - 1
    rng = np.random.default_rng(length + hq)
    q = rng.standard_normal((hq, d)).astype(np.float16)
    k = rng.standard_normal((hkv, d)).astype(np.float16)
    v = rng.standard_normal((hkv, d)).astype(np.float16)
    kc = rng.standard_normal((hkv, cap, d)).astype(np.float16)
    vc = rng.standard_normal((hkv, cap, d)).astype(np.float16)
    cos_t, sin_t = orc.rope_table(pos, d, 1e6)
    tq, tk, tv = (torch.as_tensor(a).cuda().reshape(-1) for a in (q, k, v))
    tkc, tvc = torch.as_tensor(kc).cuda().reshape(-1), torch.as_tensor(vc).cuda().reshape(-1)
    tcos, tsin = torch.as_tensor(cos_t).cuda(), torch.as_tensor(sin_t).cuda()
    out = torch.zeros(hq * d, dtype=torch.float16, device="cuda")
    scale = 1.0 / np.sqrt(d)
    if fused:
        ctx.attention_decode_rope(tq, tk, tv, tkc, tvc, hq, hkv, d, cap, length, tcos, tsin,
                                  scale, out)
    else:
        ctx.rope_kv_append(tq, tk, tv, tkc, tvc, hq, hkv, d, cap, pos, tcos, tsin)
        ctx.attention_decode(tq, tkc, tvc, hq, hkv, d, cap, length, scale, out)
    torch.cuda.synchronize()
    # oracle: rotate, round to the fp16 the device stores, append, attend
    q_r = f16(orc.rope_rotate_half(q.astype(np.float32), cos_t, sin_t))
    k_r = f16(orc.rope_rotate_half(k.astype(np.float32), cos_t, sin_t))
    if fused:
        assert np.array_equal(tq.cpu().numpy().reshape(hq, d), q)
    else:
        assert normwise(tq.cpu().numpy().reshape(hq, d), q_r) <= 1e-3
    kc_ref = kc.astype(np.float32).copy()
    vc_ref = vc.astype(np.float32).copy()
    kc_ref[:, pos] = k_r
    vc_ref[:, pos] = v.astype(np.float32)
    got_kc = tkc.cpu().numpy().reshape(hkv, cap, d).astype(np.float32)
    assert normwise(got_kc[:, pos], k_r) <= 1e-3
    assert np.array_equal(tvc.cpu().numpy().reshape(hkv, cap, d)[:, pos], v)
    # rows other than `pos` untouched
    others = [p for p in range(cap) if p != pos]
    assert np.array_equal(got_kc[:, others], kc.astype(np.float32)[:, others])
    ref = orc.sdpa_decode(q_r, kc_ref[:, :length], vc_ref[:, :length], scale)
    assert normwise(out.cpu().numpy().reshape(hq, d), ref) <= TOL


def test_attention_rejects_unsupported(ctx, aexq):
    _announce("attention rejects")
    from aiimage_amd import _abi
    t = torch.zeros(16 * 128, dtype=torch.float16, device="cuda")
    c = torch.zeros(4 * 8 * 128, dtype=torch.float16, device="cuda")
    with pytest.raises(_abi.ArgumentError):
        ctx.attention_decode(t, c, c, 16, 4, 128, 8, 9, 0.1, t)      # length > capacity
    with pytest.raises(_abi.NotSupportedError):
        ctx.attention_decode(t, c, c, 16, 4, 64, 8, 4, 0.1, t)       # head_dim 64
    with pytest.raises(_abi.ArgumentError):
        ctx.rope_kv_append(t, t, t, c, c, 16, 4, 128, 8, 8, t, t)    # position == capacity


def test_rmsnorm_and_embedding(ctx, aexq, orc):
    _announce("rmsnorm + embedding")
    from aiimage_amd import synth
    n, k = 1000, 1024
    words, scales, codes = synth.q8_weights(n, k, 31)
    table = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    toks = np.array([0, 7, 999, 512], np.int32)
    out = torch.zeros(len(toks) * k, dtype=torch.float16, device="cuda")
    ctx.embed_q8(table, torch.as_tensor(toks).cuda(), out)
    torch.cuda.synchronize()
    deq = orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F16)
    assert np.array_equal(out.cpu().numpy().reshape(len(toks), k), deq[toks].astype(np.float16))
    x = synth.activations(3, k, 32)
    gamma = synth.rms_gamma(k, 33)
    y = torch.zeros(3 * k, dtype=torch.float16, device="cuda")
    ctx.rmsnorm(aexq.describe(torch.as_tensor(x).cuda(), 3, k), aexq.describe(y, 3, k),
                torch.as_tensor(gamma).cuda(), 1e-6)
    torch.cuda.synchronize()
    ref = orc.rmsnorm(x.astype(np.float32), 1e-6, gamma)
    assert normwise(y.cpu().numpy().reshape(3, k), ref) <= TOL


def _oracle_step(orc, cfg, tok, pos, caches):
    """The decode step composed from oracle functions, rounding to fp16 where the
    device stores fp16.  caches: per layer (k [hkv][cap][d], v) float32, updated."""
    from aiimage_amd import decoder, synth
    lw, ls, _ = decoder.host_lm_head(cfg)
    lm = orc.dequant_q8(lw, ls, cfg.vocab, cfg.hidden, scale_dtype=orc.SCALE_F16)
    x = f16(lm[tok])
    cos_t, sin_t = orc.rope_table(pos, cfg.head_dim, cfg.rope_base)
    scale = np.float32(1.0 / np.sqrt(cfg.head_dim))
    for l in range(cfg.layers):
        ws, g_attn, g_mlp = decoder.host_weights(cfg, l)
        W = {}
        for name, n, k in cfg.linears():
            words, scales, _ = ws[name]
            W[name] = orc.dequant_q4(words, scales, n, k, cfg.group, synth.NIBBLE_OFFSET8,
                                     orc.SCALE_F16)
        xn = f16(orc.rmsnorm(x[None, :], cfg.eps, g_attn))
        q = f16(orc.gemm_gpu_semantics(xn, W["q_proj"]))[0]
        k = f16(orc.gemm_gpu_semantics(xn, W["k_proj"]))[0]
        v = f16(orc.gemm_gpu_semantics(xn, W["v_proj"]))[0]
        q = f16(orc.rope_rotate_half(q.reshape(cfg.heads_q, cfg.head_dim), cos_t, sin_t))
        k = f16(orc.rope_rotate_half(k.reshape(cfg.heads_kv, cfg.head_dim), cos_t, sin_t))
        kc, vc = caches[l]
        kc[:, pos] = k
        vc[:, pos] = v.reshape(cfg.heads_kv, cfg.head_dim)
        att = f16(orc.sdpa_decode(q, kc[:, :pos + 1], vc[:, :pos + 1], scale)).reshape(1, -1)
        xb = f16(orc.gemm_gpu_semantics(att, W["o_proj"])[0] + x)
        xn2 = f16(orc.rmsnorm(xb[None, :], cfg.eps, g_mlp))
        g = orc.gemm_gpu_semantics(xn2, W["gate_proj"])[0]
        u = orc.gemm_gpu_semantics(xn2, W["up_proj"])[0]
        h = f16(orc.swiglu(g.astype(np.float32), u.astype(np.float32)))[None, :]
        x = f16(orc.gemm_gpu_semantics(h, W["down_proj"])[0] + xb)
    xf = f16(orc.rmsnorm(x[None, :], cfg.eps, decoder.host_final_gamma(cfg)))
    logits = orc.gemm_gpu_semantics(xf, lm)[0]
    return x, logits


def test_decode_step_two_layers(ctx, aexq, orc):
    """Two full-width layers (config 3 shapes), 64-position cache, position 37."""
    _announce("decode step 2 layers")
    from aiimage_amd import decoder
    cfg = decoder.ModelConfig(layers=2, capacity=64)
    sess = decoder.DecodeSession(ctx, cfg)
    tok, pos = 4242, 37
    sess.token.fill_(tok)
    sess.set_position(pos)
    caches = []
    for l in range(cfg.layers):
        kc, vc = decoder.host_kv_cache(cfg, l)
        caches.append((kc.astype(np.float32), vc.astype(np.float32)))
    sess.step()
    torch.cuda.synchronize()
    x_ref, logits = _oracle_step(orc, cfg, tok, pos, caches)
    x_got = sess.xa.cpu().numpy().astype(np.float64)
    assert normwise(x_got, x_ref) <= 5e-3, normwise(x_got, x_ref)
    srt = np.sort(logits)
    ref_idx = int(np.argmax(logits))
    if srt[-1] - srt[-2] >= ARGMAX_TIE:
        assert int(sess.next_token.item()) == ref_idx
    # the appended cache rows
    for l in range(cfg.layers):
        kc = sess.layers[l]["k_cache"].cpu().numpy().reshape(cfg.heads_kv, cfg.capacity, cfg.head_dim)
        assert normwise(kc[:, pos], caches[l][0][:, pos]) <= 5e-3


def test_decode_graph_replays_match_eager(ctx, aexq):
    """A captured decode step replays to the eager result, with eager work and
    synchronisations between the replays."""
    _announce("decode graph replay")
    from aiimage_amd import decoder
    cfg = decoder.ModelConfig(layers=3, capacity=128)
    sess = decoder.DecodeSession(ctx, cfg)
    sess.token.fill_(17)
    sess.set_position(100)
    sess.step()
    torch.cuda.synchronize()
    x_eager = sess.xa.clone()
    tok_eager = int(sess.next_token.item())
    g = sess.capture()
    for i in range(3):
        sess.xa.zero_()
        sess.next_token.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(sess.xa, x_eager), i
        assert int(sess.next_token.item()) == tok_eager, i
        sess.step()            # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(sess.xa, x_eager), i
