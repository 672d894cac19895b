"""GPU checks of the fused decoder-layer step (aexq_decoder_run: every layer
of a decode step in one persistent launch; DecodeCore, DEC:463-585, paths
relative to the reference root, DEC = Packages/com.aexis/Samples/
AIImageApplicationExample/Runtime/Scripts/Qwen35DecoderSession.cs).

  * The final hidden state within 5e-3 (normwise) of the oracle composition
    and of the per-operator step, the greedy token equal unless the oracle's
    top-2 gap is below 1e-3.
  * Layer 0's appended V row equal bit for bit to the per-operator step's (the
    fused linears reproduce aexq_linear's per-row arithmetic exactly).
  * Positions on both sides of attention split boundaries.
  * Graph replays equal to the eager fused step bit for bit; an 8-token
    Generate by graph replay equal to eager fused steps and to the oracle.
  * Config 3 at full size (24 layers, 2048 cached positions).
  * The reference's own layer formats (Q4 with two's-complement nibbles and
    an fp32 scale per 16 codes; Q8 with a scale per row; fp16 scale variants)
    against the oracle and the per-operator step, and through a captured
    Generate loop.
  * No run gives up a bounded wait (the decoder's error word stays 0), and
    shapes the kernel does not take are refused at creation.
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

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


def _step(sess, tok, pos, fused=True):
    """One step of `tok` at `pos` on the fused or the per-operator path:
    (final hidden state, next token)."""
    keep = sess.fused
    if not fused:
        sess.fused = None
    try:
        sess.token.fill_(tok)
        sess.set_position(pos)
        sess.step()
        torch.cuda.synchronize()
    finally:
        sess.fused = keep
    return sess.xa.clone(), int(sess.next_token.item())


def _v_row(sess, layer, pos):
    c = sess.cfg
    return sess.layers[layer]["v_cache"].view(c.heads_kv, c.capacity, c.head_dim)[:, pos].clone()


def test_fused_step_matches_oracle_and_per_operator(ctx, aexq, orc):
    _announce("fused step: 2 layers, 64 positions, position 37")
    from aiimage_amd import decoder
    from decode_oracle import OracleDecoder, top2_gap
    cfg = decoder.ModelConfig(layers=2, capacity=64)
    sess = decoder.DecodeSession(ctx, cfg, fused=True)
    tok, pos = 4242, 37
    x_p, t_p = _step(sess, tok, pos, fused=False)
    v_p = _v_row(sess, 0, pos)
    sess.layers[0]["v_cache"].view(cfg.heads_kv, cfg.capacity, cfg.head_dim)[:, pos] = 0
    x_f, t_f = _step(sess, tok, pos, fused=True)
    assert sess.fused.error() == 0
    assert torch.equal(_v_row(sess, 0, pos), v_p)
    assert torch.isfinite(x_f.float()).all()
    x_ref, logits = OracleDecoder(orc, cfg).step(tok, pos)
    assert normwise(x_f.cpu().numpy(), x_ref) <= 5e-3
    assert normwise(x_f.cpu().numpy(), x_p.cpu().numpy()) <= 5e-3
    if top2_gap(logits) >= ARGMAX_TIE:
        assert t_f == int(np.argmax(logits)) == t_p


def test_fused_positions_across_split_boundaries(ctx, aexq, orc):
    from aiimage_amd import decoder
    from decode_oracle import OracleDecoder, top2_gap
    cfg = decoder.ModelConfig(layers=2, capacity=256)
    sess = decoder.DecodeSession(ctx, cfg, fused=True)
    info = sess.fused.info()
    sp = info["split_positions"]
    _announce(f"fused step positions, capacity 256: {info}")
    assert sp * info["splits"] >= cfg.capacity
    od = OracleDecoder(orc, cfg)
    positions = [0, sp - 1, sp, sp + 1, 2 * sp, cfg.capacity - 1]
    for i, pos in enumerate(positions):
        tok = 1000 + 37 * i
        x_f, t_f = _step(sess, tok, pos)
        x_ref, logits = od.step(tok, pos)
        err = normwise(x_f.cpu().numpy(), x_ref)
        assert err <= 5e-3, (pos, err)
        if top2_gap(logits) >= ARGMAX_TIE:
            assert t_f == int(np.argmax(logits)), pos
    assert sess.fused.error() == 0


def test_fused_graph_replays_match_eager(ctx, aexq):
    _announce("fused step graph replay: 3 layers, 128 positions")
    from aiimage_amd import decoder
    cfg = decoder.ModelConfig(layers=3, capacity=128)
    sess = decoder.DecodeSession(ctx, cfg, fused=True)
    x_eager, tok_eager = _step(sess, 17, 100)
    g = sess.capture()
    for i in range(3):
        sess.xa.zero_()
        sess.next_token.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(sess.xa, x_eager), i
        assert int(sess.next_token.item()) == tok_eager, i
        x2, t2 = _step(sess, 17, 100)      # eager work between replays
        assert torch.equal(x2, x_eager) and t2 == tok_eager, i
    assert sess.fused.error() == 0


def test_fused_generate_graph_matches_eager_and_oracle(ctx, aexq, orc):
    _announce("fused generate 8 tokens: graph vs eager vs oracle")
    from aiimage_amd import decoder
    from decode_oracle import OracleDecoder, top2_gap
    cfg = decoder.ModelConfig(layers=2, capacity=64)
    sess = decoder.DecodeSession(ctx, cfg, fused=True)
    start, pos0, count = 4242, 30, 8
    eager = sess.generate(start, pos0, count)
    x_eager = sess.xa.clone()
    g = sess.capture(advance=True)
    for rep in range(2):
        sess.xa.zero_()
        sess.history.fill_(-1)
        assert sess.generate(start, pos0, count, graph=g) == eager, rep
        assert torch.equal(sess.xa, x_eager), rep
    assert sess.fused.error() == 0
    od = OracleDecoder(orc, cfg)
    tok = start
    for i in range(count):
        x_ref, logits = od.step(tok, pos0 + i)
        want = int(np.argmax(logits))
        if top2_gap(logits) < ARGMAX_TIE:
            break
        assert eager[i] == want, (i, eager, want)
        tok = want
    else:
        assert normwise(x_eager.cpu().numpy(), x_ref) <= 5e-3


def test_fused_config3_full_size(ctx, aexq, orc):
    _announce("fused step, config 3 full size: 24 layers, 2048 positions")
    from aiimage_amd import decoder
    from decode_oracle import OracleDecoder, top2_gap
    cfg = decoder.ModelConfig()
    words, scales, codes = decoder.host_lm_head(cfg)
    rms = scales.astype(np.float64) * np.sqrt(np.mean(codes.astype(np.float64) ** 2, axis=1))
    tok = int(np.nonzero(rms < 1e-5)[0][0])
    pos = cfg.capacity - 1
    sess = decoder.DecodeSession(ctx, cfg, fused=True)
    x_p, t_p = _step(sess, tok, pos, fused=False)
    x_f, t_f = _step(sess, tok, pos)
    assert torch.isfinite(x_f.float()).all()
    g = sess.capture()
    for i in range(2):
        sess.xa.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(sess.xa, x_f), i
        assert int(sess.next_token.item()) == t_f, i
    assert sess.fused.error() == 0
    x_ref, logits = OracleDecoder(orc, cfg).step(tok, pos)
    err = normwise(x_f.cpu().numpy(), x_ref)
    assert err <= 5e-3, err
    assert normwise(x_f.cpu().numpy(), x_p.cpu().numpy()) <= 5e-3
    if top2_gap(logits) >= ARGMAX_TIE:
        assert t_f == int(np.argmax(logits)) == t_p


@pytest.mark.parametrize("workgroups", [0, 256])
def test_fused_fp32_scales_and_grid(ctx, aexq, orc, workgroups):
    """Layer scales in fp32 (the reference archives' dtype) and the 256-workgroup
    grid (half the positions per attention split, a merge slice of 8 dims):
    against the oracle and the per-operator step, the V row bit for bit."""
    from aiimage_amd import decoder
    from decode_oracle import OracleDecoder, top2_gap
    cfg = decoder.ModelConfig(layers=2, capacity=128, scales_f32=True)
    sess = decoder.DecodeSession(ctx, cfg, fused=True, workgroups=workgroups)
    info = sess.fused.info()
    _announce(f"fused step fp32 scales, grid {workgroups}: {info}")
    if workgroups:
        assert info["workgroups"] == workgroups
    tok, pos = 777, 100
    x_p, t_p = _step(sess, tok, pos, fused=False)
    v_p = _v_row(sess, 0, pos)
    sess.layers[0]["v_cache"].view(cfg.heads_kv, cfg.capacity, cfg.head_dim)[:, pos] = 0
    x_f, t_f = _step(sess, tok, pos)
    assert sess.fused.error() == 0
    assert torch.equal(_v_row(sess, 0, pos), v_p)
    x_ref, logits = OracleDecoder(orc, cfg).step(tok, pos)
    assert normwise(x_f.cpu().numpy(), x_ref) <= 5e-3
    assert normwise(x_f.cpu().numpy(), x_p.cpu().numpy()) <= 5e-3
    if top2_gap(logits) >= ARGMAX_TIE:
        assert t_f == int(np.argmax(logits)) == t_p


_FORMATS = {
    # the reference's shipping Q4 archives: two's-complement nibbles, fp32 scale per 16
    "q4_g16_f32": lambda **kw: _cfg().reference_q4(**kw),
    "q4_g16_f16": lambda **kw: _cfg()(group=16, **kw),
    # Q8 layers, one scale per output row
    "q8_row_f32": lambda **kw: _cfg().reference_q8(**kw),
    "q8_row_f16": lambda **kw: _cfg()(layer_bits=8, **kw),
}


def _cfg():
    from aiimage_amd import decoder
    return decoder.ModelConfig


@pytest.mark.parametrize("fmt", sorted(_FORMATS))
def test_fused_reference_formats(ctx, aexq, orc, fmt):
    """The fused step on the reference's own layer formats: against the oracle
    composition and the per-operator step (5e-3), layer 0's appended V row
    equal to the per-operator step's bit for bit (the same per-format
    arithmetic as aexq_linear), the greedy token unless a near-tie, at a
    position past an attention split boundary."""
    from aiimage_amd import decoder
    from decode_oracle import OracleDecoder, top2_gap
    cfg = _FORMATS[fmt](layers=2, capacity=192, vocab=8192)
    assert cfg.format_name == fmt
    sess = decoder.DecodeSession(ctx, cfg, fused=True)
    _announce(f"fused step {fmt}: {sess.fused.info()}")
    od = OracleDecoder(orc, cfg)
    for tok, pos in ((4321, 150), (17, 151)):
        x_p, t_p = _step(sess, tok, pos, fused=False)
        v_p = _v_row(sess, 0, pos)
        sess.layers[0]["v_cache"].view(cfg.heads_kv, cfg.capacity, cfg.head_dim)[:, pos] = 0
        x_f, t_f = _step(sess, tok, pos)
        assert sess.fused.error() == 0
        assert torch.equal(_v_row(sess, 0, pos), v_p), (fmt, pos)
        x_ref, logits = od.step(tok, pos)
        assert normwise(x_f.cpu().numpy(), x_ref) <= 5e-3, fmt
        assert normwise(x_f.cpu().numpy(), x_p.cpu().numpy()) <= 5e-3, fmt
        if top2_gap(logits) >= ARGMAX_TIE:
            assert t_f == int(np.argmax(logits)) == t_p, (fmt, pos)


def test_fused_reference_q4_graph_generate(ctx, aexq, orc):
    """The reference's Q4 format through the captured Generate loop: eight
    tokens by graph replay equal to eager fused steps and to the oracle."""
    from aiimage_amd import decoder
    from decode_oracle import OracleDecoder, top2_gap
    cfg = decoder.ModelConfig.reference_q4(layers=2, capacity=96, vocab=4096)
    sess = decoder.DecodeSession(ctx, cfg, fused=True)
    _announce("fused generate, reference Q4 format")
    start, pos0, count = 99, 60, 8
    eager = sess.generate(start, pos0, count)
    g = sess.capture(advance=True)
    for rep in range(2):
        assert sess.generate(start, pos0, count, graph=g) == eager, rep
    od = OracleDecoder(orc, cfg)
    tok = start
    for i in range(count):
        _, logits = od.step(tok, pos0 + i)
        if top2_gap(logits) < ARGMAX_TIE:
            break
        assert eager[i] == int(np.argmax(logits)), i
        tok = eager[i]
    del g


def test_fused_rejects_shapes_it_does_not_take(ctx, aexq):
    _announce("fused step rejections")
    from aiimage_amd import decoder
    cfg = decoder.ModelConfig(layers=1, capacity=64)
    sess = decoder.DecodeSession(ctx, cfg)
    L = sess.layers[0]
    layer = dict(L["w"], attn_norm=L["g_attn"], mlp_norm=L["g_mlp"], k_cache=L["k_cache"],
                 v_cache=L["v_cache"])
    args = dict(heads_q=cfg.heads_q, heads_kv=cfg.heads_kv, head_dim=cfg.head_dim,
                capacity=cfg.capacity, rms_eps=cfg.eps, attn_scale=sess.scale,
                rope_cos=sess.cos, rope_sin=sess.sin)
    d = ctx.decoder([layer], sess.embed, **args)       # accepted as given
    d.close()
    bad = dict(layer, q_proj=L["w"]["k_proj"])          # wrong shape
    with pytest.raises(aexq.InvalidOperationError):
        ctx.decoder([bad], sess.embed, **args)
    bad = dict(layer, o_proj=sess.lm)                   # a Q8 weight among Q4 ones
    with pytest.raises((aexq.NotSupportedError, aexq.InvalidOperationError)):
        ctx.decoder([bad], sess.embed, **args)
    # one layer in another format than layer 0's
    cfg16 = decoder.ModelConfig.reference_q4(layers=1, capacity=64)
    s16 = decoder.DecodeSession(ctx, cfg16)
    L16 = s16.layers[0]
    mixed = dict(L16["w"], attn_norm=L16["g_attn"], mlp_norm=L16["g_mlp"],
                 k_cache=L16["k_cache"], v_cache=L16["v_cache"])
    with pytest.raises(aexq.NotSupportedError, match="one unstacked format"):
        ctx.decoder([layer, mixed], sess.embed, **args)
    d = ctx.decoder([mixed, mixed], sess.embed, **args)  # all group 16: accepted
    d.close()
    del s16
    with pytest.raises(aexq.NotSupportedError):          # head_dim other than 128
        ctx.decoder([layer], sess.embed, **dict(args, head_dim=64))
    with pytest.raises(aexq.NotSupportedError):          # cache beyond the split budget
        ctx.decoder([layer], sess.embed, **dict(args, capacity=1 << 16))
    with pytest.raises(aexq.NotSupportedError, match="64"):  # more layers than the LDS table holds
        ctx.decoder([layer] * 65, sess.embed, **args)
    d = ctx.decoder([layer] * 64, sess.embed, **args)  # the largest table is accepted
    d.close()
