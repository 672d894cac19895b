"""From a sharded model archive to a decode step (MAS:50-138 -> GL:60-141 ->
DEC:463-585; MAS = Packages/com.aexis/Samples/AIImageApplicationExample/
Runtime/Scripts/Qwen35MobileAssetSet.cs, DEC = .../Qwen35DecoderSession.cs,
GL = Packages/com.aexis/Runtime/Execution/Layers/AexisGemmLayer.cs).

A two-layer model is written with the oracle's record writers in the
reference's mobile-asset form (tests/archive_model.py): Q4 groups of 16 made
from Q8 rows (the shipping builder's path) or Q8 rows, raw fp32 RMSNorm
records, the tied Q8 embedding, shards under a SHA-256 manifest.  It is loaded
through MobileAssetSet.try_load and the archive walk (decoder.load_assets),
and then:

  * every device weight dequantises bit-exactly to the oracle's reading of its
    record, and the norms equal the raw records;
  * fused and per-operator decode steps match the oracle composition over the
    same records (5e-3 normwise; the greedy token unless a near-tie), layer
    0's appended V row equal in both;
  * a short Generate by graph replay equals the eager fused steps.
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


def _normwise(y, r):
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.max(np.abs(y - r)) / max(np.max(np.abs(r)), 1e-30))


def _same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def _step(sess, tok, pos, fused):
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


@pytest.mark.parametrize("bits", [4, 8])
def test_archive_to_decode(ctx, aexq, orc, tmp_path, bits):
    import archive_model
    from decode_oracle import OracleDecoder, top2_gap

    from aiimage_amd import decoder
    mk = decoder.ModelConfig.reference_q4 if bits == 4 else decoder.ModelConfig.reference_q8
    cfg = mk(layers=2, capacity=128, vocab=8192)
    _announce(f"archive to decode: {cfg.format_name}")
    model = archive_model.write_model(orc, cfg, str(tmp_path), 0xAE1A0000 + bits)
    weights = decoder.load_assets(ctx, str(tmp_path), cfg)

    # the loaded weights are the records, bit for bit
    for l, layer in enumerate(weights.layers):
        W, g_attn, g_mlp = model["layers"][l]
        for name, n, k in cfg.linears():
            info = layer["w"][name].info()
            assert info.bits == bits and info.block == (16 if bits == 4 else k), (l, name)
            assert _same_bits(ctx.dequant(layer["w"][name]).cpu().numpy(), W[name]), (l, name)
        assert np.array_equal(layer["g_attn"], g_attn) and np.array_equal(layer["g_mlp"], g_mlp)
    assert _same_bits(ctx.dequant(weights.lm).cpu().numpy(), model["lm"])
    assert np.array_equal(weights.g_final, model["g_final"])

    sess = decoder.DecodeSession(ctx, cfg, fused=True, weights=weights)
    od = OracleDecoder.from_weights(orc, cfg, model)
    for tok, pos in ((5, 70), (8000, 71)):
        x_p, t_p = _step(sess, tok, pos, fused=False)
        vc = sess.layers[0]["v_cache"].view(cfg.heads_kv, cfg.capacity, cfg.head_dim)
        v_p = vc[:, pos].clone()
        vc[:, pos] = 0
        x_f, t_f = _step(sess, tok, pos, fused=True)
        assert sess.fused.error() == 0
        assert torch.equal(vc[:, pos], v_p), pos
        x_ref, logits = od.step(tok, pos)
        assert _normwise(x_f.cpu().numpy(), x_ref) <= 5e-3, pos
        assert _normwise(x_p.cpu().numpy(), x_ref) <= 5e-3, pos
        if top2_gap(logits) >= ARGMAX_TIE:
            assert t_f == t_p == int(np.argmax(logits)), pos

    # Generate: graph replay equal to eager fused steps
    eager = sess.generate(7, 90, 6)
    g = sess.capture(advance=True)
    assert sess.generate(7, 90, 6, graph=g) == eager
    assert sess.fused.error() == 0
    del g
