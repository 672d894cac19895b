"""The LM head with the argmax fused (Q8 row scales): the streaming kernel at
M = 1 and the wide MFMA kernel at M = 2..8, both with the partials merged
inside the launch by its last workgroup.  Logits, indices and top-2 gaps against the
oracle (MM:645-686 first-maximum rule) at ragged vocabulary sizes (the last
tile partly past N, odd N with fp16 row scales), K = 256..1024, fp16 and fp32
row scales, the tiled Pack4 logits layout, RMSNorm-in at several rows with row
scales far from 1, and a planted tie across workgroups (two identical weight
rows far apart: the lower index wins, with a top-2 gap of zero).
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


def _normwise(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def _weight(ctx, aexq, n, k, seed, sdt):
    from aiimage_amd import synth
    words, scales, codes = synth.q8_weights(n, k, seed, scale_dtype=sdt)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    return w, words, scales, codes


def _check_rows(got_idx, gap, ref):
    srt = np.sort(ref, axis=1)
    ref_gap = srt[:, -1] - srt[:, -2]
    ref_idx = np.argmax(ref, axis=1)
    for r in range(ref.shape[0]):
        if ref_gap[r] >= ARGMAX_TIE:
            assert got_idx[r] == ref_idx[r], (r, got_idx[r], ref_idx[r])
    if gap is not None:
        np.testing.assert_allclose(gap, ref_gap, atol=1e-5)


@pytest.mark.parametrize("m,n,k,sdt", [
    (2, 100000, 768, np.float16),
    (3, 30011, 1024, np.float32),
    (5, 4097, 512, np.float16),
    (8, 65 * 64 + 17, 256, np.float32),
    (7, 151936, 1024, np.float16),
    (1, 30011, 1024, np.float16),
])
def test_lmhead_rows_formats(ctx, aexq, orc, m, n, k, sdt):
    _announce(f"lm head m={m} n={n} k={k} scales={np.dtype(sdt).name}")
    from aiimage_amd import synth
    seed = 0xAE1D0000 + 97 * m + n
    w, words, scales, _ = _weight(ctx, aexq, n, k, seed, sdt)
    x16 = synth.activations(m, k, seed + 1)
    xd = aexq.describe(torch.as_tensor(x16).cuda(), m, k)
    layout = aexq.LAYOUT_PACK4_TILED
    logits = aexq.new_activation(m, n, torch.float32, layout)
    logits.fill_(7.0)
    am = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    gap = torch.zeros(m, dtype=torch.float32, device="cuda")
    ctx.lmhead_argmax(w, xd, aexq.describe(logits, m, n, layout), am, gap)
    torch.cuda.synchronize()
    stride = aexq.storage_elements(layout, m, n)
    got = logits.cpu().numpy().reshape(m, stride)
    sd = orc.SCALE_F16 if sdt == np.float16 else orc.SCALE_F32
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32),
                                 orc.dequant_q8(words, scales, n, k, scale_dtype=sd))
    assert _normwise(got[:, :n], ref) <= 1e-5
    gi = am.cpu().numpy()
    _check_rows(gi, gap.cpu().numpy(), ref)
    # without logits: the same indices
    am2 = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    ctx.lmhead_argmax(w, xd, None, am2)
    torch.cuda.synchronize()
    assert np.array_equal(am2.cpu().numpy(), gi)
    w.release()


@pytest.mark.parametrize("m", [1, 6])
def test_lmhead_tie_across_workgroups(ctx, aexq, orc, m):
    """Rows 1000 and 150000 hold the same codes and scale, scaled so that they
    win every row: the logits tie exactly and the first index is the argmax,
    with a top-2 gap of zero."""
    _announce(f"lm head planted tie m={m}")
    from aiimage_amd import synth
    n, k = 151936, 1024
    words, scales, codes = synth.q8_weights(n, k, 0xAE1D7000 + m)
    x16 = synth.activations(m, k, 0xAE1D7001 + m)
    # the winning row: codes following the sign of the first activation row
    win = np.where(x16[0].astype(np.float32) >= 0, 127, -127).astype(np.int8)
    codes = codes.copy()
    codes[1000] = win
    codes[150000] = win
    scales = scales.copy()
    scales[1000] = scales[150000] = np.float16(0.05)
    words = codes.reshape(-1).view(np.uint32).copy()
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    xd = aexq.describe(torch.as_tensor(x16).cuda(), m, k)
    am = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    gap = torch.full((m,), -1.0, dtype=torch.float32, device="cuda")
    ctx.lmhead_argmax(w, xd, None, am, gap)
    torch.cuda.synchronize()
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32),
                                 orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F16))
    assert int(am[0]) == 1000
    assert float(gap[0]) == 0.0
    assert int(orc.argmax_rows(ref.astype(np.float32))[0]) == 1000
    _check_rows(am.cpu().numpy()[1:], None, ref[1:])
    w.release()


@pytest.mark.parametrize("m", [2, 8])
def test_lmhead_rmsnorm_in_rows(ctx, aexq, orc, m):
    """RMSNorm-in at several rows, with row scales far from
    1 (RMS 1e-5 and 4e4 with gamma up to 2): logits within 1e-3 of the oracle
    of rmsnorm -> fp16 -> Q8 matvec, no NaN, indices off near-ties."""
    _announce(f"lm head rmsnorm-in m={m}")
    from aiimage_amd import synth
    n, k, eps = 50021, 1024, 1e-6
    words, scales, _ = synth.q8_weights(n, k, 0xAE1D8000 + m)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    x = synth.activations(m, k, 0xAE1D8001 + m).astype(np.float32)
    row_scale = np.array([1e-5, 4e4 / 4.0, 1.0, 3e-3, 20.0, 1e-4, 0.5, 7.0][:m], np.float32)
    x16 = (x * row_scale[:, None]).astype(np.float16)
    gamma = (synth.rms_gamma(k, 0xAE1D8002) * 2.0).astype(np.float32)
    gd = torch.as_tensor(gamma).cuda()
    xd = aexq.describe(torch.as_tensor(x16).cuda(), m, k)
    layout = aexq.LAYOUT_PACK4_LINEAR
    logits = aexq.new_activation(m, n, torch.float32, layout)
    am = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    ctx.lmhead_argmax(w, xd, aexq.describe(logits, m, n, layout), am,
                      rmsnorm=True, rms_gamma=gd, rms_eps=eps)
    torch.cuda.synchronize()
    got = logits.cpu().numpy().reshape(m, -1)[:, :n]
    assert np.all(np.isfinite(got))
    xn = orc.rmsnorm(x16.astype(np.float32), eps, gamma).astype(np.float16).astype(np.float32)
    ref = orc.gemm_gpu_semantics(xn, orc.dequant_q8(words, scales, n, k,
                                                    scale_dtype=orc.SCALE_F16))
    for r in range(m):
        assert _normwise(got[r], ref[r]) <= 1e-3, r
    _check_rows(am.cpu().numpy(), None, ref)
    w.release()
