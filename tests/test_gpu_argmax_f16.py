"""The fp16-logit argmax: the reference's LM head writes its logits to an
ARGBHalf texture unless a reshape promotes it (GL:383-396, GL:1453-1466) and
ArgMaxPack4LinearMat reads those fp16 values (DEC:792, MM:645-686), so its
greedy token is the first maximum of fp16-rounded logits.  AEXQ_EPI_ARGMAX_F16
(or an fp16 logits tensor) selects that comparison.

  * A planted pair of rows whose logits differ in fp32 but round to the same
    fp16 value: the fp16 mode picks the lower index with a top-2 gap of 0, the
    fp32 mode the larger logit; at M = 1 (streaming kernel, in-launch merge),
    M = 4 (wide MFMA kernel, in-launch merge) and through the logits-then-argmax
    path (K not a multiple of 16); with fp16 and fp32 logits tensors.
  * The full 151,936-row head at M = 1 and 8 against the first maximum of the
    oracle's logits rounded to fp16, allowing only a logit within the fp32
    accumulation tolerance of an fp16 rounding boundary to round either way.
  * aexq_argmax over an fp16 logits tensor with planted ties.
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


@pytest.fixture(scope="module")
def ctx(aexq):
    c = aexq.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def _planted(orc, n, k, m, seed, lo=1000, hi=150000):
    """Q8 weights with fp32 row scales where rows `lo` and `hi` carry the same
    codes and scales chosen so that, for activation row 0, logit[hi] exceeds
    logit[lo] by 0.15 fp16 ulp and both round to the same fp16 value 5.0."""
    from aiimage_amd import synth
    words, scales, codes = synth.q8_weights(n, k, seed, scale_dtype=np.float32)
    x16 = synth.activations(m, k, seed + 1)
    x0 = x16[0].astype(np.float64)
    win = np.where(x0 >= 0, 127, -127).astype(np.int8)
    codes = codes.copy()
    codes[lo] = win
    codes[hi] = win
    d = float(np.dot(win.astype(np.float64), x0))
    ulp = 2.0 ** -8                       # fp16 spacing in [4, 8)
    scales = scales.copy()
    scales[lo] = np.float32((5.0 + 0.25 * ulp) / d)
    scales[hi] = np.float32((5.0 + 0.40 * ulp) / d)
    words = codes.reshape(-1).view(np.uint32).copy()
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32),
                                 orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F32))
    # the construction holds for the oracle's logits (and with margin for the GPU's)
    assert ref[0, hi] - ref[0, lo] > 0.1 * ulp
    assert _f16(ref[0, lo]) == _f16(ref[0, hi]) == 5.0
    assert ref[0].max() == ref[0, hi] and np.sort(ref[0])[-3] < 4.0
    return words, scales, x16, ref


@pytest.mark.parametrize("m,k", [(1, 1024), (4, 1024), (1, 1000), (3, 1000)])
def test_planted_pair_equal_in_fp16(ctx, aexq, orc, m, k):
    n, lo, hi = 151936, 1000, 150000
    _announce(f"argmax fp16 planted pair m={m} k={k}")
    words, scales, x16, ref = _planted(orc, n, k, m, 0xAE1F1600 + 10 * m + k)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    xd = aexq.describe(torch.as_tensor(x16).cuda(), m, k)

    def run(f16_mode, logits_dtype=None):
        am = torch.full((m,), -1, dtype=torch.int32, device="cuda")
        gap = torch.full((m,), -1.0, dtype=torch.float32, device="cuda")
        lg, lgd = None, None
        if logits_dtype is not None:
            lg = aexq.new_activation(m, n, logits_dtype, aexq.LAYOUT_PACK4_TILED)
            lgd = aexq.describe(lg, m, n, aexq.LAYOUT_PACK4_TILED)
        ctx.lmhead_argmax(w, xd, lgd, am, gap, argmax_f16=f16_mode)
        torch.cuda.synchronize()
        return am.cpu().numpy(), gap.cpu().numpy(), lg

    # fp32 comparison: the larger logit wins, by its fp32 margin
    am, gap, _ = run(False)
    assert am[0] == hi
    np.testing.assert_allclose(gap[0], ref[0, hi] - ref[0, lo], rtol=0.05)
    # fp16 comparison: equal after rounding, the first index wins, the gap is 0
    for f16_mode, ldt in ((True, None), (True, torch.float32), (False, torch.float16),
                          (True, torch.float16)):
        am, gap, lg = run(f16_mode, ldt)
        assert am[0] == lo, (f16_mode, ldt, am[0])
        assert gap[0] == 0.0, (f16_mode, ldt, gap[0])
        if lg is not None:
            stride = aexq.storage_elements(aexq.LAYOUT_PACK4_TILED, m, n)
            row = lg.float().cpu().numpy().reshape(m, stride)[0, :n]
            if ldt == torch.float16:
                assert row[lo] == row[hi] == 5.0
            else:
                # fp32 logits keep the unrounded values
                assert row[hi] > row[lo]
                assert abs(row[hi] - ref[0, hi]) < 1e-5 and abs(row[lo] - ref[0, lo]) < 1e-5
    w.release()


def _check_fp16_first_max(got_idx, got_gap, ref, tol_rel=1e-5):
    """got_idx must be a first maximum of some rounding of ref to fp16 in which
    every logit within tol of a rounding boundary may round either way."""
    for r in range(ref.shape[0]):
        row = ref[r].astype(np.float64)
        tol = tol_rel * np.abs(row).max()
        lo16 = _f16(row - tol)
        hi16 = _f16(row + tol)
        g = int(got_idx[r])
        # g can be a maximum: no logit is surely above its highest rounding
        assert hi16[g] >= lo16.max(), (r, g)
        # no earlier index surely reaches g's value
        assert not np.any(lo16[:g] >= hi16[g]), (r, g)
        r16 = _f16(row)
        best = r16.max()
        first = int(np.argmax(r16 == best))
        if np.array_equal(lo16, hi16):
            assert g == first, (r, g, first)
            srt = np.sort(r16)
            assert got_gap[r] == np.float32(srt[-1] - srt[-2]), (r, got_gap[r])
        else:
            assert 0.0 <= got_gap[r] <= 2.0 * (float(hi16.max()) - float(np.sort(lo16)[-2])) + 1e-3


@pytest.mark.parametrize("m", [1, 8])
def test_full_vocab_against_rounded_oracle(ctx, aexq, orc, m):
    """The synthetic head at full size: its top-2 gaps exceed an fp16 step, so
    the index equals the fp32 one and the gap becomes the difference of the
    two fp16-rounded logits, exactly (the planted pair above covers the case
    where the rounding decides)."""
    from aiimage_amd import synth
    n, k = 151936, 1024
    _announce(f"argmax fp16 full vocabulary m={m}")
    words, scales, _ = synth.q8_weights(n, k, 0xAE1F1700 + m)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    x16 = synth.activations(m, k, 0xAE1F1701 + m)
    xd = aexq.describe(torch.as_tensor(x16).cuda(), m, k)
    am = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    gap = torch.full((m,), -1.0, dtype=torch.float32, device="cuda")
    ctx.lmhead_argmax(w, xd, None, am, gap, argmax_f16=True)
    torch.cuda.synchronize()
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32),
                                 orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F16))
    _check_fp16_first_max(am.cpu().numpy(), gap.cpu().numpy(), ref)
    # the same rule through the final RMSNorm fused in front
    gamma = synth.rms_gamma(k, 0xAE1F1702)
    gd = torch.as_tensor(gamma).cuda()
    am2 = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    gap2 = torch.full((m,), -1.0, dtype=torch.float32, device="cuda")
    ctx.lmhead_argmax(w, xd, None, am2, gap2, rmsnorm=True, rms_gamma=gd, rms_eps=1e-6,
                      argmax_f16=True)
    torch.cuda.synchronize()
    xn = orc.rmsnorm(x16.astype(np.float32), 1e-6, gamma).astype(np.float16).astype(np.float32)
    ref2 = orc.gemm_gpu_semantics(xn, orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F16))
    _check_fp16_first_max(am2.cpu().numpy(), gap2.cpu().numpy(), ref2)
    w.release()


@pytest.mark.parametrize("m,n", [(1, 151936), (5, 4099)])
def test_argmax_over_fp16_logits(ctx, aexq, orc, m, n):
    """aexq_argmax reads fp16 logits: the first maximum (planted ties at the
    top, far apart), the top-2 gap of those values, and NaN-free random rows."""
    _announce(f"aexq_argmax fp16 logits m={m} n={n}")
    rng = np.random.default_rng(0xAE1F18 + m)
    lg = rng.standard_normal((m, n)).astype(np.float16)
    for r in range(m):
        a, b = sorted(rng.choice(n, 2, replace=False))
        lg[r, a] = lg[r, b] = np.float16(9.5)
    t = torch.as_tensor(lg).cuda()
    am = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    gap = torch.full((m,), -1.0, dtype=torch.float32, device="cuda")
    ctx.argmax(aexq.describe(t, m, n), am, gap)
    torch.cuda.synchronize()
    want = orc.argmax_rows(lg.astype(np.float32))
    assert np.array_equal(am.cpu().numpy(), want)
    assert np.all(gap.cpu().numpy() == 0.0)
    lg2 = rng.standard_normal((m, n)).astype(np.float16)
    t2 = torch.as_tensor(lg2).cuda()
    ctx.argmax(aexq.describe(t2, m, n), am, gap)
    torch.cuda.synchronize()
    f = lg2.astype(np.float32)
    assert np.array_equal(am.cpu().numpy(), orc.argmax_rows(f))
    srt = np.sort(f, axis=1)
    assert np.array_equal(gap.cpu().numpy(), (srt[:, -1] - srt[:, -2]).astype(np.float32))


def test_argmax_f16_flag_is_for_the_lm_head(ctx, aexq):
    """A linear refuses the flag; the LM head accepts it alone or with RMSNorm-in."""
    from aiimage_amd import _abi, synth
    n, k = 256, 256
    words, scales, _ = synth.q8_weights(n, k, 5)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    x = torch.as_tensor(synth.activations(1, k, 6)).cuda()
    y = aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    import ctypes
    args = aexq.make_args()
    args.flags |= _abi.EPI_ARGMAX_F16
    xd = aexq.describe(x, 1, k)
    yd = aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR)
    st = ctx._lib.aexq_linear(ctx.handle, w.handle, ctypes.byref(xd), ctypes.byref(yd),
                              ctypes.byref(args))
    with pytest.raises(_abi.ArgumentError, match="LM head"):
        _abi.check(st, "aexq_linear")
    am = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    ctx.lmhead_argmax(w, xd, None, am, argmax_f16=True)
    torch.cuda.synchronize()
    assert 0 <= int(am.item()) < n
    w.release()
