"""GPU parity of the streaming (M <= 8) kernel's epilogue paths against the CPU
oracle: the residual add with fp16 and fp32 outputs on ragged N and on waves
that stream several tiles, RMSNorm-in without an affine gamma, the M = 2..8
kernel with RMSNorm-in and the residual, and the activation reload between
the batch entries of a weight stack with a batched x.

Bars as in the other parity tests: normwise max|y - r| / max|r| <= 1e-3 of the
float64 oracle; a stacked launch equals the single launches bit for bit.
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


def dev(a, dtype=None):
    t = torch.as_tensor(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def _weight(ctx, aexq, orc, bits, n, k, seed):
    """Device weight and its float64 dequantization (Q4: offset-8, fp16 scales per 32)."""
    from aiimage_amd import synth
    if bits == 8:
        words, scales, _ = synth.q8_weights(n, k, seed)
        w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
        wf = orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F16)
    else:
        words, scales, _ = synth.q4_weights(n, k, seed, group=32, code=synth.NIBBLE_OFFSET8)
        w = ctx.weight(aexq.QuantizedTensor(n * k, 32, words, scales, bits=4,
                                            nibble_code=synth.NIBBLE_OFFSET8), n, k)
        wf = orc.dequant_q4(words, scales, n, k, 32, synth.NIBBLE_OFFSET8, orc.SCALE_F16)
    return w, wf


@pytest.mark.parametrize("bits,n,k,ydt,per_cu", [
    (4, 1000, 2048, torch.float16, 0),     # ragged N, one tile per wave
    (4, 1000, 2048, torch.float32, 0),     # fp32 output and residual
    (4, 16000, 1024, torch.float16, 1),    # several tiles per wave, ragged N
    (8, 8000, 1024, torch.float16, 1),
    (8, 8000, 1024, torch.float32, 1),
])
def test_residual_add_streaming(ctx, aexq, orc, monkeypatch, bits, n, k, ydt, per_cu):
    _announce(f"residual bits={bits} n={n} k={k} y={ydt} per_cu={per_cu}")
    from aiimage_amd import synth
    if per_cu:
        # a one-workgroup-per-CU grid makes each wave stream several row tiles
        monkeypatch.setenv("AEXQ_QMV_BLOCKS_PER_CU", str(per_cu))
    w, wf = _weight(ctx, aexq, orc, bits, n, k, 700 + n + bits)
    x16 = synth.activations(1, k, 701)
    res = synth.activations(1, n, 702).astype(np.float32)
    rd = dev(res, ydt)
    y = aexq.new_activation(1, n, ydt, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), 1, k)
    yd = aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR)
    rdesc = aexq.describe(rd, 1, n, aexq.LAYOUT_PACK4_LINEAR)
    plan = ctx.plan_check(w, xd, yd, residual=rdesc)
    assert plan.startswith("kernel=qmv"), plan
    if per_cu:
        tiles = int(plan.split("tiles=")[1].split()[0])
        grid = int(plan.split("grid=")[1].split()[0])
        assert tiles > 4 * grid, plan   # more tiles than waves
    ctx.linear(w, xd, yd, residual=rdesc)
    torch.cuda.synchronize()
    rq = rd.cpu().numpy().astype(np.float64)
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), wf)[0] + rq
    assert normwise(y.cpu().numpy()[:n], ref) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
def test_rmsnorm_in_without_gamma(ctx, aexq, orc, bits):
    _announce(f"rmsnorm without gamma bits={bits}")
    from aiimage_amd import synth
    n, k, eps = 2048, 1024, 1e-6
    w, wf = _weight(ctx, aexq, orc, bits, n, k, 710 + bits)
    x16 = synth.activations(1, k, 711) * np.float16(3.0)
    y = aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    ctx.linear(w, aexq.describe(dev(x16), 1, k), aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR),
               rmsnorm=True, rms_eps=eps)
    torch.cuda.synchronize()
    xn = orc.rmsnorm(x16.astype(np.float32), eps).astype(np.float16).astype(np.float32)
    ref = orc.gemm_gpu_semantics(xn, wf)[0]
    assert normwise(y.cpu().numpy()[:n], ref) <= TOL


@pytest.mark.parametrize("m", [2, 5, 8])
def test_small_m_streaming_rms_residual(ctx, aexq, orc, m):
    """K = 1056 (33 chunks of 32) keeps M = 2..8 on the streaming kernel."""
    _announce(f"streaming m={m} rms+residual")
    from aiimage_amd import synth
    n, k, eps = 1500, 1056, 1e-6
    w, wf = _weight(ctx, aexq, orc, 4, n, k, 720 + m)
    x16 = synth.activations(m, k, 721)
    gamma = synth.rms_gamma(k, 722)
    res = synth.activations(m, n, 723)
    y = aexq.new_activation(m, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    rdesc = aexq.describe(dev(res), m, n, aexq.LAYOUT_PACK4_LINEAR)
    kw = dict(rmsnorm=True, rms_gamma=dev(gamma), rms_eps=eps, residual=rdesc)
    plan = ctx.plan_check(w, xd, yd, **kw)
    assert "mmax=8" in plan, plan
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    xn = orc.rmsnorm(x16.astype(np.float32), eps, gamma).astype(np.float16).astype(np.float32)
    ref = orc.gemm_gpu_semantics(xn, wf) + res.astype(np.float64)
    got = y.cpu().numpy().reshape(m, -1)[:, :n]
    assert normwise(got, ref) <= TOL


@pytest.mark.parametrize("bits", [4, 8])
def test_stacked_batched_x_rms_matches_single(ctx, aexq, orc, monkeypatch, bits):
    """A weight stack with one activation row per copy: each wave re-loads (and
    re-normalises) x when its tiles cross into the next copy.  Every copy must
    match the single launch on its own x up to fp16 rounding (a single launch
    stages its row once per workgroup and reduces sum(x^2) in another order, so
    1/rms may differ in its last bit), and the oracle to 1e-3."""
    _announce(f"stacked batched x rms bits={bits}")
    from aiimage_amd import synth
    monkeypatch.setenv("AEXQ_QMV_BLOCKS_PER_CU", "1")
    n, k, eps, copies = 3000, 1024, 1e-6, 4
    w, wf = _weight(ctx, aexq, orc, bits, n, k, 730 + bits)
    gamma = dev(synth.rms_gamma(k, 731))
    xs = synth.activations(copies, k, 732)
    xd_all = dev(xs)
    singles = []
    for c in range(copies):
        y = aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
        ctx.linear(w, aexq.describe(dev(xs[c:c + 1]), 1, k),
                   aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR),
                   rmsnorm=True, rms_gamma=gamma, rms_eps=eps)
        singles.append(y)
    st = w.replicate(copies)
    out = torch.zeros(copies * n, dtype=torch.float16, device="cuda")
    xd = aexq.describe(xd_all, 1, k, batch=copies, batch_stride=k)
    yd = aexq.describe(out, 1, n, aexq.LAYOUT_PACK4_LINEAR, batch=copies, batch_stride=n)
    ctx.linear(st, xd, yd, rmsnorm=True, rms_gamma=gamma, rms_eps=eps)
    torch.cuda.synchronize()
    for c in range(copies):
        got_c = out[c * n:(c + 1) * n].float().cpu().numpy()
        one_c = singles[c][:n].float().cpu().numpy()
        assert normwise(got_c, one_c) <= 2.0 ** -10, c
    xn = orc.rmsnorm(xs.astype(np.float32), eps, synth.rms_gamma(k, 731))
    ref = orc.gemm_gpu_semantics(xn.astype(np.float16).astype(np.float32), wf)
    got = out.cpu().numpy().reshape(copies, n)
    assert normwise(got, ref) <= TOL
