"""GPU parity of the fused RMSNorm-in at activation scales far from N(0, 1).

The reference normalises in a dispatch of its own and rounds the result into
an fp16 texture: fp16(x * rsqrt(max(mean(x^2) + eps, 1e-20)) * gamma)
(AexisCommon.compute:4548-4561, paths relative to the reference root,
Packages/com.aexis/Runtime/Resources/Aexis/).  That value is bounded by
sqrt(K) * |gamma| whatever the row's scale, so the fused kernels must form it
after the sum of squares and round only then: rows of RMS 1e-6 and 1e-5 (whose
fp16 inputs are subnormal, and whose norm is set by eps) and rows with
|x| ~ 4e4 against gamma = 2 (x * gamma alone overflows fp16) are checked here
on every kernel family that fuses the norm:

  * M = 1 with one activation row per launch: the workgroup stages the row in
    LDS (single linear, q/k/v group, gate/up SwiGLU pair);
  * M = 1 where every wave normalises its own registers: K beyond the staged
    row length, and a weight stack with one activation row per copy;
  * M = 5 on the streaming kernel (K = 1056 keeps it off the MFMA kernels);
  * M = 16 on the MFMA kernels (the RMSNorm inside the wide kernel and the
    row pre-pass).

Bar: normwise max|y - r| / max|r| <= 1e-3 of the float64 oracle applied to the
same fp16 inputs, and every output finite.
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL = 1e-3
EPS = 1e-6


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


def dev(a):
    return torch.as_tensor(np.ascontiguousarray(a)).cuda()


def _weight(ctx, aexq, orc, bits, n, k, seed):
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


# (name, activation scale, gamma): "big" rows have |x| around 4e4 (clipped to
# the fp16 range) and gamma = 2, so x * gamma exceeds 65504
SCALES = [("rms1e-6", 1e-6, None), ("rms1e-5", 1e-5, None), ("big", 2e4, 2.0)]


def _inputs(m, k, seed, scale, gval):
    from aiimage_amd import synth
    x = synth.activations(m, k, seed).astype(np.float64) * scale
    x = np.clip(x, -60000.0, 60000.0).astype(np.float16)
    if gval is None:
        gamma = synth.rms_gamma(k, seed + 1)
    else:
        gamma = np.full(k, gval, np.float32)
    return x, gamma


def _reference(orc, x16, gamma, wf):
    xn = orc.rmsnorm(x16.astype(np.float32), EPS, gamma).astype(np.float16).astype(np.float32)
    return orc.gemm_gpu_semantics(xn, wf)


def _check(got, ref, what):
    got = np.asarray(got, np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = normwise(got, ref)
    assert err <= TOL, f"{what}: normwise error {err:.3e}"


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("name,scale,gval", SCALES)
def test_staged_single_row(ctx, aexq, orc, bits, name, scale, gval):
    _announce(f"rms staged m=1 bits={bits} {name}")
    n, k = 2048, 1024
    w, wf = _weight(ctx, aexq, orc, bits, n, k, 900 + bits)
    x16, gamma = _inputs(1, k, 901, scale, gval)
    y = aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), 1, k)
    yd = aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR)
    kw = dict(rmsnorm=True, rms_gamma=dev(gamma), rms_eps=EPS)
    assert ctx.plan_check(w, xd, yd, **kw).startswith("kernel=qmv")
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    _check(y.cpu().numpy()[:n], _reference(orc, x16, gamma, wf)[0], name)


@pytest.mark.parametrize("name,scale,gval", SCALES)
def test_staged_qkv_group(ctx, aexq, orc, name, scale, gval):
    _announce(f"rms staged qkv group {name}")
    k = 1024
    shapes = [2048, 512, 512]
    ws = [_weight(ctx, aexq, orc, 4, n, k, 910 + i) for i, n in enumerate(shapes)]
    x16, gamma = _inputs(1, k, 911, scale, gval)
    ys = [aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR) for n in shapes]
    ctx.linear_group([w for w, _ in ws], aexq.describe(dev(x16), 1, k),
                     [aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR) for y, n in zip(ys, shapes)],
                     rmsnorm=True, rms_gamma=dev(gamma), rms_eps=EPS)
    torch.cuda.synchronize()
    for (w, wf), y, n in zip(ws, ys, shapes):
        _check(y.cpu().numpy()[:n], _reference(orc, x16, gamma, wf)[0], f"{name} n={n}")


@pytest.mark.parametrize("name,scale,gval", SCALES)
def test_staged_gate_up_pair(ctx, aexq, orc, name, scale, gval):
    """fp32 outputs: silu(g) * u of rows whose norm is set by eps is about
    1e-7, inside fp16's subnormal range, where an fp16 output would measure
    its own rounding rather than the normalised activations'."""
    _announce(f"rms staged gate/up pair {name}")
    n, k = 3584, 1024
    wg, gf = _weight(ctx, aexq, orc, 4, n, k, 920)
    wu, uf = _weight(ctx, aexq, orc, 4, n, k, 921)
    x16, gamma = _inputs(1, k, 922, scale, gval)
    y = aexq.new_activation(1, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    ctx.linear(wg, aexq.describe(dev(x16), 1, k), aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR),
               rmsnorm=True, rms_gamma=dev(gamma), rms_eps=EPS, up=wu)
    torch.cuda.synchronize()
    g = _reference(orc, x16, gamma, gf)[0]
    u = _reference(orc, x16, gamma, uf)[0]
    ref = orc.swiglu(g.astype(np.float32), u.astype(np.float32)).astype(np.float64)
    _check(y.cpu().numpy()[:n], ref, name)


@pytest.mark.parametrize("name,scale,gval", SCALES)
def test_per_wave_long_row(ctx, aexq, orc, name, scale, gval):
    """K = 8192 is past the staged row length: every wave normalises the row
    in its own registers."""
    _announce(f"rms per-wave m=1 k=8192 {name}")
    n, k = 1536, 8192
    w, wf = _weight(ctx, aexq, orc, 4, n, k, 930)
    x16, gamma = _inputs(1, k, 931, scale, gval)
    y = aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), 1, k)
    yd = aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR)
    kw = dict(rmsnorm=True, rms_gamma=dev(gamma), rms_eps=EPS)
    assert ctx.plan_check(w, xd, yd, **kw).startswith("kernel=qmv")
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    _check(y.cpu().numpy()[:n], _reference(orc, x16, gamma, wf)[0], name)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("name,scale,gval", SCALES)
def test_per_wave_batched_rows(ctx, aexq, orc, monkeypatch, bits, name, scale, gval):
    """A weight stack with one activation row per copy: waves re-load and
    re-normalise x as their tiles cross into the next copy."""
    _announce(f"rms per-wave batched bits={bits} {name}")
    monkeypatch.setenv("AEXQ_QMV_BLOCKS_PER_CU", "1")
    n, k, copies = 3000, 1024, 3
    w, wf = _weight(ctx, aexq, orc, bits, n, k, 940 + bits)
    xs, gamma = _inputs(copies, k, 941, scale, gval)
    st = w.replicate(copies)
    out = torch.zeros(copies * n, dtype=torch.float16, device="cuda")
    xd = aexq.describe(dev(xs), 1, k, batch=copies, batch_stride=k)
    yd = aexq.describe(out, 1, n, aexq.LAYOUT_PACK4_LINEAR, batch=copies, batch_stride=n)
    ctx.linear(st, xd, yd, rmsnorm=True, rms_gamma=dev(gamma), rms_eps=EPS)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(copies, n)
    ref = _reference(orc, xs, gamma, wf)
    for c in range(copies):
        _check(got[c], ref[c], f"{name} copy {c}")


@pytest.mark.parametrize("name,scale,gval", SCALES)
def test_streaming_m5(ctx, aexq, orc, name, scale, gval):
    _announce(f"rms streaming m=5 {name}")
    m, n, k = 5, 1500, 1056
    w, wf = _weight(ctx, aexq, orc, 4, n, k, 950)
    x16, gamma = _inputs(m, k, 951, scale, gval)
    # one row of every scale in the same launch
    x16[1] = _inputs(1, k, 952, 1.0, gval)[0][0]
    y = aexq.new_activation(m, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    kw = dict(rmsnorm=True, rms_gamma=dev(gamma), rms_eps=EPS)
    assert "mmax=8" in ctx.plan_check(w, xd, yd, **kw)
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(m, -1)[:, :n]
    ref = _reference(orc, x16, gamma, wf)
    for r in range(m):
        _check(got[r], ref[r], f"{name} row {r}")


@pytest.mark.parametrize("prepass", [False, True])
@pytest.mark.parametrize("name,scale,gval", SCALES)
def test_mfma_m16(ctx, aexq, orc, monkeypatch, prepass, name, scale, gval):
    _announce(f"rms mfma m=16 prepass={prepass} {name}")
    if prepass:
        monkeypatch.setenv("AEXQ_RMS_PREPASS", "1")
    m, n, k = 16, 2048, 1024
    w, wf = _weight(ctx, aexq, orc, 4, n, k, 960)
    x16, gamma = _inputs(m, k, 961, scale, gval)
    y = aexq.new_activation(m, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    kw = dict(rmsnorm=True, rms_gamma=dev(gamma), rms_eps=EPS)
    plan = ctx.plan_check(w, xd, yd, **kw)
    assert plan.startswith("kernel=qmm"), plan
    assert ("rms_prepass=1" in plan) == prepass, plan
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(m, -1)[:, :n]
    ref = _reference(orc, x16, gamma, wf)
    for r in range(m):
        _check(got[r], ref[r], f"{name} row {r}")
