"""GPU parity of the tiled GEMM path (M > 32 activation rows, and 9..32 rows
where K or the Q4 scale groups rule out the MFMA block kernel:
aexq_qgemm_dl.hpp, the LDS-direct kernel, and aexq_qgemm.hpp, the
register-staged one) against the CPU oracle, through the C ABI.

Bars as in the other parity tests: normwise max|y - r| / max|r| <= 1e-3 of the
float64 oracle for fp16 outputs, 1e-5 for fp32 outputs; stacked weight copies
equal the single launch bit for bit.  Q8, and Q4 under AEXQ_EPI_EXACT_DEQUANT,
keep the dequantised weight exactly float(q) * scale (codes as exact fp16
integers, scales applied in fp32); the default Q4 form multiplies fp16 weight
tiles fp16(q * s), so its fp32 outputs are held to 1e-5 against the oracle of
those fp16 weights (conftest.q4_reference, chosen by the plan's
fp16_dequant field) and to 1e-3 against the exact oracle.
"""
import sys

import numpy as np
import pytest
from conftest import DequantRef, for_plan, q4_reference

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL32 = 1e-5


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


def _weight(ctx, aexq, orc, bits, n, k, seed, group=32, scale_f16=True, code=1):
    """Device weight and its float64 dequantisation by the oracle."""
    from aiimage_amd import synth
    sdt = np.float16 if scale_f16 else np.float32
    odt = orc.SCALE_F16 if scale_f16 else orc.SCALE_F32
    if bits == 8:
        words, scales, _ = synth.q8_weights(n, k, seed, scale_dtype=sdt)
        w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
        return w, orc.dequant_q8(words, scales, n, k, scale_dtype=odt)
    words, scales, _ = synth.q4_weights(n, k, seed, group=group, code=code, scale_dtype=sdt)
    w = ctx.weight(aexq.QuantizedTensor(n * k, group, words, scales, bits=4, nibble_code=code),
                   n, k)
    return w, q4_reference(orc, words, scales, n, k, group, code, scale_f16)


@pytest.mark.parametrize("bits,group,scale_f16,n,k,m,y32", [
    (4, 32, True, 3072, 1024, 64, False),    # q/k/v grouped shape, one 64-row tile
    (4, 32, True, 1024, 3584, 512, False),   # down_proj at M = 512
    (8, 0, True, 1024, 2048, 512, False),    # Q8 o_proj at M = 512
    (8, 0, False, 1000, 1088, 200, True),    # ragged N and M, K = 17 steps (not a multiple of 128)
    (8, 0, True, 1001, 1024, 100, False),    # odd N with fp16 row scales: the last row's scale
    (4, 64, False, 520, 1024, 97, True),     # one scale per 64 codes, fp32 scales
    (4, 32, True, 130, 64, 33, True),        # a single K step, 2 rows past a tile
    (4, 32, False, 256, 512, 129, True),     # reference nibble code below
    # 9..32 rows where the MFMA block kernel does not apply: the tiled GEMM
    (8, 0, True, 1000, 1088, 16, False),     # K = 17 steps at M = 16
    (4, 64, True, 768, 1024, 24, True),      # Q4 groups of 64 at M = 24
    (4, 128, False, 515, 2048, 9, True),     # Q4 groups of 128 at M = 9
    (8, 0, False, 257, 576, 32, True),       # K = 9 steps at M = 32
])
def test_gemm_formats(ctx, aexq, orc, bits, group, scale_f16, n, k, m, y32):
    _announce(f"qgemm q{bits} g={group} f16={scale_f16} n={n} k={k} m={m}")
    from aiimage_amd import synth
    code = 0 if (bits == 4 and m == 129) else 1   # two's complement (reference) vs offset-8
    w, wf = _weight(ctx, aexq, orc, bits, n, k, n + k + m, group=group or k,
                    scale_f16=scale_f16, code=code)
    x16 = synth.activations(m, k, m + 5)
    ydt = torch.float32 if y32 else torch.float16
    y = aexq.new_activation(m, n, ydt, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    plan = ctx.plan_check(w, xd, yd)
    assert plan.startswith("kernel=qgemm"), plan
    ctx.linear(w, xd, yd)
    torch.cuda.synchronize()
    stride = aexq.storage_elements(aexq.LAYOUT_PACK4_LINEAR, m, n)
    got = y.cpu().numpy().astype(np.float64).reshape(m, stride)
    assert np.all(got[:, n:] == 0)
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), for_plan(wf, plan))
    assert normwise(got[:, :n], ref) <= (TOL32 if y32 else TOL)
    if isinstance(wf, DequantRef):
        exact = orc.gemm_gpu_semantics(x16.astype(np.float32), wf.exact)
        assert normwise(got[:, :n], exact) <= TOL


@pytest.mark.parametrize("bits,m,n,k", [(4, 64, 3584, 1024), (4, 150, 1000, 1024),
                                         (8, 96, 640, 1024), (8, 16, 640, 1088),
                                         (4, 20, 1000, 576)])
def test_gemm_swiglu_rmsnorm(ctx, aexq, orc, bits, m, n, k):
    """gate/up with RMSNorm-in (row pre-pass) and SwiGLU-out on the tiled path,
    also at 16 and 20 rows with K not a multiple of 128 (no MFMA block kernel)."""
    _announce(f"qgemm swiglu rms q{bits} m={m} n={n} k={k}")
    from aiimage_amd import synth
    eps = 1e-6
    wg, gf = _weight(ctx, aexq, orc, bits, n, k, 61 + m)
    wu, uf = _weight(ctx, aexq, orc, bits, n, k, 62 + m)
    x16 = synth.activations(m, k, 63)
    gamma = synth.rms_gamma(k, 64)
    y = aexq.new_activation(m, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    kw = dict(rmsnorm=True, rms_gamma=dev(gamma), rms_eps=eps, up=wu)
    plan = ctx.plan_check(wg, xd, yd, **kw)
    assert plan.startswith("kernel=qgemm") and "rms_prepass=1" in plan and "swiglu=1" in plan, plan
    ctx.linear(wg, xd, yd, **kw)
    torch.cuda.synchronize()
    xn = orc.rmsnorm(x16.astype(np.float32), eps, gamma).astype(np.float16).astype(np.float32)
    g = orc.gemm_gpu_semantics(xn, for_plan(gf, plan))
    u = orc.gemm_gpu_semantics(xn, for_plan(uf, plan))
    ref = np.stack([orc.swiglu(g[r].astype(np.float32), u[r].astype(np.float32)) for r in range(m)])
    got = y.cpu().numpy().astype(np.float64).reshape(m, -1)[:, :n]
    assert normwise(got, ref) <= TOL


@pytest.mark.parametrize("path", ["qgemm", "qmm"])
@pytest.mark.parametrize("bcast,layout", [(1, "linear"), (3, "linear"), (4, "tiled")])
def test_gemm_bias_residual(ctx, aexq, orc, monkeypatch, path, bcast, layout):
    """alpha/beta/C per row, per element and per column, with the residual, on
    the tiled GEMM and (switched off) on the 32-row MFMA blocks."""
    _announce(f"qgemm bias bcast={bcast} layout={layout} path={path}")
    from aiimage_amd import synth
    if path == "qmm":
        monkeypatch.setenv("AEXQ_QGEMM_OFF", "1")
    n, k, m = 512, 1024, 70
    w, wf = _weight(ctx, aexq, orc, 8, n, k, 71, scale_f16=False)
    x16 = synth.activations(m, k, 72)
    rng = np.random.default_rng(73 + bcast)
    c = rng.standard_normal({1: m, 3: m * n, 4: n}[bcast]).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    lay = aexq.LAYOUT_PACK4_LINEAR if layout == "linear" else aexq.LAYOUT_PACK4_TILED
    y = aexq.new_activation(m, n, torch.float32, lay)
    stride = aexq.storage_elements(lay, m, n)
    rbuf = np.zeros((m, stride), np.float32)
    rbuf[:, :n] = res
    rd = dev(rbuf)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, lay)
    kw = dict(alpha=0.75, beta=1.5, c=dev(c), broadcast_c=bcast,
              residual=aexq.describe(rd, m, n, lay))
    assert ctx.plan_check(w, xd, yd, **kw).startswith(f"kernel={path}")
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    s = orc.gemm_gpu_semantics(x16.astype(np.float32), wf)
    if bcast == 1:
        cc = np.repeat(c[:, None], n, 1)
    elif bcast == 3:
        cc = c.reshape(m, n)
    else:
        cc = np.repeat(c[None, :], m, 0)
    # Pack4 linear: alpha * (beta C + sum) (MM:1101); tiled: beta C + alpha sum (MM:2301)
    ref = (0.75 * (1.5 * cc + s) if layout == "linear" else 1.5 * cc + 0.75 * s) + res
    got = y.cpu().numpy().reshape(m, stride)[:, :n]
    assert normwise(got, ref) <= TOL32


@pytest.mark.parametrize("splitk", ["1", "4"])
@pytest.mark.parametrize("bits", [4, 8])
def test_gemm_stacked_copies_batched_x_match_single(ctx, aexq, orc, monkeypatch, bits, splitk):
    """Size-independent property: a replicated weight stack with one activation
    matrix per copy gives exactly each copy's single launch (the same K
    chunking for both: the plan would split the single launch only)."""
    _announce(f"qgemm stacked q{bits} splitk={splitk}")
    monkeypatch.setenv("AEXQ_SPLITK", splitk)
    from aiimage_amd import synth
    n, k, m, copies = 640, 1024, 80, 3
    w, wf = _weight(ctx, aexq, orc, bits, n, k, 81 + bits)
    xs = synth.activations(copies * m, k, 82)
    singles = []
    for c in range(copies):
        y1 = aexq.new_activation(m, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
        x1 = aexq.describe(dev(xs[c * m:(c + 1) * m]), m, k)
        y1d = aexq.describe(y1, m, n, aexq.LAYOUT_PACK4_LINEAR)
        plan1 = ctx.plan_check(w, x1, y1d)
        ctx.linear(w, x1, y1d)
        singles.append(y1)
    st = w.replicate(copies)
    ys = torch.zeros(copies * m * n, dtype=torch.float16, device="cuda")
    xd = aexq.describe(dev(xs), m, k, batch=copies, batch_stride=m * k)
    yd = aexq.describe(ys, m, n, aexq.LAYOUT_PACK4_LINEAR, batch=copies, batch_stride=m * n)
    assert ctx.plan_check(st, xd, yd).startswith("kernel=qgemm")
    ctx.linear(st, xd, yd)
    torch.cuda.synchronize()
    for c in range(copies):
        assert torch.equal(ys[c * m * n:(c + 1) * m * n], singles[c]), c
    ref = orc.gemm_gpu_semantics(xs[:m].astype(np.float32), for_plan(wf, plan1))
    assert normwise(singles[0].cpu().numpy().reshape(m, n), ref) <= TOL


@pytest.mark.parametrize("scale_f16,n,k,m,swiglu", [
    (False, 512, 1024, 48, False),    # the reference's shipping Q4: group 16, fp32 scales
    (False, 1000, 2048, 300, False),  # ragged N, three 64-row tiles and a partial one
    (True, 1024, 3584, 64, False),    # fp16 scales, down_proj shape
    (False, 1024, 1024, 128, True),   # gate/up pair
    (False, 640, 1088, 96, False),    # 17 K steps: the two-step loop's odd tail
    (True, 384, 1216, 80, True),      # 19 K steps, gate/up pair
])
@pytest.mark.parametrize("splitk", ["", "3"])
@pytest.mark.parametrize("exact", [False, True])
def test_gemm_group16(ctx, aexq, orc, monkeypatch, scale_f16, n, k, m, swiglu, splitk, exact):
    """Q4 with one scale per 16 codes on the tiled GEMM, in both forms: fp16
    weight tiles (each lane's eight codes of an extent share one scale, one
    MFMA per extent) and the exact one (two MFMAs per 32-code extent, each
    group's product scaled in fp32).  With three forced K chunks the chunks'
    step counts differ (a tail of the three-step loop, or none)."""
    if splitk:
        monkeypatch.setenv("AEXQ_SPLITK", splitk)
    _announce(f"qgemm group16 f16={scale_f16} n={n} k={k} m={m} swiglu={swiglu} splitk={splitk}")
    from aiimage_amd import synth
    w, wf = _weight(ctx, aexq, orc, 4, n, k, 91 + m, group=16, scale_f16=scale_f16, code=0)
    x16 = synth.activations(m, k, 92)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    kw = dict(exact=exact)
    if swiglu:
        wu, uf = _weight(ctx, aexq, orc, 4, n, k, 93 + m, group=16, scale_f16=scale_f16, code=0)
        kw["up"] = wu
    plan = ctx.plan_check(w, xd, yd, **kw)
    assert plan.startswith("kernel=qgemm") and "direct=1" in plan, plan
    assert f"fp16_dequant={0 if exact else 1}" in plan, plan
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    g = orc.gemm_gpu_semantics(x16.astype(np.float32), for_plan(wf, plan))
    if swiglu:
        u = orc.gemm_gpu_semantics(x16.astype(np.float32), for_plan(uf, plan))
        ref = np.stack([orc.swiglu(g[r].astype(np.float32), u[r].astype(np.float32))
                        for r in range(m)])
    else:
        ref = g
    stride = aexq.storage_elements(aexq.LAYOUT_PACK4_LINEAR, m, n)
    got = y.cpu().numpy().reshape(m, stride)
    assert np.all(got[:, n:] == 0)
    assert normwise(got[:, :n], ref) <= TOL32


@pytest.mark.parametrize("group", [16, 32])
def test_gemm_q4_extreme_scales_exact(ctx, aexq, orc, group):
    """Per-group fp32 scaling keeps the dequantised weight exactly float(q) *
    scale for every fp16 scale: subnormal, large and above 4096 (where q * s
    would overflow an fp16 product) among the groups -- the fp32-output bar
    against the float64 oracle."""
    _announce(f"qgemm q4 extreme scales g={group}")
    from aiimage_amd import synth
    n, k, m = 512, 1024, 130
    words, scales, _ = synth.q4_weights(n, k, 95, group=group, code=synth.NIBBLE_OFFSET8)
    bits = scales.view(np.uint16).copy()
    bits[:300] = np.arange(1, 301, dtype=np.uint16)              # subnormal scales
    bits[300:310] = np.float16(1000.0).view(np.uint16)
    bits[310:320] = np.float16(4096.0).view(np.uint16)
    bits[320:330] = np.float16(5000.0).view(np.uint16)           # q * s beyond fp16 range
    sc = bits.view(np.float16)
    w = ctx.weight(aexq.QuantizedTensor(n * k, group, words, sc, bits=4,
                                        nibble_code=synth.NIBBLE_OFFSET8), n, k)
    wf = orc.dequant_q4(words, sc, n, k, group, synth.NIBBLE_OFFSET8, orc.SCALE_F16)
    x16 = synth.activations(m, k, 96)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    plan = ctx.plan_check(w, xd, yd, exact=True)
    assert "direct=1" in plan and "fp16_dequant=0" in plan, plan
    ctx.linear(w, xd, yd, exact=True)
    torch.cuda.synchronize()
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), wf)
    assert normwise(y.cpu().numpy().reshape(m, n), ref) <= TOL32


@pytest.mark.parametrize("big", [8000.0, 9000.0, float("inf")])
def test_gemm_fp16_dequant_needs_finite_products(ctx, aexq, orc, big):
    """The fp16 weight tile is chosen only when 8 |s| fits fp16 for every scale
    of the weight: a weight with one fp32 scale of 9000 (q * s up to 72000)
    takes the exact form by itself and stays within the fp32 bar; 8000 (64000,
    finite) keeps the fp16 tile; an infinite scale takes the exact form and
    propagates to its output column as the oracle's does."""
    _announce(f"qgemm fp16 dequant guard {big}")
    from aiimage_amd import synth
    n, k, m = 256, 512, 96
    words, scales, _ = synth.q4_weights(n, k, 97, group=16, code=synth.NIBBLE_TWOS,
                                        scale_dtype=np.float32)
    scales = scales.copy()
    scales[5] = np.float32(big)
    w = ctx.weight(aexq.QuantizedTensor(n * k, 16, words, scales, bits=4,
                                        nibble_code=synth.NIBBLE_TWOS), n, k)
    x16 = synth.activations(m, k, 98)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    plan = ctx.plan_check(w, xd, yd)
    want_fd = big < 65504.0 / 8
    assert f"fp16_dequant={int(want_fd)}" in plan, plan
    ctx.linear(w, xd, yd)
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(m, n).astype(np.float64)
    ref = orc.gemm_gpu_semantics(
        x16.astype(np.float32),
        for_plan(q4_reference(orc, words, scales, n, k, 16, synth.NIBBLE_TWOS, False), plan))
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), fin)
    assert normwise(got[fin], ref[fin]) <= TOL32


@pytest.mark.parametrize("bits,group", [(8, 0), (4, 32), (4, 16)])
@pytest.mark.parametrize("k", [64, 128, 192, 320])
@pytest.mark.parametrize("m", [40, 100])
def test_gemm_direct_step_counts(ctx, aexq, orc, bits, group, k, m):
    """The LDS-direct kernel runs its K steps three per loop iteration with a
    tail of one or two: 1, 2, 3 and 5 steps, on 64-row (M = 40) and 128-row
    (M = 100) tiles, two weight tiles with the second one partial."""
    _announce(f"qgemm direct q{bits} g={group} k={k} m={m}")
    from aiimage_amd import synth
    n = 200
    w, wf = _weight(ctx, aexq, orc, bits, n, k, 7 * k + m + bits, group=group or k, code=0)
    x16 = synth.activations(m, k, k + m)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    plan = ctx.plan_check(w, xd, yd)
    assert "direct=1" in plan and f"bm={64 if m <= 64 else 128}" in plan, plan
    ctx.linear(w, xd, yd)
    torch.cuda.synchronize()
    stride = aexq.storage_elements(aexq.LAYOUT_PACK4_LINEAR, m, n)
    got = y.cpu().numpy().reshape(m, stride)
    assert np.all(got[:, n:] == 0)
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), for_plan(wf, plan))
    assert normwise(got[:, :n], ref) <= TOL32


@pytest.mark.parametrize("bits,group,scale_f16", [(8, 0, True), (8, 0, False), (4, 16, True),
                                                   (4, 16, False), (4, 32, True), (4, 32, False)])
@pytest.mark.parametrize("m", [40, 100])
def test_gemm_direct_pairs(ctx, aexq, orc, bits, group, scale_f16, m):
    """gate/up pairs on the LDS-direct kernel, both tile heights, fp16 and fp32
    scales, against the oracle."""
    _announce(f"qgemm direct pair q{bits} g={group} f16={scale_f16} m={m}")
    from aiimage_amd import synth
    n, k = 320, 256
    wg, gf = _weight(ctx, aexq, orc, bits, n, k, 301 + m, group=group or k,
                     scale_f16=scale_f16, code=0)
    wu, uf = _weight(ctx, aexq, orc, bits, n, k, 302 + m, group=group or k,
                     scale_f16=scale_f16, code=0)
    x16 = synth.activations(m, k, 303)
    xd = aexq.describe(dev(x16), m, k)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    plan = ctx.plan_check(wg, xd, yd, up=wu)
    assert plan.startswith("kernel=qgemm") and "direct=1" in plan, plan
    ctx.linear(wg, xd, yd, up=wu)
    torch.cuda.synchronize()
    g = orc.gemm_gpu_semantics(x16.astype(np.float32), for_plan(gf, plan))
    u = orc.gemm_gpu_semantics(x16.astype(np.float32), for_plan(uf, plan))
    ref = np.stack([orc.swiglu(g[r].astype(np.float32), u[r].astype(np.float32)) for r in range(m)])
    assert normwise(y.cpu().numpy().reshape(m, -1)[:, :n], ref) <= TOL32


@pytest.mark.parametrize("group,scale_f16", [(16, False), (32, False), (16, True)])
@pytest.mark.parametrize("k", [64, 192, 320])
@pytest.mark.parametrize("m", [40, 100])
@pytest.mark.parametrize("exact", [False, True])
def test_gemm_direct_group_scaling(ctx, aexq, orc, group, scale_f16, k, m, exact):
    """Q4 scales on the LDS-direct kernel in both forms (fp16 weight tiles; exact
    per-group fp32 scaling), fp32 and fp16 scales: 1, 3 and 5 K steps, both
    tile heights."""
    _announce(f"qgemm direct per-group g={group} f16={scale_f16} k={k} m={m}")
    from aiimage_amd import synth
    n = 200
    w, wf = _weight(ctx, aexq, orc, 4, n, k, 11 * k + m, group=group, scale_f16=scale_f16,
                    code=0)
    x16 = synth.activations(m, k, 3 * k + m)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    plan = ctx.plan_check(w, xd, yd, exact=exact)
    assert "direct=1" in plan and f"fp16_dequant={0 if exact else 1}" in plan, plan
    ctx.linear(w, xd, yd, exact=exact)
    torch.cuda.synchronize()
    stride = aexq.storage_elements(aexq.LAYOUT_PACK4_LINEAR, m, n)
    got = y.cpu().numpy().reshape(m, stride)
    assert np.all(got[:, n:] == 0)
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), for_plan(wf, plan))
    assert normwise(got[:, :n], ref) <= TOL32
