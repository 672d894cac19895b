"""Seeded random linears across the plan's boundaries, through the C ABI,
against the float64 oracle: M on both sides of every kernel family's edge (1,
2..8 streaming, up to 32 on the MFMA blocks, above 32 on the tiled GEMM), N
ragged and odd, K with and without 256-wide steps, Q8 and Q4 (groups of 16, 32
and 64, both nibble codes), fp16 and fp32 scales, fp16 and fp32 outputs, and
one epilogue per case (none, RMSNorm-in, SwiGLU-out with RMSNorm-in, residual,
alpha/beta with a per-row or per-column bias); a combination the strict plan
refuses (SwiGLU-out off the paths that take it) is skipped with the refusal's
text.  Bars as in the other parity
tests: normwise 1e-3 of the largest reference value for fp16 outputs and for
anything through RMSNorm-in or SwiGLU, 1e-5 for plain fp32 outputs.  The case
list is fixed by its seed; a failure names the case.
"""
import sys

import numpy as np
import pytest
from conftest import for_plan, q4_reference

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL32 = 1e-5
M_CHOICES = (1, 2, 3, 5, 8, 9, 16, 17, 31, 32, 33, 64, 100, 257)
K_CHOICES = (256, 512, 768, 1024, 1088, 1536, 2048)


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


def _cases(count=72, seed=2026):
    g = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        bits = int(g.choice([4, 8]))
        group = int(g.choice([16, 32, 64])) if bits == 4 else 0
        k = int(g.choice(K_CHOICES))
        if bits == 4 and k % group:
            continue
        m = int(g.choice(M_CHOICES))
        n = int(g.integers(1, 3000))
        epi = str(g.choice(["plain", "rms", "swiglu", "residual", "bias"]))
        out.append(dict(i=len(out), bits=bits, group=group, k=k, m=m, n=n, epi=epi,
                        sf16=bool(g.integers(0, 2)), y32=bool(g.integers(0, 2)),
                        code=int(g.integers(0, 2)), seed=int(g.integers(1, 1 << 30))))
    return out


def _weight(ctx, aexq, orc, c, seed):
    from aiimage_amd import synth
    n, k = c["n"], c["k"]
    sdt = np.float16 if c["sf16"] else np.float32
    odt = orc.SCALE_F16 if c["sf16"] else orc.SCALE_F32
    if c["bits"] == 8:
        words, scales, _ = synth.q8_weights(n, k, seed, scale_dtype=sdt)
        w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
        return w, orc.dequant_q8(words, scales, n, k, scale_dtype=odt)
    words, scales, _ = synth.q4_weights(n, k, seed, group=c["group"], code=c["code"],
                                        scale_dtype=sdt)
    w = ctx.weight(aexq.QuantizedTensor(n * k, c["group"], words, scales, bits=4,
                                        nibble_code=c["code"]), n, k)
    return w, q4_reference(orc, words, scales, n, k, c["group"], c["code"], c["sf16"])


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"c{c['i']}")
def test_random_linear_against_oracle(ctx, aexq, orc, case):
    c = case
    _announce("random linear " + " ".join(f"{k}={v}" for k, v in c.items()))
    from aiimage_amd import synth
    m, n, k, epi = c["m"], c["n"], c["k"], c["epi"]
    w, wf = _weight(ctx, aexq, orc, c, c["seed"])
    x16 = synth.activations(m, k, c["seed"] + 1)
    ydt = torch.float32 if c["y32"] else torch.float16
    layout = aexq.LAYOUT_PACK4_LINEAR
    y = aexq.new_activation(m, n, ydt, layout)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, layout)
    xr = x16.astype(np.float32)
    kw = {}
    tol = TOL32 if c["y32"] else TOL
    keep = []
    if epi in ("rms", "swiglu"):
        eps = 1e-6
        gamma = synth.rms_gamma(k, c["seed"] + 2)
        gd = dev(gamma)
        keep.append(gd)
        kw.update(rmsnorm=True, rms_gamma=gd, rms_eps=eps)
        xr = orc.rmsnorm(xr, eps, gamma).astype(np.float16).astype(np.float32)
        tol = TOL
    stride = aexq.storage_elements(layout, m, n)
    if epi == "swiglu":
        wu, uf = _weight(ctx, aexq, orc, c, c["seed"] + 3)
        keep.append(wu)
        kw["up"] = wu
    elif epi == "residual":
        res = synth.activations(m, n, c["seed"] + 4).astype(np.float32)
        rbuf = np.zeros((m, stride), np.float32)
        rbuf[:, :n] = res
        rt = dev(rbuf.reshape(-1)).to(ydt)
        keep.append(rt)
        kw["residual"] = aexq.describe(rt, m, n, layout)
    elif epi == "bias":
        per_col = bool(c["seed"] & 1)
        alpha, beta = 0.75, 1.25
        if per_col:
            bias = synth.activations(1, n, c["seed"] + 5).astype(np.float32).reshape(-1)
            bc = 4
        else:
            bias = synth.activations(1, m, c["seed"] + 5).astype(np.float32).reshape(-1)
            bc = 1
        bt = dev(bias)
        keep.append(bt)
        kw.update(alpha=alpha, beta=beta, c=bt, broadcast_c=bc)
    try:
        plan = ctx.plan_check(w, xd, yd, **kw)
    except aexq.NotSupportedError as e:  # the strict plan's refusal (no fallback)
        w.release()
        pytest.skip(f"refused by the plan: {e}")
    # the weights this plan multiplies (the tiled GEMM's fp16 Q4 tiles, or exact)
    wf = for_plan(wf, plan)
    ref = orc.gemm_gpu_semantics(xr, wf)
    if epi == "swiglu":
        u = orc.gemm_gpu_semantics(xr, for_plan(uf, plan))
        ref = np.stack([orc.swiglu(ref[r].astype(np.float32), u[r].astype(np.float32))
                        for r in range(m)])
    elif epi == "residual":
        ref = ref + rt.cpu().numpy().astype(np.float64).reshape(m, stride)[:, :n]
    elif epi == "bias":
        ref = orc.gemm_gpu_semantics(xr, wf, alpha=alpha, beta=beta, c=bias, broadcast_c=bc)
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    stride = aexq.storage_elements(layout, m, n)
    got = y.cpu().numpy().astype(np.float64).reshape(m, stride)
    assert np.all(np.isfinite(got[:, :n])), plan
    err = normwise(got[:, :n], ref)
    assert err <= tol, (err, plan)
    w.release()


def _group_cases(count=16, seed=2027):
    g = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        bits = int(g.choice([4, 8]))
        group = int(g.choice([16, 32, 64])) if bits == 4 else 0
        k = int(g.choice(K_CHOICES))
        if bits == 4 and k % group:
            continue
        out.append(dict(i=len(out), bits=bits, group=group, k=k, m=int(g.choice(M_CHOICES)),
                        ns=[int(v) for v in g.integers(1, 2500, size=int(g.integers(2, 4)))],
                        rms=bool(g.integers(0, 2)), sf16=bool(g.integers(0, 2)),
                        y32=bool(g.integers(0, 2)), code=int(g.integers(0, 2)),
                        seed=int(g.integers(1, 1 << 30))))
    return out


@pytest.mark.parametrize("case", _group_cases(), ids=lambda c: f"g{c['i']}")
def test_random_grouped_linear_against_oracle(ctx, aexq, orc, case):
    """aexq_linear_group: two or three weights of one format and K sharing one
    x (the q/k/v form), optional RMSNorm-in, each output against the oracle."""
    c = case
    _announce("random group " + " ".join(f"{k}={v}" for k, v in c.items()))
    from aiimage_amd import synth
    m, k = c["m"], c["k"]
    layout = aexq.LAYOUT_PACK4_LINEAR
    ydt = torch.float32 if c["y32"] else torch.float16
    ws, wfs, ys, yds = [], [], [], []
    for i, n in enumerate(c["ns"]):
        w, wf = _weight(ctx, aexq, orc, dict(c, n=n), c["seed"] + 7 * i)
        y = aexq.new_activation(m, n, ydt, layout)
        ws.append(w)
        wfs.append(wf)
        ys.append(y)
        yds.append(aexq.describe(y, m, n, layout))
    x16 = synth.activations(m, k, c["seed"] + 1)
    xd = aexq.describe(dev(x16), m, k)
    xr = x16.astype(np.float32)
    kw, tol = {}, TOL32 if c["y32"] else TOL
    if c["rms"]:
        eps = 1e-6
        gamma = synth.rms_gamma(k, c["seed"] + 2)
        gd = dev(gamma)
        kw.update(rmsnorm=True, rms_gamma=gd, rms_eps=eps)
        xr = orc.rmsnorm(xr, eps, gamma).astype(np.float16).astype(np.float32)
        tol = TOL
    plan = ctx.plan_check(ws[0], xd, yds[0], **kw)
    ctx.linear_group(ws, xd, yds, **kw)
    torch.cuda.synchronize()
    for i, n in enumerate(c["ns"]):
        ref = orc.gemm_gpu_semantics(xr, for_plan(wfs[i], plan))
        stride = aexq.storage_elements(layout, m, n)
        got = ys[i].cpu().numpy().astype(np.float64).reshape(m, stride)[:, :n]
        err = normwise(got, ref)
        assert err <= tol, (i, n, err)
    for w in ws:
        w.release()


def _batch_cases(count=16, seed=2028):
    g = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        bits = int(g.choice([4, 8]))
        group = int(g.choice([16, 32])) if bits == 4 else 0
        k = int(g.choice(K_CHOICES))
        if bits == 4 and k % group:
            continue
        out.append(dict(i=len(out), bits=bits, group=group, k=k, m=int(g.choice(M_CHOICES)),
                        n=int(g.integers(1, 2000)), copies=int(g.integers(2, 5)),
                        sf16=bool(g.integers(0, 2)), y32=bool(g.integers(0, 2)),
                        code=int(g.integers(0, 2)), seed=int(g.integers(1, 1 << 30))))
    return out


@pytest.mark.parametrize("case", _batch_cases(), ids=lambda c: f"b{c['i']}")
def test_random_batched_linear_against_oracle(ctx, aexq, orc, case):
    """A replicated weight stack with one activation matrix per copy (batched
    x and y, batch strides of whole matrices): every copy's output against the
    oracle for that copy's activations."""
    c = case
    _announce("random batched " + " ".join(f"{k}={v}" for k, v in c.items()))
    from aiimage_amd import synth
    m, n, k, copies = c["m"], c["n"], c["k"], c["copies"]
    base, wf = _weight(ctx, aexq, orc, c, c["seed"])
    w = base.replicate(copies)
    layout = aexq.LAYOUT_PACK4_LINEAR
    ydt = torch.float32 if c["y32"] else torch.float16
    per_y = aexq.tensor_elements(layout, m, n)
    y = aexq.new_activation(m, n, ydt, layout, batch=copies)
    xs = [synth.activations(m, k, c["seed"] + 10 + b) for b in range(copies)]
    xd = aexq.describe(dev(np.concatenate([x.reshape(-1) for x in xs])), m, k,
                       batch=copies, batch_stride=m * k)
    yd = aexq.describe(y, m, n, layout, batch=copies, batch_stride=per_y)
    plan = ctx.plan_check(w, xd, yd)
    ctx.linear(w, xd, yd)
    torch.cuda.synchronize()
    stride = aexq.storage_elements(layout, m, n)
    tol = TOL32 if c["y32"] else TOL
    out = y.cpu().numpy().astype(np.float64)
    for b in range(copies):
        ref = orc.gemm_gpu_semantics(xs[b].astype(np.float32), for_plan(wf, plan))
        got = out[b * per_y:b * per_y + m * stride].reshape(m, stride)[:, :n]
        err = normwise(got, ref)
        assert err <= tol, (b, err)
    w.release()
    base.release()
