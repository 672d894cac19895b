"""GPU parity of split K in the MFMA kernels (the wide-step kernel at M <= 32
and the tiled GEMM at M > 32) against the CPU oracle, through the C ABI.

A single layer's linear at M = 16..512 has few output tiles (8 for a
1024-row output), so the plan cuts every tile's K steps into chunks that run
as separate workgroups; their fp32 partials are summed in chunk order by the
fix-up launch, which also applies the epilogue (Q8 row scale, bias, SwiGLU,
residual, output layout).  Bars: normwise max|y - r| / max|r| <= 1e-3 of the
float64 oracle for fp16 outputs, 1e-5 for fp32 outputs; split and unsplit
launches agree to fp32 summation order; the same launch repeated is bit-exact.
"""
import sys

import numpy as np
import pytest
from conftest import for_plan, q4_reference

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


def _splitk(plan):
    for tok in plan.split():
        if tok.startswith("splitk="):
            return int(tok[7:])
    raise AssertionError(plan)


def _kstep(plan):
    """K per step of a tiled-GEMM plan (64, or 128 for Q4 fp16 tiles at 64-row tiles)."""
    for tok in plan.split():
        if tok.startswith("kstep="):
            return int(tok[6:])
    raise AssertionError(plan)


# (bits, scale_f16, n, k, m, fp32 out, kernel): a layer's linears at the
# config-4 row counts, one copy each, plus ragged N and M
CASES = [
    (4, True, 1024, 2048, 16, False, "qmm"),    # o_proj, M = 16
    (4, True, 1024, 3584, 32, True, "qmm"),     # down_proj, M = 32 (two 16-row tiles)
    (8, True, 3072, 2048, 16, False, "qmm"),    # Q8, 3072 rows
    (8, False, 1000, 2048, 23, True, "qmm"),    # ragged N and M, fp32 scales
    (4, True, 1024, 2048, 64, False, "qgemm"),  # o_proj, M = 64
    (4, True, 1024, 3584, 512, True, "qgemm"),  # down_proj, M = 512 (split fp16 scales)
    (8, True, 1024, 3584, 64, True, "qgemm"),   # Q8 down_proj, M = 64
    (8, False, 520, 2048, 97, True, "qgemm"),   # ragged, fp32 scales
]


@pytest.mark.parametrize("bits,scale_f16,n,k,m,y32,kernel", CASES)
def test_split_matches_oracle(ctx, aexq, orc, monkeypatch, bits, scale_f16, n, k, m, y32, kernel):
    _announce(f"splitk q{bits} f16={scale_f16} n={n} k={k} m={m} y32={y32} {kernel}")
    from aiimage_amd import synth
    w, wf = _weight(ctx, aexq, orc, bits, n, k, n + k + m, scale_f16=scale_f16)
    x16 = synth.activations(m, k, m + 11)
    ydt = torch.float32 if y32 else torch.float16
    lay = aexq.LAYOUT_PACK4_LINEAR
    xd = aexq.describe(dev(x16), m, k)
    y = aexq.new_activation(m, n, ydt, lay)
    yd = aexq.describe(y, m, n, lay)
    plan = ctx.plan_check(w, xd, yd)
    assert plan.startswith(f"kernel={kernel}") and _splitk(plan) > 1, plan
    ctx.linear(w, xd, yd)
    torch.cuda.synchronize()
    stride = aexq.storage_elements(lay, m, n)
    got = y.cpu().numpy().astype(np.float64).reshape(m, stride)
    assert np.all(got[:, n:] == 0)
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), for_plan(wf, plan))
    assert normwise(got[:, :n], ref) <= (TOL32 if y32 else TOL)
    # the same launch again: bit-exact
    y2 = aexq.new_activation(m, n, ydt, lay)
    ctx.linear(w, xd, aexq.describe(y2, m, n, lay))
    # unsplit: the same sums in another order
    monkeypatch.setenv("AEXQ_SPLITK", "1")
    y1 = aexq.new_activation(m, n, ydt, lay)
    yd1 = aexq.describe(y1, m, n, lay)
    assert _splitk(ctx.plan_check(w, xd, yd1)) == 1
    ctx.linear(w, xd, yd1)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    one = y1.cpu().numpy().astype(np.float64).reshape(m, stride)[:, :n]
    assert normwise(got[:, :n], one) <= (TOL32 if y32 else TOL)


@pytest.mark.parametrize("bits,group,n,k,m,pair", [
    (4, 16, 1024, 2048, 16, False),   # the reference's shipping Q4: group 16, fp32 scales
    (4, 16, 1024, 3584, 32, True),    # ... gate/up pair at M = 32
    (8, 0, 1024, 1152, 16, False),    # K = 9 x 128: not a multiple of the wide step
])
def test_split_narrow_kernel(ctx, aexq, orc, monkeypatch, bits, group, n, k, m, pair):
    """The 128-wide-slice MFMA kernel (K not a multiple of 256, or switched to
    with AEXQ_QMM_NARROW) splits K per wave tile the same way."""
    _announce(f"splitk narrow q{bits} g={group} n={n} k={k} m={m} pair={pair}")
    monkeypatch.setenv("AEXQ_QMM_NARROW", "1")
    from aiimage_amd import synth
    w, wf = _weight(ctx, aexq, orc, bits, n, k, 91 + m, group=group or k, scale_f16=False,
                    code=0)
    x16 = synth.activations(m, k, 92)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    kw = {}
    if pair:
        wu, uf = _weight(ctx, aexq, orc, bits, n, k, 93 + m, group=group or k, scale_f16=False,
                         code=0)
        kw = dict(up=wu)
    plan = ctx.plan_check(w, xd, yd, **kw)
    assert plan.startswith("kernel=qmm") and "wide=0" in plan and _splitk(plan) > 1, plan
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    g = orc.gemm_gpu_semantics(x16.astype(np.float32), for_plan(wf, plan))
    if pair:
        u = orc.gemm_gpu_semantics(x16.astype(np.float32), for_plan(uf, plan))
        ref = np.stack([orc.swiglu(g[r].astype(np.float32), u[r].astype(np.float32))
                        for r in range(m)])
    else:
        ref = g
    assert normwise(y.cpu().numpy().reshape(m, n), ref) <= TOL32


@pytest.mark.parametrize("scale_f16,m,pair,rms", [
    (False, 16, False, False),   # the reference's shipping Q4: group 16, fp32 scales
    (False, 32, True, True),     # gate/up pair at M = 32 with RMSNorm-in in the kernel
    (True, 9, False, True),      # fp16 scales, RMSNorm-in
])
def test_wide_kernel_group16(ctx, aexq, orc, scale_f16, m, pair, rms):
    """Group-16 Q4 on the wide kernel: two MFMAs per 32-code extent, each
    group's product scaled in fp32 (exact float(q) * scale)."""
    _announce(f"wide group16 f16={scale_f16} m={m} pair={pair} rms={rms}")
    from aiimage_amd import synth
    n, k, eps = 1024, 2048, 1e-6
    w, wf = _weight(ctx, aexq, orc, 4, n, k, 131 + m, group=16, scale_f16=scale_f16, code=0)
    kw = {}
    if pair:
        wu, uf = _weight(ctx, aexq, orc, 4, n, k, 132 + m, group=16, scale_f16=scale_f16, code=0)
        kw["up"] = wu
    gamma = synth.rms_gamma(k, 133)
    if rms:
        kw.update(rmsnorm=True, rms_gamma=dev(gamma), rms_eps=eps)
    x16 = synth.activations(m, k, 134)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    plan = ctx.plan_check(w, xd, yd, **kw)
    assert plan.startswith("kernel=qmm") and "wide=1" in plan, plan
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    xr = x16.astype(np.float32)
    if rms:
        xr = orc.rmsnorm(xr, eps, gamma).astype(np.float16).astype(np.float32)
    g = orc.gemm_gpu_semantics(xr, for_plan(wf, plan))
    if pair:
        u = orc.gemm_gpu_semantics(xr, for_plan(uf, plan))
        ref = np.stack([orc.swiglu(g[r].astype(np.float32), u[r].astype(np.float32))
                        for r in range(m)])
    else:
        ref = g
    # RMSNorm-in rounds the normalised input to fp16 as the pre-pass does; with
    # it the fp32 output meets the fp16 bar (1 / rms may differ in the last bit)
    assert normwise(y.cpu().numpy().reshape(m, n), ref) <= (TOL if rms else TOL32)


@pytest.mark.parametrize("chunks", ["2", "3", "5", "64"])
@pytest.mark.parametrize("kernel,m", [("qmm", 16), ("qgemm", 48)])
def test_forced_chunk_counts(ctx, aexq, orc, monkeypatch, chunks, kernel, m):
    """Uneven chunkings (K steps not a multiple of the chunk count; more chunks
    asked for than there are steps) through AEXQ_SPLITK."""
    _announce(f"splitk forced {chunks} {kernel} m={m}")
    from aiimage_amd import synth
    monkeypatch.setenv("AEXQ_SPLITK", chunks)
    n, k = 640, 3584   # 14 wide steps; 56 GEMM steps of 64, 28 of 128
    w, wf = _weight(ctx, aexq, orc, 4, n, k, 31 + m)
    x16 = synth.activations(m, k, 32)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    plan = ctx.plan_check(w, xd, yd)
    steps = k // (256 if kernel == "qmm" else _kstep(plan))
    want = min(int(chunks), steps)
    cs = -(-steps // want)
    assert plan.startswith(f"kernel={kernel}") and _splitk(plan) == -(-steps // cs), plan
    ctx.linear(w, xd, yd)
    torch.cuda.synchronize()
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), for_plan(wf, plan))
    assert normwise(y.cpu().numpy().reshape(m, n), ref) <= TOL32


@pytest.mark.parametrize("bits,m", [(4, 16), (8, 32), (4, 64), (8, 200)])
def test_split_swiglu_rmsnorm(ctx, aexq, orc, bits, m):
    """gate/up with RMSNorm-in and SwiGLU-out: both halves' partials summed, then
    silu(gate) * up in the fix-up."""
    _announce(f"splitk swiglu q{bits} m={m}")
    from aiimage_amd import synth
    n, k, eps = 1024, 2048, 1e-6
    wg, gf = _weight(ctx, aexq, orc, bits, n, k, 41 + m)
    wu, uf = _weight(ctx, aexq, orc, bits, n, k, 42 + m)
    x16 = synth.activations(m, k, 43)
    gamma = synth.rms_gamma(k, 44)
    y = aexq.new_activation(m, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    kw = dict(rmsnorm=True, rms_gamma=dev(gamma), rms_eps=eps, up=wu)
    plan = ctx.plan_check(wg, xd, yd, **kw)
    assert "swiglu=1" in plan and _splitk(plan) > 1, plan
    ctx.linear(wg, xd, yd, **kw)
    torch.cuda.synchronize()
    xn = orc.rmsnorm(x16.astype(np.float32), eps, gamma).astype(np.float16).astype(np.float32)
    g = orc.gemm_gpu_semantics(xn, for_plan(gf, plan))
    u = orc.gemm_gpu_semantics(xn, for_plan(uf, plan))
    ref = np.stack([orc.swiglu(g[r].astype(np.float32), u[r].astype(np.float32)) for r in range(m)])
    got = y.cpu().numpy().astype(np.float64).reshape(m, -1)[:, :n]
    assert normwise(got, ref) <= TOL


@pytest.mark.parametrize("bcast,layout,m", [(1, "linear", 24), (3, "linear", 70), (4, "tiled", 16),
                                            (4, "tiled", 300)])
def test_split_bias_residual(ctx, aexq, orc, bcast, layout, m):
    """alpha/beta/C (per row, per element, per column) and the residual run in
    the fix-up, in both Gemm bias forms."""
    _announce(f"splitk bias bcast={bcast} layout={layout} m={m}")
    from aiimage_amd import synth
    n, k = 512, 2048
    w, wf = _weight(ctx, aexq, orc, 8, n, k, 51 + m, scale_f16=False)
    x16 = synth.activations(m, k, 52)
    rng = np.random.default_rng(53 + bcast)
    c = rng.standard_normal({1: m, 3: m * n, 4: n}[bcast]).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    lay = aexq.LAYOUT_PACK4_LINEAR if layout == "linear" else aexq.LAYOUT_PACK4_TILED
    y = aexq.new_activation(m, n, torch.float32, lay)
    stride = aexq.storage_elements(lay, m, n)
    rbuf = np.zeros((m, stride), np.float32)
    rbuf[:, :n] = res
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, lay)
    kw = dict(alpha=0.75, beta=1.5, c=dev(c), broadcast_c=bcast,
              residual=aexq.describe(dev(rbuf), m, n, lay))
    assert _splitk(ctx.plan_check(w, xd, yd, **kw)) > 1
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    s = orc.gemm_gpu_semantics(x16.astype(np.float32), wf)
    if bcast == 1:
        cc = np.repeat(c[:, None], n, 1)
    elif bcast == 3:
        cc = c.reshape(m, n)
    else:
        cc = np.repeat(c[None, :], m, 0)
    ref = (0.75 * (1.5 * cc + s) if layout == "linear" else 1.5 * cc + 0.75 * s) + res
    got = y.cpu().numpy().reshape(m, stride)[:, :n]
    assert normwise(got, ref) <= TOL32


@pytest.mark.parametrize("m", [16, 40])
def test_split_grouped_head_packed(ctx, aexq, orc, m):
    """A q/k/v group (three matrices' partial planes side by side) into
    attention head-packed outputs."""
    _announce(f"splitk qkv head-packed m={m}")
    from aiimage_amd import synth
    k, hd = 1024, 128
    shapes = [(2048, 16), (512, 4), (512, 4)]
    ws, refs, ys, yds = [], [], [], []
    x16 = synth.activations(m, k, 61)
    xd = aexq.describe(dev(x16), m, k)
    for i, (n, heads) in enumerate(shapes):
        w, wf = _weight(ctx, aexq, orc, 4, n, k, 62 + i)
        ws.append(w)
        y = aexq.new_activation(m, n, torch.float16, aexq.LAYOUT_HEAD_PACKED, head_dim=hd)
        ys.append(y)
        yds.append(aexq.describe(y, m, n, aexq.LAYOUT_HEAD_PACKED, head_dim=hd))
        plan = ctx.plan_check(w, xd, yds[-1])
        refs.append(orc.gemm_gpu_semantics(x16.astype(np.float32), for_plan(wf, plan)))
    ctx.linear_group(ws, xd, yds)
    torch.cuda.synchronize()
    for (n, heads), y, ref in zip(shapes, ys, refs):
        got = orc.head_unpack(y.cpu().numpy().astype(np.float32), m, heads, hd)
        assert normwise(got, ref) <= TOL


def test_batched_stack_keeps_whole_tiles(ctx, aexq, orc):
    """A stack with enough tiles to fill the part runs unsplit."""
    _announce("splitk batched stack unsplit")
    from aiimage_amd import synth
    n, k, m, copies = 1024, 2048, 16, 160
    w, _ = _weight(ctx, aexq, orc, 4, n, k, 71)
    st = w.replicate(copies)
    x = dev(synth.activations(m, k, 72))
    ys = torch.zeros(copies * m * n, dtype=torch.float16, device="cuda")
    plan = ctx.plan_check(st, aexq.describe(x, m, k),
                          aexq.describe(ys, m, n, aexq.LAYOUT_PACK4_LINEAR, batch=copies,
                                        batch_stride=m * n))
    assert _splitk(plan) == 1, plan
    st.release()


def test_split_graph_replays_match_eager(ctx, aexq, orc):
    """A layer's split launches (q/k/v group, gate/up pair, o_proj, down at M = 16
    and 64) captured in a HIP graph: every replay, with eager work between
    replays, equals the eager result bit for bit (the partial planes are fully
    rewritten by each launch; nothing is cleared with a memset node)."""
    _announce("splitk graph replays")
    from aiimage_amd import synth
    P4 = aexq.LAYOUT_PACK4_LINEAR
    ws = {}
    for i, (name, n, k) in enumerate(synth.LAYER_LINEARS):
        ws[name] = _weight(ctx, aexq, orc, 4, n, k, 101 + i)[0]
    gamma = dev(synth.rms_gamma(1024, 102))
    for m in (16, 64):
        xs = {k: dev(synth.activations(m, k, 103 + k)) for k in (1024, 2048, 3584)}
        xd = {k: aexq.describe(v, m, k) for k, v in xs.items()}
        ys = {name: torch.zeros(m * n, dtype=torch.float16, device="cuda")
              for name, n, _ in synth.LAYER_LINEARS}
        yd = {name: aexq.describe(ys[name], m, n, P4) for name, n, _ in synth.LAYER_LINEARS}

        def step():
            ctx.linear_group([ws["q_proj"], ws["k_proj"], ws["v_proj"]], xd[1024],
                             [yd["q_proj"], yd["k_proj"], yd["v_proj"]],
                             rmsnorm=True, rms_gamma=gamma, rms_eps=1e-6)
            ctx.linear(ws["gate_proj"], xd[1024], yd["gate_proj"], rmsnorm=True,
                       rms_gamma=gamma, rms_eps=1e-6, up=ws["up_proj"])
            ctx.linear(ws["o_proj"], xd[2048], yd["o_proj"])
            ctx.linear(ws["down_proj"], xd[3584], yd["down_proj"])

        assert _splitk(ctx.plan_check(ws["down_proj"], xd[3584], yd["down_proj"])) > 1
        step()
        torch.cuda.synchronize()
        eager = {k: v.clone() for k, v in ys.items()}
        stream = torch.cuda.Stream()
        ctx.set_stream(stream)
        try:
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                step()
            stream.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                step()
        finally:
            ctx.set_stream(torch.cuda.current_stream())
        for rep in range(3):
            for v in ys.values():
                v.zero_()
            # eager work between replays: another launch through the same scratch
            other = torch.zeros(m * 1024, dtype=torch.float16, device="cuda")
            ctx.linear(ws["o_proj"], xd[2048], aexq.describe(other, m, 1024, P4))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            for name in ys:
                assert torch.equal(ys[name], eager[name]), (m, rep, name)
        del g


@pytest.mark.parametrize("bits,m,pair,group", [
    (4, 16, False, False), (4, 9, True, False), (8, 24, False, False), (8, 32, True, False),
    (4, 16, False, True),   # a q/k/v group sharing one normalised input
])
def test_rmsnorm_in_kernel(ctx, aexq, orc, monkeypatch, bits, m, pair, group):
    """RMSNorm-in inside the wide kernel (launches with one item per workgroup):
    no pre-pass launch, the oracle's RMSNorm -> fp16 -> Gemm within the fp16 bar,
    and the pre-pass path's result within one fp16 rounding of the inputs."""
    _announce(f"rmsnorm in-kernel q{bits} m={m} pair={pair} group={group}")
    from aiimage_amd import synth
    k, eps = 1024, 1e-6
    shapes = [2048, 512, 512] if group else [1024]
    ws, wfs = [], []
    for i, n in enumerate(shapes):
        w, wf = _weight(ctx, aexq, orc, bits, n, k, 121 + i + m)
        ws.append(w)
        wfs.append(wf)
    kw = dict(rmsnorm=True, rms_gamma=dev(synth.rms_gamma(k, 122)), rms_eps=eps)
    if pair:
        wu, uf = _weight(ctx, aexq, orc, bits, shapes[0], k, 123 + m)
        kw["up"] = wu
    x16 = synth.activations(m, k, 124)
    xd = aexq.describe(dev(x16), m, k)
    P4 = aexq.LAYOUT_PACK4_LINEAR

    def run():
        ys = [aexq.new_activation(m, n, torch.float16, P4) for n in shapes]
        yds = [aexq.describe(y, m, n, P4) for y, n in zip(ys, shapes)]
        if group:
            ctx.linear_group(ws, xd, yds, **kw)
        else:
            ctx.linear(ws[0], xd, yds[0], **kw)
        torch.cuda.synchronize()
        return ys, ctx.plan_check(ws[0], xd, yds[0], **kw)

    ys, plan = run()
    assert "wide=1" in plan and "rms_prepass=0" in plan, plan
    monkeypatch.setenv("AEXQ_RMS_PREPASS", "1")
    ys_pre, plan_pre = run()
    assert "rms_prepass=1" in plan_pre, plan_pre
    xn = orc.rmsnorm(x16.astype(np.float32), eps, synth.rms_gamma(k, 122))
    xn = xn.astype(np.float16).astype(np.float32)
    for y, yp, wf, n in zip(ys, ys_pre, wfs, shapes):
        g = orc.gemm_gpu_semantics(xn, for_plan(wf, plan))
        if pair:
            u = orc.gemm_gpu_semantics(xn, for_plan(uf, plan))
            ref = np.stack([orc.swiglu(g[r].astype(np.float32), u[r].astype(np.float32))
                            for r in range(m)])
        else:
            ref = g
        got = y.cpu().numpy().astype(np.float64).reshape(m, n)
        assert normwise(got, ref) <= TOL
        assert normwise(got, yp.cpu().numpy().astype(np.float64).reshape(m, n)) <= TOL
