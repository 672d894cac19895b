"""GPU parity of the attention head-packed layout (MM:1192-1389) through the C
ABI: q/k/v outputs stored head-packed by every kernel family (streaming M = 1
and M <= 8, the MFMA blocks, the tiled GEMM, the generic kernel) and o_proj
reading a head-packed input, against the oracle's restatement of the layout
(orc.head_pack / head_unpack) around its float64 Gemm.

Bars as in the other parity tests: normwise <= 1e-3 for fp16 outputs and
1e-5 for fp32 outputs; the lanes of heads past the last one are exactly 0.
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


def dev(a):
    return torch.as_tensor(np.ascontiguousarray(a)).cuda()


def _q4(ctx, aexq, orc, n, k, seed):
    from aiimage_amd import synth
    words, scales, _ = synth.q4_weights(n, k, seed, group=32, code=synth.NIBBLE_OFFSET8)
    w = ctx.weight(aexq.QuantizedTensor(n * k, 32, words, scales, bits=4,
                                        nibble_code=synth.NIBBLE_OFFSET8), n, k)
    return w, q4_reference(orc, words, scales, n, k, 32, synth.NIBBLE_OFFSET8, True)


def test_qkv_group_head_packed_m1_rmsnorm(ctx, aexq, orc):
    """The decode q/k/v group (16 q heads, 4 k/v heads of 128) at M = 1 with
    RMSNorm-in, every output head-packed, on the streaming kernel."""
    _announce("qkv head-packed m=1")
    from aiimage_amd import synth
    k, hd, eps = 1024, 128, 1e-6
    shapes = [("q", 16), ("k", 4), ("v", 4)]
    ws, wfs, ys, yds = [], [], [], []
    for i, (_, heads) in enumerate(shapes):
        w, wf = _q4(ctx, aexq, orc, heads * hd, k, 300 + i)
        y = aexq.new_activation(1, heads * hd, torch.float16, aexq.LAYOUT_HEAD_PACKED, head_dim=hd)
        ws.append(w), wfs.append(wf), ys.append(y)
        yds.append(aexq.describe(y, 1, heads * hd, aexq.LAYOUT_HEAD_PACKED, head_dim=hd))
    x16 = synth.activations(1, k, 310)
    gamma = synth.rms_gamma(k, 311)
    xd = aexq.describe(dev(x16), 1, k)
    kw = dict(rmsnorm=True, rms_gamma=dev(gamma), rms_eps=eps)
    assert ctx.plan_check(ws[0], xd, yds[0], **kw).startswith("kernel=qmv")
    ctx.linear_group(ws, xd, yds, **kw)
    torch.cuda.synchronize()
    xn = orc.rmsnorm(x16.astype(np.float32), eps, gamma).astype(np.float16).astype(np.float32)
    for (name, heads), wf, y in zip(shapes, wfs, ys):
        ref = orc.head_pack(orc.gemm_gpu_semantics(xn, wf.exact).astype(np.float32), heads, hd)
        assert normwise(y.cpu().numpy(), ref) <= TOL, name


@pytest.mark.parametrize("m,k,y32,kernel", [
    (5, 1056, False, "qmv"),      # streaming, M <= 8 (K = 33 chunks keeps it off the MFMA path)
    (20, 1024, False, "qmm"),     # MFMA 32-row blocks
    (70, 1024, True, "qgemm"),    # tiled GEMM, two 64-row tiles
    (40, 1024, True, "qmm"),      # MFMA over two row blocks (tiled GEMM switched off)
    (3, 40, True, "generic"),     # K not a whole 32-code chunk: the generic kernel
])
def test_head_packed_output_families(ctx, aexq, orc, monkeypatch, m, k, y32, kernel):
    """6 heads of 64 (the second slice holds two heads): every kernel family
    writes the layout, lanes of heads 6 and 7 stay 0."""
    _announce(f"head-packed y m={m} k={k} kernel={kernel}")
    from aiimage_amd import synth
    if kernel == "qmm" and m > 32:
        monkeypatch.setenv("AEXQ_QGEMM_OFF", "1")
    heads, hd = 6, 64
    n = heads * hd
    if k % 32:
        words, scales, _ = synth.q8_weights(n, k, 320 + m)
        w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
        wf = orc.dequant_q8(words, scales, n, k)
    else:
        w, wf = _q4(ctx, aexq, orc, n, k, 320 + m)
    x16 = synth.activations(m, k, 321)
    ydt = torch.float32 if y32 else torch.float16
    y = aexq.new_activation(m, n, ydt, aexq.LAYOUT_HEAD_PACKED, head_dim=hd)
    y.fill_(7.0)   # the zero lanes must be written, not left over
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_HEAD_PACKED, head_dim=hd)
    plan = ctx.plan_check(w, xd, yd)
    assert plan.startswith(f"kernel={kernel}"), plan
    ctx.linear(w, xd, yd, alpha=0.5)
    torch.cuda.synchronize()
    got = y.cpu().numpy().astype(np.float64)
    ref = orc.head_pack((0.5 * orc.gemm_gpu_semantics(x16.astype(np.float32),
                                                      for_plan(wf, plan))).astype(np.float32),
                        heads, hd)
    tail = got.reshape(2, m, hd, 4)[1, :, :, 2:]
    assert np.all(tail == 0)
    assert normwise(got, ref) <= (TOL32 if y32 else TOL)


@pytest.mark.parametrize("m,heads,hd,xdt", [(1, 16, 128, np.float16), (40, 16, 128, np.float16),
                                            (3, 6, 64, np.float32)])
def test_head_packed_input_o_proj(ctx, aexq, orc, m, heads, hd, xdt):
    """o_proj reading the SDPA context in the head-packed layout (MM:1320-1389)."""
    _announce(f"head-packed x m={m} heads={heads}")
    from aiimage_amd import synth
    k = heads * hd
    n = 1024
    w, wf = _q4(ctx, aexq, orc, n, k, 330 + m)
    xl = synth.activations(m, k, 331).astype(np.float32)
    xhp = orc.head_pack(xl, heads, hd).astype(xdt)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(xhp), m, k, aexq.LAYOUT_HEAD_PACKED, head_dim=hd)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    plan = ctx.plan_check(w, xd, yd)
    ctx.linear(w, xd, yd)
    torch.cuda.synchronize()
    xr = orc.head_unpack(xhp.astype(np.float32), m, heads, hd)
    ref = orc.gemm_gpu_semantics(xr, for_plan(wf, plan))
    assert normwise(y.cpu().numpy().reshape(m, n), ref) <= TOL32


def test_head_packed_rejections(ctx, aexq, orc):
    _announce("head-packed rejections")
    from aiimage_amd import _abi, synth
    heads, hd, k = 4, 64, 256
    n = heads * hd
    w, _ = _q4(ctx, aexq, orc, n, k, 340)
    x = dev(synth.activations(1, k, 341))
    y = aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_HEAD_PACKED, head_dim=hd)
    yd = aexq.describe(y, 1, n, aexq.LAYOUT_HEAD_PACKED, head_dim=hd)
    with pytest.raises(_abi.NotSupportedError):   # residual add into head-packed y
        ctx.linear(w, aexq.describe(x, 1, k), yd, residual=yd)
    xhp = aexq.new_activation(1, k, torch.float16, aexq.LAYOUT_HEAD_PACKED, head_dim=hd)
    with pytest.raises(_abi.NotSupportedError):   # LM head over a head-packed x
        ctx.lmhead_argmax(w, aexq.describe(xhp, 1, k, aexq.LAYOUT_HEAD_PACKED, head_dim=hd), None,
                          torch.zeros(1, dtype=torch.int32, device="cuda"))
