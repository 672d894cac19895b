"""GPU parity of libaexq.so against the CPU oracle, through the C ABI.

Bars (from the benchmark definition): dequantized weights bit-exact with the
reference unpack; outputs within max|y - r| / max|r| <= 1e-3 of the float64
oracle; greedy argmax equal except where the oracle's top-2 gap < 1e-3.
"""
import ctypes
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL = 1e-3          # normwise relative error bar for fp16/fp32 outputs
ARGMAX_TIE = 1e-3   # near-tie window for argmax agreement


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


# ------------------------------------------------------------------ dequant

@pytest.mark.parametrize("scale_f16", [False, True])
@pytest.mark.parametrize("k", [1024, 40])
def test_dequant_q8_bit_exact(ctx, aexq, orc, scale_f16, k):
    from aiimage_amd import synth
    _announce(f"dequant q8 k={k} f16={scale_f16}")
    n = 96
    words, scales, codes = synth.q8_weights(n, k, seed=11, scale_dtype=np.float16 if scale_f16 else np.float32)
    # every byte value appears: overwrite the first rows with the 255 codes that exist
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    got = ctx.dequant(w).cpu().numpy()
    want = orc.dequant_q8(words, scales, n, k,
                          scale_dtype=orc.SCALE_F16 if scale_f16 else orc.SCALE_F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_q8_all_codes_and_subnormal_scales(ctx, aexq, orc):
    _announce("dequant q8 all codes")
    n, k = 4, 256
    codes = np.tile(np.arange(-128, 128, dtype=np.int16).astype(np.int8), (n, 1))
    words = codes.reshape(-1).view(np.uint32).copy()
    scales = np.array([1, 0x03FF, 0x0400, 0x3C00], np.uint16).view(np.float16)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    got = ctx.dequant(w).cpu().numpy()
    want = orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F16)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert got[0, 129] == 2.0 ** -24      # code 1 times the smallest subnormal


@pytest.mark.parametrize("code", [0, 1])
@pytest.mark.parametrize("group,scale_f16", [(16, False), (32, True), (64, True), (1024, False)])
def test_dequant_q4_bit_exact(ctx, aexq, orc, code, group, scale_f16):
    _announce(f"dequant q4 code={code} group={group}")
    n, k = 64, 1024
    rng = np.random.default_rng(group + code)
    nib = rng.integers(0, 16, n * k, dtype=np.uint8)     # every 4-bit pattern, both codes
    words = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8).view(np.uint32).copy()
    sdt = np.float16 if scale_f16 else np.float32
    scales = (rng.standard_normal(n * k // group) * 0.003).astype(sdt)
    qt = aexq.QuantizedTensor(n * k, group, words, scales, bits=4, nibble_code=code)
    got = ctx.dequant(ctx.weight(qt, n, k)).cpu().numpy()
    want = orc.dequant_q4(words, scales, n, k, group, nibble_code=code,
                          scale_dtype=orc.SCALE_F16 if scale_f16 else orc.SCALE_F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_q4_ragged_k_generic(ctx, aexq, orc):
    _announce("dequant q4 ragged k")
    n, k, group = 5, 48, 16          # K not a multiple of 32: element-wise path
    rng = np.random.default_rng(3)
    q = rng.integers(-7, 8, (n, k)).astype(np.int8)
    from aiimage_amd import synth
    words = synth.pack_nibbles(q, 0)
    scales = rng.random(n * k // group).astype(np.float32)
    got = ctx.dequant(ctx.weight(aexq.QuantizedTensor(n * k, group, words, scales, bits=4), n, k))
    want = orc.dequant_q4(words, scales, n, k, group, nibble_code=0)
    assert np.array_equal(got.cpu().numpy(), want)


# ------------------------------------------------------------------ Q8 matvec

def _q8_case(ctx, aexq, orc, n, k, m, seed, scale_f16=True, layout=None):
    from aiimage_amd import synth
    words, scales, _ = synth.q8_weights(n, k, seed, scale_dtype=np.float16 if scale_f16 else np.float32)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    x16 = synth.activations(m, k, seed + 1)
    layout = aexq.output_layout_for(n) if layout is None else layout
    y = aexq.new_activation(m, n, torch.float16, layout)
    xd = dev(x16)
    ctx.linear(w, aexq.describe(xd, m, k), aexq.describe(y, m, n, layout))
    torch.cuda.synchronize()
    stride = aexq.storage_elements(layout, m, n)
    ys = y.cpu().numpy().astype(np.float32).reshape(m, stride)
    wf = orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F16 if scale_f16 else orc.SCALE_F32)
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), wf)
    return ys, ref, stride


def test_q8_matvec_config1(ctx, aexq, orc):
    """Benchmark config 1: Q8, M=1, K=1024, N=3584, per-row fp16 scales."""
    _announce("q8 matvec config1")
    ys, ref, _ = _q8_case(ctx, aexq, orc, 3584, 1024, 1, seed=0xAE0C0F11)
    err = normwise(ys[:, :3584], ref)
    assert err <= TOL, err
    # fp16 output rounding dominates: every element within a few fp16 ulps
    assert np.all(np.abs(ys[:, :3584] - ref) <= np.abs(ref) * 2.0 ** -10 + np.max(np.abs(ref)) * 1e-5)


@pytest.mark.parametrize("n,k,m", [(1024, 2048, 1), (1024, 3584, 1), (512, 1024, 3),
                                   (3584, 1024, 8), (100, 256, 1), (37, 512, 2), (6, 16, 1)])
def test_q8_matvec_shapes(ctx, aexq, orc, n, k, m):
    _announce(f"q8 matvec n={n} k={k} m={m}")
    ys, ref, stride = _q8_case(ctx, aexq, orc, n, k, m, seed=n + k + m, scale_f16=(n % 2 == 0))
    assert normwise(ys[:, :n], ref) <= TOL
    if stride > n:
        assert np.all(ys[:, n:] == 0)     # Pack4 tail lanes are zero


# ------------------------------------------------------------------ Q4 layer (config 2)

def _q4_weight(ctx, aexq, n, k, seed, group=32, code=1, scale_f16=True):
    from aiimage_amd import synth
    words, scales, _ = synth.q4_weights(n, k, seed, group=group, code=code,
                                        scale_dtype=np.float16 if scale_f16 else np.float32)
    qt = aexq.QuantizedTensor(n * k, group, words, scales, bits=4, nibble_code=code)
    return ctx.weight(qt, n, k), words, scales


def _q4_ref(orc, words, scales, n, k, group, code, scale_f16, x):
    wf = orc.dequant_q4(words, scales, n, k, group, nibble_code=code,
                        scale_dtype=orc.SCALE_F16 if scale_f16 else orc.SCALE_F32)
    return orc.gemm_gpu_semantics(np.asarray(x, np.float32), wf)


def test_q4_layer_config2(ctx, aexq, orc):
    """Benchmark config 2: one decoder layer's seven Q4 linears at M=1, with the
    fused RMSNorm-in (q/k/v, gate/up) and SwiGLU-out (gate/up) epilogues."""
    from aiimage_amd import synth
    seed = 0xAE0C0F12
    eps = 1e-6
    x16 = synth.activations(1, 1024, seed)
    gamma = synth.rms_gamma(1024, seed + 1)
    xn = orc.rmsnorm(x16.astype(np.float32), eps, gamma).astype(np.float16).astype(np.float32)
    xd, gd = dev(x16), dev(gamma)
    outs = {}
    for i, (name, n, k) in enumerate(synth.LAYER_LINEARS):
        if name in ("gate_proj", "up_proj"):
            continue
        _announce(f"q4 layer {name}")
        w, words, scales = _q4_weight(ctx, aexq, n, k, seed + 10 + i)
        if k == 1024:
            xin, xdesc = xn, aexq.describe(xd, 1, k)
            kw = dict(rmsnorm=True, rms_gamma=gd, rms_eps=eps)
        else:
            xk = synth.activations(1, k, seed + 20 + i)
            xin, xdesc, kw = xk.astype(np.float32), aexq.describe(dev(xk), 1, k), {}
        y = aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
        ctx.linear(w, xdesc, aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR), **kw)
        torch.cuda.synchronize()
        ref = _q4_ref(orc, words, scales, n, k, 32, 1, True, xin)
        outs[name] = normwise(y.cpu().numpy()[None, :n], ref)
    _announce("q4 layer gate/up swiglu")
    n, k = 3584, 1024
    wg, gw, gs = _q4_weight(ctx, aexq, n, k, seed + 14)
    wu, uw, us = _q4_weight(ctx, aexq, n, k, seed + 15)
    y = aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    ctx.linear(wg, aexq.describe(xd, 1, k), aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR),
               rmsnorm=True, rms_gamma=gd, rms_eps=eps, up=wu)
    torch.cuda.synchronize()
    g = _q4_ref(orc, gw, gs, n, k, 32, 1, True, xn)
    u = _q4_ref(orc, uw, us, n, k, 32, 1, True, xn)
    ref = orc.swiglu(g.astype(np.float32), u.astype(np.float32))
    outs["swiglu"] = normwise(y.cpu().numpy()[:n], ref)
    assert all(v <= TOL for v in outs.values()), outs


@pytest.mark.parametrize("group,scale_f16", [(16, False), (32, False), (1024, False), (64, True)])
def test_q4_reference_format_twos_complement(ctx, aexq, orc, group, scale_f16):
    """The reference's shipping Q4: two's-complement nibbles, fp32 scales, group 16."""
    _announce(f"q4 twos group={group}")
    from aiimage_amd import synth
    n, k, m = 2048, 1024, 1
    w, words, scales = _q4_weight(ctx, aexq, n, k, 77 + group, group=group, code=0,
                                  scale_f16=scale_f16)
    x16 = synth.activations(m, k, 78)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    ctx.linear(w, aexq.describe(dev(x16), m, k), aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR))
    torch.cuda.synchronize()
    ref = _q4_ref(orc, words, scales, n, k, group, 0, scale_f16, x16.astype(np.float32))
    assert normwise(y.cpu().numpy()[None, :n], ref) <= 1e-5    # fp32 output: tighter


def test_q4_from_q8_rows_archive_pipeline(ctx, aexq, orc):
    """Q8 archive -> WriteQ4FromQ8Rows (group 16) -> ReadQ4PackedArray -> GPU linear."""
    _announce("q4 from q8 rows archive")
    rng = np.random.default_rng(21)
    n, k = 512, 1024
    wf = rng.standard_normal((n, k)).astype(np.float32) * 0.05
    q8, s8 = orc.q8_pack_rows(wf, n, k)
    rec = orc.record_write_q4_from_q8_rows(q8, s8, n, k, 16)
    rc, packed, scales, blk, _ = orc.record_read_q4_packed(rec, n * k, 16)
    assert rc == 0
    w = ctx.weight(aexq.QuantizedTensor(n * k, blk, packed, scales, bits=4), n, k)
    x16 = rng.standard_normal((2, k)).astype(np.float16)
    y = aexq.new_activation(2, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    ctx.linear(w, aexq.describe(dev(x16), 2, k), aexq.describe(y, 2, n, aexq.LAYOUT_PACK4_LINEAR))
    torch.cuda.synchronize()
    ref = _q4_ref(orc, packed, scales, n, k, 16, 0, False, x16.astype(np.float32))
    assert normwise(y.cpu().numpy().reshape(2, n), ref) <= 1e-5


# ------------------------------------------------------------------ Gemm semantics / KATs

def test_reference_gemm_kat_int8(ctx, aexq, orc):
    """NcnnInt8WeightOnlyGpuTests Gemm KAT: M=1, K=4, N=2, bias per column, tol 1e-5."""
    _announce("gemm kat int8")
    import json, os
    kat = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                      "reference_kats.json")))["q8_gemm_kernel"]
    layer = aexq.HipGemmLayer(ctx, "gemm_0").load_layer(
        {0: 1.0, 1: 1.0, 3: 1, 5: 1, 6: 1, 7: 1, 8: 2, 9: 4, 10: 4},
        np.array(kat["weights"], np.float32), bias=np.array(kat["bias"], np.float32))
    x = dev(np.array([kat["input"]], np.float32))
    y = aexq.new_activation(1, 2, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    ctx.linear(layer.weight, aexq.describe(x, 1, 4), aexq.describe(y, 1, 2, aexq.LAYOUT_PACK4_LINEAR),
               c=layer.c, broadcast_c=4)
    torch.cuda.synchronize()
    packed, scales = orc.q8_pack_rows(kat["weights"], 2, 4)
    ref = orc.gemm_gpu_semantics(np.array([kat["input"]], np.float32),
                                 orc.dequant_q8(packed, scales, 2, 4), 1.0, 1.0,
                                 np.array(kat["bias"], np.float32), 4)
    got = y.cpu().numpy()[:2]
    assert np.all(np.abs(got - ref[0]) <= kat["tolerance"]), (got, ref)
    # the float upload packs exactly like the oracle packer (GS:12838-12885)
    deq = ctx.dequant(layer.weight).cpu().numpy()
    assert np.array_equal(deq, orc.dequant_q8(packed, scales, 2, 4))


@pytest.mark.parametrize("bcast", [0, 1, 3, 4])
@pytest.mark.parametrize("layout", [1, 2])
def test_alpha_beta_bias_semantics(ctx, aexq, orc, bcast, layout):
    """Pack4 linear: alpha*(beta*C + sum) (MM:1101); tiled: beta*C + alpha*sum (MM:2301)."""
    _announce(f"bias bcast={bcast} layout={layout}")
    from aiimage_amd import synth
    n, k, m = 256, 512, 2
    words, scales, _ = synth.q8_weights(n, k, 5, scale_dtype=np.float32)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    rng = np.random.default_rng(bcast)
    csz = {0: 1, 1: m, 3: m * n, 4: n}[bcast]
    c = rng.standard_normal(csz).astype(np.float32)
    x16 = synth.activations(m, k, 6)
    y = aexq.new_activation(m, n, torch.float32, layout)
    ctx.linear(w, aexq.describe(dev(x16), m, k), aexq.describe(y, m, n, layout), alpha=0.5,
               beta=2.0, c=dev(c), broadcast_c=bcast)
    torch.cuda.synchronize()
    stride = aexq.storage_elements(layout, m, n)
    got = y.cpu().numpy().reshape(m, stride)[:, :n]
    wf = orc.dequant_q8(words, scales, n, k)
    s = orc.gemm_gpu_semantics(x16.astype(np.float32), wf)
    cc = {0: lambda: np.full((m, n), c[0]), 1: lambda: np.repeat(c[:, None], n, 1),
          3: lambda: c.reshape(m, n), 4: lambda: np.repeat(c[None, :], m, 0)}[bcast]()
    ref = 0.5 * (2.0 * cc + s) if layout == 1 else 2.0 * cc + 0.5 * s
    assert normwise(got, ref) <= 1e-5


def test_residual_add_epilogue(ctx, aexq, orc):
    _announce("residual add")
    from aiimage_amd import synth
    n, k = 1024, 2048
    w, words, scales = _q4_weight(ctx, aexq, n, k, 91)
    x16 = synth.activations(1, k, 92)
    res = synth.activations(1, n, 93)
    y = aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    rd = dev(res)
    ctx.linear(w, aexq.describe(dev(x16), 1, k), aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR),
               residual=aexq.describe(rd, 1, n, aexq.LAYOUT_PACK4_LINEAR))
    torch.cuda.synchronize()
    ref = _q4_ref(orc, words, scales, n, k, 32, 1, True, x16.astype(np.float32)) + res.astype(np.float64)
    assert normwise(y.cpu().numpy()[None, :n], ref) <= TOL


def test_generic_path_fp32_activations_and_ragged_k(ctx, aexq, orc):
    _announce("generic fp32 x ragged k")
    rng = np.random.default_rng(8)
    n, k, m = 33, 20, 17          # K=20: no 16-byte chunks; M=17: two row blocks
    wf = rng.standard_normal((n, k)).astype(np.float32)
    w = ctx.weight_from_float(wf, n, k, bits=8)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_LINEAR)
    plan = ctx.plan_check(w, aexq.describe(dev(x), m, k), aexq.describe(y, m, n))
    assert plan.startswith("kernel=generic")
    ctx.linear(w, aexq.describe(dev(x), m, k), aexq.describe(y, m, n))
    torch.cuda.synchronize()
    packed, scales = orc.q8_pack_rows(wf, n, k)
    ref = orc.gemm_gpu_semantics(x, orc.dequant_q8(packed, scales, n, k))
    assert normwise(y.cpu().numpy().reshape(m, n), ref) <= 1e-5


def test_float_upload_transposed_source(ctx, aexq, orc):
    """outputChannelsAreContiguous=false: a [K][N] source packs to the same codes."""
    _announce("float upload transB=0")
    rng = np.random.default_rng(12)
    n, k = 64, 128
    wf = rng.standard_normal((n, k)).astype(np.float32)
    a = ctx.dequant(ctx.weight_from_float(wf, n, k, bits=4, trans_b=True)).cpu().numpy()
    b = ctx.dequant(ctx.weight_from_float(wf.T.copy(), n, k, bits=4, trans_b=False)).cpu().numpy()
    assert np.array_equal(a, b)
    p4, s4, blk = orc.q4_pack_rows(wf, n, k)
    assert np.array_equal(a, orc.dequant_q4(p4, s4, n, k, blk, nibble_code=0))


def test_strict_plan_rejects_without_fallback(ctx, aexq):
    _announce("strict plan")
    from aiimage_amd import _abi, synth
    n, k = 256, 1024
    words, scales, _ = synth.q8_weights(n, k, 1)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    x = dev(synth.activations(1, k, 2))
    y = aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(x, 1, k)
    yd = aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR)
    assert ctx.plan_check(w, xd, yd).startswith("kernel=qmv")
    bad = aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR)
    bad.layout = _abi.LAYOUT_HEAD_PACKED
    bad.storage = _abi.Shape(3, 48, 1, 1, 4)     # 4 heads of 48 do not make width 256
    with pytest.raises(_abi.InvalidOperationError):
        ctx.linear(w, xd, bad)
    with pytest.raises(_abi.InvalidOperationError):
        ctx.linear(w, aexq.describe(x, 1, k), aexq.describe(y, 1, n // 2, aexq.LAYOUT_PACK4_LINEAR))
    with pytest.raises(_abi.NotSupportedError):   # SwiGLU with a bias term
        ctx.linear(w, xd, yd, up=w, c=dev(np.zeros(n, np.float32)), broadcast_c=4)
    with pytest.raises(_abi.ArgumentError):       # Q8 direct upload with block != K
        ctx.weight(aexq.QuantizedTensor(n * k, 256, words, scales, bits=8), n, k)
    assert "one scale per output channel" in _abi.last_error()
    # empty matrices (no rows, no columns) are refused before anything launches
    no_rows = aexq.describe(x, 1, k)
    no_rows.logical = _abi.Shape(2, k, 0, 1, 1)
    no_cols = aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR)
    no_cols.logical = _abi.Shape(2, 0, 1, 1, 1)
    am = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    for call in (lambda: ctx.linear(w, no_rows, yd), lambda: ctx.linear(w, xd, no_cols),
                 lambda: ctx.lmhead_argmax(w, no_rows, None, am),
                 lambda: ctx.argmax(no_cols, am)):
        with pytest.raises(_abi.InvalidOperationError):
            call()
        assert "is empty" in _abi.last_error()
    torch.cuda.synchronize()
    assert int(am.item()) == -7


# ------------------------------------------------------------------ LM head + argmax

@pytest.mark.parametrize("m", [1, 8])
def test_lmhead_argmax_full_vocab(ctx, aexq, orc, m):
    """Config 5: Q8 per-row LM head K=1024, N=151,936, fp32 logits, fused argmax."""
    _announce(f"lm head m={m}")
    from aiimage_amd import synth
    n, k = synth.VOCAB, synth.HIDDEN
    words, scales, _ = synth.q8_weights(n, k, 0xAE0C0F15)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    x16 = synth.activations(m, k, 0xAE0C0F16)
    layout = aexq.LAYOUT_PACK4_TILED
    logits = aexq.new_activation(m, n, torch.float32, layout)
    am = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    gap = torch.zeros(m, dtype=torch.float32, device="cuda")
    ctx.lmhead_argmax(w, aexq.describe(dev(x16), m, k), aexq.describe(logits, m, n, layout), am, gap)
    torch.cuda.synchronize()
    stride = aexq.storage_elements(layout, m, n)
    got = logits.cpu().numpy().reshape(m, stride)[:, :n]
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32),
                                 orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F16))
    assert normwise(got, ref) <= 1e-5
    ref_idx = orc.argmax_rows(ref.astype(np.float32))
    srt = np.sort(ref, axis=1)
    ref_gap = srt[:, -1] - srt[:, -2]
    gi = am.cpu().numpy()
    for r in range(m):
        if ref_gap[r] >= ARGMAX_TIE:
            assert gi[r] == ref_idx[r], (r, gi[r], ref_idx[r])
    np.testing.assert_allclose(gap.cpu().numpy(), ref_gap, atol=1e-5)
    # logits-free call gives the same indices
    am2 = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    ctx.lmhead_argmax(w, aexq.describe(dev(x16), m, k), None, am2)
    torch.cuda.synchronize()
    assert np.array_equal(am2.cpu().numpy(), gi)


@pytest.mark.parametrize("m,n", [(1, 151936), (4, 30011)])
def test_lmhead_argmax_rmsnorm_in(ctx, aexq, orc, m, n):
    """aexq_lmhead_argmax_ex: the final RMSNorm fused into the LM head launch.
    Logits and indices against the oracle of rmsnorm -> fp16 -> Q8 matvec, and
    the indices equal to those of the unfused rmsnorm + LM head; epilogues other
    than RMSNorm-in are refused."""
    _announce(f"lm head rmsnorm-in m={m} n={n}")
    from aiimage_amd import synth
    k, eps = synth.HIDDEN, 1e-6
    words, scales, _ = synth.q8_weights(n, k, 0xAE0C0F31 + m)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    x16 = synth.activations(m, k, 0xAE0C0F32 + m)
    gamma = synth.rms_gamma(k, 0xAE0C0F33)
    gd, xdev = dev(gamma), dev(x16)
    xd = aexq.describe(xdev, m, k)
    layout = aexq.LAYOUT_PACK4_LINEAR
    logits = aexq.new_activation(m, n, torch.float32, layout)
    am = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    gap = torch.zeros(m, dtype=torch.float32, device="cuda")
    ctx.lmhead_argmax(w, xd, aexq.describe(logits, m, n, layout), am, gap,
                      rmsnorm=True, rms_gamma=gd, rms_eps=eps)
    torch.cuda.synchronize()
    xn = orc.rmsnorm(x16.astype(np.float32), eps, gamma).astype(np.float16).astype(np.float32)
    ref = orc.gemm_gpu_semantics(xn, orc.dequant_q8(words, scales, n, k,
                                                    scale_dtype=orc.SCALE_F16))
    stride = aexq.storage_elements(layout, m, n)
    assert normwise(logits.cpu().numpy().reshape(m, stride)[:, :n], ref) <= 1e-3
    ref_idx = orc.argmax_rows(ref.astype(np.float32))
    srt = np.sort(ref, axis=1)
    ref_gap = srt[:, -1] - srt[:, -2]
    gi = am.cpu().numpy()
    for r in range(m):
        if ref_gap[r] >= ARGMAX_TIE:
            assert gi[r] == ref_idx[r], (r, gi[r], ref_idx[r])
    # the unfused form: aexq_rmsnorm into fp16, then the plain LM head
    xn_dev = torch.zeros(m * k, dtype=torch.float16, device="cuda")
    ctx.rmsnorm(xd, aexq.describe(xn_dev, m, k), gd, eps)
    am2 = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    ctx.lmhead_argmax(w, aexq.describe(xn_dev, m, k), None, am2)
    torch.cuda.synchronize()
    for r in range(m):
        if ref_gap[r] >= ARGMAX_TIE:
            assert int(am2[r]) == gi[r], r
    with pytest.raises(aexq.NotSupportedError):
        args = aexq.make_args(rms_gamma=gd, rms_eps=eps, rmsnorm=True, residual=xd)
        aexq.check(ctx._lib.aexq_lmhead_argmax_ex(
            ctx.handle, w.handle, ctypes.byref(xd), None, ctypes.byref(args),
            ctypes.c_void_p(am.data_ptr()), None), "aexq_lmhead_argmax_ex")


@pytest.mark.parametrize("bits,m,n", [(8, 20, 50000), (8, 40, 30011), (4, 8, 40000), (4, 24, 20000)])
def test_lmhead_argmax_mfma_rows(ctx, aexq, orc, bits, m, n):
    """LM heads of 2..32 rows per launch take the wide MFMA kernel with the argmax
    partials fused (M = 40: two launches whose partials land in their own rows);
    logits, indices and top-2 gaps against the oracle."""
    _announce(f"lm head mfma q{bits} m={m} n={n}")
    from aiimage_amd import synth
    k = synth.HIDDEN
    if bits == 8:
        words, scales, _ = synth.q8_weights(n, k, 0xAE0C0F25 + m)
        w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
        wf = orc.dequant_q8(words, scales, n, k, scale_dtype=orc.SCALE_F16)
    else:
        words, scales, _ = synth.q4_weights(n, k, 0xAE0C0F25 + m, group=32, code=synth.NIBBLE_OFFSET8)
        w = ctx.weight(aexq.QuantizedTensor(n * k, 32, words, scales, bits=4,
                                            nibble_code=synth.NIBBLE_OFFSET8), n, k)
        wf = orc.dequant_q4(words, scales, n, k, 32, synth.NIBBLE_OFFSET8, orc.SCALE_F16)
    x16 = synth.activations(m, k, 0xAE0C0F26 + m)
    layout = aexq.LAYOUT_PACK4_LINEAR
    logits = aexq.new_activation(m, n, torch.float32, layout)
    am = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    gap = torch.zeros(m, dtype=torch.float32, device="cuda")
    xd = aexq.describe(dev(x16), m, k)
    ld = aexq.describe(logits, m, n, layout)
    ctx.lmhead_argmax(w, xd, ld, am, gap)
    torch.cuda.synchronize()
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), wf)
    stride = aexq.storage_elements(layout, m, n)
    assert normwise(logits.cpu().numpy().reshape(m, stride)[:, :n], ref) <= 1e-5
    ref_idx = orc.argmax_rows(ref.astype(np.float32))
    srt = np.sort(ref, axis=1)
    ref_gap = srt[:, -1] - srt[:, -2]
    gi = am.cpu().numpy()
    for r in range(m):
        if ref_gap[r] >= ARGMAX_TIE:
            assert gi[r] == ref_idx[r], (r, gi[r], ref_idx[r])
    np.testing.assert_allclose(gap.cpu().numpy(), ref_gap, atol=1e-5)
    am2 = torch.full((m,), -1, dtype=torch.int32, device="cuda")
    ctx.lmhead_argmax(w, xd, None, am2)
    torch.cuda.synchronize()
    assert np.array_equal(am2.cpu().numpy(), gi)


def test_argmax_reference_kats_and_rules(ctx, aexq, orc):
    _announce("argmax kats")
    from aiimage_amd import _abi
    cases = []
    v = -np.arange(17, dtype=np.float32); v[13] = 100.0; cases.append((v, 13))
    cases.append((np.array([1, 5, 5, 2], np.float32), 1))
    cases.append((np.array([np.nan, 5, 7], np.float32), 0))
    cases.append((np.array([1, np.nan, 3], np.float32), 2))
    cases.append((np.full(5, -np.inf, np.float32), 0))
    big = np.random.default_rng(1).standard_normal(100000).astype(np.float32)
    big[777] = big[99999] = 9.0
    cases.append((big, 777))
    for vals, want in cases:
        t = dev(vals)
        am = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        ctx.argmax(aexq.describe(t, 1, vals.size), am)
        torch.cuda.synchronize()
        assert am.item() == want == orc.argmax_rows(vals)[0]
    # tiled Pack4 KAT: 37 vocab, tile width 4 packs -> 34
    v = -(np.arange(37, dtype=np.float32) + 1); v[34] = 100.0
    storage = np.zeros(4 * 3 * 4, np.float32); storage[:37] = v
    d = _abi.Tensor()
    d.logical = _abi.Shape(2, 37, 1, 1, 1)
    d.storage = _abi.Shape(3, 4, 3, 1, 4)
    d.layout = _abi.LAYOUT_PACK4_TILED
    d.dtype = _abi.DTYPE_F32
    t = dev(storage)
    d.data = t.data_ptr()
    d.batch = 1
    am = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    ctx.argmax(d, am)
    torch.cuda.synchronize()
    assert am.item() == 34


# ------------------------------------------------------------------ stacked / grouped launches

def test_grouped_and_stacked_launch_matches_single(ctx, aexq):
    """Size-independent property: a grouped launch over a replicated weight stack
    gives, for every copy, exactly the single-launch output."""
    _announce("grouped stacked")
    from aiimage_amd import synth
    k = 1024
    ws = []
    for i, (name, n, kk) in enumerate(synth.LAYER_LINEARS):
        if kk == k:
            ws.append((n, _q4_weight(ctx, aexq, n, k, 300 + i)[0]))
    copies = 3
    x = dev(synth.activations(1, k, 400))
    singles = []
    for n, w in ws:
        y = aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
        ctx.linear(w, aexq.describe(x, 1, k), aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR))
        singles.append(y)
    stacks = [w.replicate(copies) for _, w in ws]
    outs = [torch.zeros(copies * n, dtype=torch.float16, device="cuda") for n, _ in ws]
    ydesc = [aexq.describe(o, 1, n, aexq.LAYOUT_PACK4_LINEAR, batch=copies, batch_stride=n)
             for o, (n, _) in zip(outs, ws)]
    ctx.linear_group(stacks, aexq.describe(x, 1, k), ydesc)
    torch.cuda.synchronize()
    for s, o, (n, _) in zip(singles, outs, ws):
        for c in range(copies):
            assert torch.equal(o[c * n:(c + 1) * n], s[:n])


def test_linearity_at_full_layer_size(ctx, aexq):
    """y(2x) == 2 y(x) exactly for power-of-two scaling (fp32 output, no bias)."""
    _announce("linearity")
    from aiimage_amd import synth
    n, k = 3584, 1024
    w, _, _ = _q4_weight(ctx, aexq, n, k, 500)
    x = synth.activations(1, k, 501).astype(np.float32)
    y1 = aexq.new_activation(1, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    y2 = aexq.new_activation(1, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    ctx.linear(w, aexq.describe(dev(x, torch.float16), 1, k), aexq.describe(y1, 1, n, 1))
    ctx.linear(w, aexq.describe(dev(2 * x, torch.float16), 1, k), aexq.describe(y2, 1, n, 1))
    torch.cuda.synchronize()
    assert torch.equal(y2, 2 * y1)


# ------------------------------------------------------------------ small-M MFMA path (config 4)

def _mm_case(ctx, aexq, orc, fmt, n, k, m, seed, group=32, code=1, scale_f16=True, ydtype=None,
             **kw):
    """One linear on the M >= 2 path; returns (y [m][n] float64, ref, plan string)."""
    from aiimage_amd import synth
    sdt = np.float16 if scale_f16 else np.float32
    if fmt == 8:
        words, scales, _ = synth.q8_weights(n, k, seed, scale_dtype=sdt)
        w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
        wf = orc.dequant_q8(words, scales, n, k,
                            scale_dtype=orc.SCALE_F16 if scale_f16 else orc.SCALE_F32)
    else:
        w, words, scales = _q4_weight(ctx, aexq, n, k, seed, group=group, code=code,
                                      scale_f16=scale_f16)
        wf = orc.dequant_q4(words, scales, n, k, group, nibble_code=code,
                            scale_dtype=orc.SCALE_F16 if scale_f16 else orc.SCALE_F32)
    x16 = synth.activations(m, k, seed + 1)
    ydtype = ydtype or torch.float16
    y = aexq.new_activation(m, n, ydtype, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    plan = ctx.plan_check(w, xd, yd, **kw)
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    stride = aexq.storage_elements(aexq.LAYOUT_PACK4_LINEAR, m, n)
    got = y.cpu().numpy().astype(np.float64).reshape(m, stride)
    assert np.all(got[:, n:] == 0)
    return got[:, :n], wf, x16, plan


@pytest.mark.parametrize("fmt,n,k,m", [(8, 3584, 1024, 16), (8, 1024, 2048, 64), (8, 1024, 1024, 512),
                                       (4, 3584, 1024, 16), (4, 1024, 3584, 64), (4, 2048, 1024, 512),
                                       (4, 512, 1024, 5), (8, 256, 384, 31)])
def test_small_m_mfma_config4(ctx, aexq, orc, fmt, n, k, m):
    """Batched decode / short prefill shapes on the MFMA path against the float64 oracle."""
    _announce(f"mfma q{fmt} n={n} k={k} m={m}")
    got, wf, x16, plan = _mm_case(ctx, aexq, orc, fmt, n, k, m, seed=n + k + m)
    # M > 32: the tiled GEMM; M <= 32: one MFMA launch of 16- or 32-row blocks
    assert plan.startswith("kernel=qgemm" if m > 32 else "kernel=qmm"), plan
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), wf)
    assert normwise(got, ref) <= TOL


@pytest.mark.parametrize("group,scale_f16,code", [(16, False, 0), (16, True, 0), (32, False, 0)])
def test_small_m_mfma_reference_q4_formats(ctx, aexq, orc, group, scale_f16, code):
    """The reference's shipping Q4 (two's complement, group 16, fp32 scales) and its
    neighbours at M > 1, fp32 output for a tight bar."""
    _announce(f"mfma q4 group={group} f16={scale_f16}")
    got, wf, x16, plan = _mm_case(ctx, aexq, orc, 4, 1024, 1024, 12, seed=40 + group,
                                  group=group, code=code, scale_f16=scale_f16,
                                  ydtype=torch.float32)
    assert plan.startswith("kernel=qmm"), plan
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), wf)
    assert normwise(got, ref) <= 1e-5


@pytest.mark.parametrize("prepass", [False, True])
def test_small_m_mfma_swiglu_rmsnorm(ctx, aexq, orc, monkeypatch, prepass):
    """M=20 gate/up with RMSNorm-in and SwiGLU-out on the MFMA path: inside the
    wide kernel (one item per workgroup) or as the row pre-pass."""
    _announce(f"mfma swiglu rmsnorm m=20 prepass={prepass}")
    if prepass:
        monkeypatch.setenv("AEXQ_RMS_PREPASS", "1")
    from aiimage_amd import synth
    n, k, m, eps = 3584, 1024, 20, 1e-6
    wg, gw, gs = _q4_weight(ctx, aexq, n, k, 61)
    wu, uw, us = _q4_weight(ctx, aexq, n, k, 62)
    x16 = synth.activations(m, k, 63)
    gamma = synth.rms_gamma(k, 64)
    y = aexq.new_activation(m, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    kw = dict(rmsnorm=True, rms_gamma=dev(gamma), rms_eps=eps, up=wu)
    plan = ctx.plan_check(wg, xd, yd, **kw)
    assert plan.startswith("kernel=qmm") and f"rms_prepass={int(prepass)}" in plan, plan
    ctx.linear(wg, xd, yd, **kw)
    torch.cuda.synchronize()
    xn = orc.rmsnorm(x16.astype(np.float32), eps, gamma).astype(np.float16).astype(np.float32)
    g = _q4_ref(orc, gw, gs, n, k, 32, 1, True, xn)
    u = _q4_ref(orc, uw, us, n, k, 32, 1, True, xn)
    ref = np.stack([orc.swiglu(g[r].astype(np.float32), u[r].astype(np.float32)) for r in range(m)])
    got = y.cpu().numpy().astype(np.float64).reshape(m, -1)[:, :n]
    assert normwise(got, ref) <= TOL


@pytest.mark.parametrize("bcast", [1, 3])
def test_small_m_mfma_row_blocks_bias_residual(ctx, aexq, orc, monkeypatch, bcast):
    """M=33 crosses the 32-row launch blocks: row-indexed C and the residual must
    follow each block's rows (the tiled GEMM, which would take M > 32, switched off)."""
    _announce(f"mfma m=33 bcast={bcast}")
    from aiimage_amd import synth
    monkeypatch.setenv("AEXQ_QGEMM_OFF", "1")
    n, k, m = 512, 1024, 33
    words, scales, _ = synth.q8_weights(n, k, 71, scale_dtype=np.float32)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    x16 = synth.activations(m, k, 72)
    rng = np.random.default_rng(73)
    c = rng.standard_normal(m if bcast == 1 else m * n).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    y = aexq.new_activation(m, n, torch.float32, aexq.LAYOUT_PACK4_LINEAR)
    rd = dev(res)
    xd = aexq.describe(dev(x16), m, k)
    yd = aexq.describe(y, m, n, aexq.LAYOUT_PACK4_LINEAR)
    kw = dict(alpha=0.75, beta=1.5, c=dev(c), broadcast_c=bcast,
              residual=aexq.describe(rd, m, n, aexq.LAYOUT_PACK4_LINEAR))
    assert ctx.plan_check(w, xd, yd, **kw).startswith("kernel=qmm")
    ctx.linear(w, xd, yd, **kw)
    torch.cuda.synchronize()
    s = orc.gemm_gpu_semantics(x16.astype(np.float32), orc.dequant_q8(words, scales, n, k))
    cc = np.repeat(c[:, None], n, 1) if bcast == 1 else c.reshape(m, n)
    ref = 0.75 * (1.5 * cc + s) + res
    got = y.cpu().numpy().reshape(m, n)
    assert normwise(got, ref) <= 1e-5


@pytest.mark.parametrize("splitk", ["1", "4"])
def test_small_m_mfma_stacked_copies_match_single(ctx, aexq, monkeypatch, splitk):
    """Size-independent property at M=16: every copy of a replicated weight stack
    gives exactly the single-weight output (the same K chunking for both: the
    plan would split the single launch only)."""
    _announce(f"mfma stacked copies splitk={splitk}")
    monkeypatch.setenv("AEXQ_SPLITK", splitk)
    from aiimage_amd import synth
    n, k, m, copies = 2048, 1024, 16, 5
    w, _, _ = _q4_weight(ctx, aexq, n, k, 81)
    x = dev(synth.activations(m, k, 82))
    y1 = aexq.new_activation(m, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    ctx.linear(w, aexq.describe(x, m, k), aexq.describe(y1, m, n, aexq.LAYOUT_PACK4_LINEAR))
    st = w.replicate(copies)
    ys = torch.zeros(copies * m * n, dtype=torch.float16, device="cuda")
    ctx.linear(st, aexq.describe(x, m, k),
               aexq.describe(ys, m, n, aexq.LAYOUT_PACK4_LINEAR, batch=copies, batch_stride=m * n))
    torch.cuda.synchronize()
    for c in range(copies):
        assert torch.equal(ys[c * m * n:(c + 1) * m * n], y1)
