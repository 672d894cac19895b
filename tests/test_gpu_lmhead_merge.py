"""The LM head's in-launch argmax merge (MM:645-686 first-maximum rule): every
workgroup leaves its (best, index, second) partial as three tagged words and
the grid's last workgroup merges them with packed keys.  The cases the keys
encode specially, on each fused kernel -- the streaming kernel at M = 1 and at
M = 3 (K = 1008, not a multiple of 128), the wide MFMA kernel at M = 4:

  * a NaN logit at index 0 wins every row (gap NaN);
  * a NaN logit elsewhere never wins and is left out of the gap;
  * zero logits at rows 5000 (a zero row times a negative scale), 70000 and
    140000 tie as the maximum, every other logit negative: the lowest index
    wins, gap 0;
  * consecutive launches whose grids shrink and grow again (stale partials of
    an earlier, larger grid lie past the smaller grid's) each give their own
    argmax, through both the allocating and the no-allocation entry points.

Expected values come from the oracle's logits and its argmax (the reference's
scan), the gap from the best of the other candidates, NaN ignored.
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

N = 151936
# (rows, K): streaming M = 1, streaming M = 3 (K % 128 != 0), MFMA M = 4
SHAPES = [(1, 1024), (3, 1008), (4, 1024)]


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


def _expect(orc, ref):
    """(index, gap) per row: the oracle's scan, and best minus the best of the
    other candidates with NaN left out (inf when there is none)."""
    idx = orc.argmax_rows(np.ascontiguousarray(ref, np.float32))
    gaps = []
    for r in range(ref.shape[0]):
        best = ref[r, idx[r]]
        rest = np.delete(ref[r], idx[r])
        rest = rest[~np.isnan(rest)]
        gaps.append(np.nan if np.isnan(best) else (best - rest.max() if rest.size else np.inf))
    return np.asarray(idx), np.asarray(gaps, np.float64)


def _run(ctx, aexq, w, x16, m, k, noalloc=False):
    xd = aexq.describe(torch.as_tensor(x16).cuda(), m, k)
    am = torch.full((m,), -2, dtype=torch.int32, device="cuda")
    gap = torch.full((m,), -2.0, dtype=torch.float32, device="cuda")
    if noalloc:
        ctx.lmhead_argmax_noalloc(w, xd, am, gap)
    else:
        ctx.lmhead_argmax(w, xd, None, am, gap)
    torch.cuda.synchronize()
    return am.cpu().numpy(), gap.cpu().numpy()


def _check(got, want, tie=1e-3):
    """Index and gap per row where the oracle's gap is NaN or at least `tie`
    (a nearer tie may resolve either way within the logits' tolerance)."""
    gi, gg = got
    wi, wg = want
    for r in range(len(wi)):
        if np.isnan(wg[r]):
            assert gi[r] == wi[r] and np.isnan(gg[r]), (r, gi[r], wi[r], gg[r])
        elif wg[r] >= tie:
            assert gi[r] == wi[r], (r, gi[r], wi[r])
            assert abs(float(gg[r]) - wg[r]) <= tie, (r, gg[r], wg[r])


def _weight(ctx, aexq, codes, scales, k):
    words = np.ascontiguousarray(codes).reshape(-1).view(np.uint32).copy()
    return ctx.weight(aexq.QuantizedTensor(N * k, k, words, scales, bits=8), N, k), words


@pytest.mark.parametrize("m,k", SHAPES)
def test_merge_nan_rows(ctx, aexq, orc, m, k):
    from aiimage_amd import synth
    _announce(f"lm head merge NaN rows m={m} k={k}")
    _, scales, codes = synth.q8_weights(N, k, 0xAE1E1000 + m)
    x16 = synth.activations(m, k, 0xAE1E1001 + m)
    # NaN elsewhere: rows 777 and 151000 never win, even beside a planted winner
    win = np.where(x16[0].astype(np.float32) >= 0, 127, -127).astype(np.int8)
    codes = codes.copy()
    codes[90000] = win
    scales = scales.copy()
    scales[90000] = np.float16(0.05)
    scales[777] = np.float16(np.nan)
    scales[151000] = np.float16(np.nan)
    w, words = _weight(ctx, aexq, codes, scales, k)
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32),
                                 orc.dequant_q8(words, scales, N, k, scale_dtype=orc.SCALE_F16))
    want = _expect(orc, ref)
    assert want[0][0] == 90000 and want[1][0] >= 1e-3
    _check(_run(ctx, aexq, w, x16, m, k), want)
    w.release()
    # NaN at index 0 wins every row
    scales[0] = np.float16(np.nan)
    w, words = _weight(ctx, aexq, codes, scales, k)
    got = _run(ctx, aexq, w, x16, m, k)
    assert np.array_equal(got[0], np.zeros(m, np.int32)), got
    assert np.all(np.isnan(got[1])), got
    w.release()


@pytest.mark.parametrize("m,k", SHAPES)
def test_merge_zero_tie(ctx, aexq, orc, m, k):
    from aiimage_amd import synth
    _announce(f"lm head merge zero tie m={m} k={k}")
    rng = np.random.default_rng(0xAE1E2000 + m)
    # every nonzero row has negative codes against positive activations: a
    # negative logit; three zero rows give 0.0
    block = rng.integers(1, 128, size=(1024, k), dtype=np.int8)
    codes = -np.tile(block, (N // 1024 + 1, 1))[:N]
    scales = rng.uniform(0.01, 0.05, size=N).astype(np.float16)
    for r, s in ((5000, -0.03), (70000, 0.03), (140000, 0.04)):
        codes[r] = 0
        scales[r] = np.float16(s)
    x16 = (np.abs(synth.activations(m, k, 0xAE1E2001 + m).astype(np.float32)) + 0.01).astype(np.float16)
    w, words = _weight(ctx, aexq, codes, scales, k)
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32),
                                 orc.dequant_q8(words, scales, N, k, scale_dtype=orc.SCALE_F16))
    assert np.all(ref[:, [5000, 70000, 140000]] == 0.0)
    want = _expect(orc, ref)
    assert np.all(want[0] == 5000) and np.all(want[1] == 0.0)
    gi, gg = _run(ctx, aexq, w, x16, m, k)
    assert np.all(gi == 5000) and np.all(gg == 0.0), (gi, gg)
    # the logits the kernel compared: zero at the three rows (the epilogue
    # leaves row 5000 at +0.0 too), negative elsewhere
    layout = aexq.LAYOUT_PACK4_LINEAR
    logits = aexq.new_activation(m, N, torch.float32, layout)
    am = torch.full((m,), -2, dtype=torch.int32, device="cuda")
    ctx.lmhead_argmax(w, aexq.describe(torch.as_tensor(x16).cuda(), m, k),
                      aexq.describe(logits, m, N, layout), am)
    torch.cuda.synchronize()
    lg = logits.cpu().numpy().reshape(m, -1)[:, :N]
    assert np.all(lg[:, [5000, 70000, 140000]] == 0.0)
    assert np.all(np.delete(lg, [5000, 70000, 140000], axis=1) < 0.0)
    assert np.all(am.cpu().numpy() == 5000)
    w.release()


@pytest.mark.parametrize("m,k", SHAPES)
def test_merge_grids_shrink_and_grow(ctx, aexq, orc, monkeypatch, m, k):
    """Launch after launch at changing grid sizes, each with its own
    activations (and so its own argmax): a launch never takes an earlier
    launch's partials for its own."""
    from aiimage_amd import synth
    _announce(f"lm head merge changing grids m={m} k={k}")
    words, scales, _ = synth.q8_weights(N, k, 0xAE1E3000 + m)
    w = ctx.weight(aexq.QuantizedTensor(N * k, k, words, scales, bits=8), N, k)
    deq = orc.dequant_q8(words, scales, N, k, scale_dtype=orc.SCALE_F16)
    env = "AEXQ_QMM_BLOCKS_PER_CU" if m == 4 else "AEXQ_QMV_BLOCKS_PER_CU"
    for step, (per_cu, noalloc) in enumerate(((8, False), (2, False), (8, False), (1, True),
                                              (6, True), (3, False))):
        monkeypatch.setenv(env, str(per_cu))
        x16 = synth.activations(m, k, 0xAE1E3100 + 7 * step + m)
        ref = orc.gemm_gpu_semantics(x16.astype(np.float32), deq)
        wi, wg = _expect(orc, ref)
        _check(_run(ctx, aexq, w, x16, m, k, noalloc=noalloc), (wi, wg))
    w.release()


def test_merge_one_and_two_levels(ctx, aexq, orc, monkeypatch):
    """A grid of 2048 workgroups merged in two levels (runs of 64, 31 run
    mergers, then the grid's last workgroup) and in one: the same index and
    the same gap bits, both the oracle's."""
    from aiimage_amd import synth
    m, k = 4, 1024
    _announce(f"lm head merge one and two levels m={m} k={k} grid 8 per CU")
    words, scales, _ = synth.q8_weights(N, k, 0xAE1E3200)
    w = ctx.weight(aexq.QuantizedTensor(N * k, k, words, scales, bits=8), N, k)
    deq = orc.dequant_q8(words, scales, N, k, scale_dtype=orc.SCALE_F16)
    x16 = synth.activations(m, k, 0xAE1E3201)
    wi, wg = _expect(orc, orc.gemm_gpu_semantics(x16.astype(np.float32), deq))
    monkeypatch.setenv("AEXQ_QMM_BLOCKS_PER_CU", "8")
    two = _run(ctx, aexq, w, x16, m, k)
    monkeypatch.setenv("AEXQ_ARGMAX_ONE_LEVEL", "1")
    one = _run(ctx, aexq, w, x16, m, k)
    _check(two, (wi, wg))
    _check(one, (wi, wg))
    assert np.array_equal(two[0], one[0]), (two[0], one[0])
    assert np.array_equal(two[1].view(np.uint32), one[1].view(np.uint32)), (two[1], one[1])
    w.release()


@pytest.mark.parametrize("dtype,rows,width,packed", [
    (torch.float32, 40, 151936, False),   # two launches of up to 32 rows, 16-byte loads
    (torch.float32, 3, 100003, False),    # odd row stride: element loads
    (torch.float16, 5, 151936, False),    # fp16 logits, 16-byte loads
    (torch.float16, 2, 4099, True),       # Pack4 rows of 4100 fp16: 8-byte aligned, element loads
])
def test_argmax_over_logits_one_launch(ctx, aexq, orc, dtype, rows, width, packed):
    """aexq_argmax: the argmax launch over existing logits rows merges its
    partials in the launch too; rows of any stride and count, fp32 or fp16,
    planted NaN / tie cases in the first rows."""
    _announce(f"argmax over logits {dtype} rows={rows} width={width} packed={packed}")
    layout = aexq.LAYOUT_PACK4_LINEAR if packed else aexq.LAYOUT_LINEAR
    g = torch.Generator(device="cpu").manual_seed(0xAE1E4000 + rows)
    vals = torch.randn(rows, width, generator=g).to(dtype)
    vals[0, 0] = float("nan")                          # NaN at index 0 wins row 0
    if rows > 1:
        vals[1, 3] = float("nan")                      # NaN elsewhere never wins
        vals[1, width - 1] = vals[1, width // 2] = 9.0  # tie: the lower index
    lg = aexq.new_activation(rows, width, dtype, layout)
    stride = lg.numel() // rows
    lg.view(rows, stride)[:, :width] = vals.cuda()
    am = torch.full((rows,), -2, dtype=torch.int32, device="cuda")
    gap = torch.full((rows,), -2.0, dtype=torch.float32, device="cuda")
    ctx.argmax(aexq.describe(lg, rows, width, layout), am, gap)
    torch.cuda.synchronize()
    ref = vals.float().numpy()
    want = _expect(orc, ref)
    got = (am.cpu().numpy(), gap.cpu().numpy())
    assert np.array_equal(got[0], want[0]), (got[0], want[0])
    for r in range(rows):
        if np.isnan(want[1][r]):
            assert np.isnan(got[1][r])
        else:
            assert got[1][r] == np.float32(want[1][r]), (r, got[1][r], want[1][r])
    assert got[0][0] == 0
    if rows > 1:
        assert got[0][1] == width // 2 and got[1][1] == 0.0
