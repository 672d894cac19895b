"""Pins the CPU oracle (oracle/aexq_oracle.c) before it is trusted as the checker.

Each test checks an oracle function against a known-answer vector from the
reference's own tests (tests/golden/reference_kats.json), against an
independent route through numpy, or against a closed form, chosen so that a
dropped term, a wrong sign, a transposed index or a wrong rounding mode fails.
"""
import json
import math
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


# ---------------------------------------------------------------- scalars

def test_half_to_float_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint32)
    ours = np.array([orc.half_to_float(int(b)) for b in bits], np.float32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(ours[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(ours[np.isnan(ref)]))
    assert np.array_equal(ours[np.isinf(ref)], ref[np.isinf(ref)])
    # subnormal smallest and largest are preserved, not flushed
    assert orc.half_to_float(0x0001) == 2.0 ** -24
    assert orc.half_to_float(0x03FF) == 1023 * 2.0 ** -24


def test_float_to_half_matches_numpy_rne(orc):
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32),
        (rng.standard_normal(2000) * 1e-5).astype(np.float32),   # subnormal range
        (rng.standard_normal(1000) * 6e4).astype(np.float32),    # near overflow
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 2.0 ** -25, 2.0 ** -24 * 1.5,
                  2.0 ** -24 * 2.5, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32),
    ])
    ours = np.array([orc.float_to_half(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_round_to_int_is_ties_to_even(orc):
    cases = {0.5: 0, 1.5: 2, 2.5: 2, -0.5: 0, -1.5: -2, -2.5: -2, 63.5: 64, -63.5: -64,
             95.25: 95, 31.75: 32, 126.49: 126, -126.51: -127}
    for v, want in cases.items():
        assert orc.round_to_int(v) == want, v
    assert orc.round_to_int(float("nan")) == -2 ** 31


# ---------------------------------------------------------------- packers

def test_q8_packer_reference_kat(orc):
    kat = KATS["q8_weight_packer"]
    packed, scales = orc.q8_pack_rows(kat["weights"], kat["rows"], kat["cols"])
    np.testing.assert_allclose(scales, kat["expected_scales"], atol=kat["scale_tolerance"], rtol=0)
    got = packed.view(np.int8).reshape(kat["rows"], kat["cols"])
    assert got.tolist() == kat["expected_bytes"]


def test_q8_packer_transposed_layout_keeps_per_channel_scales(orc):
    rng = np.random.default_rng(3)
    w = rng.standard_normal((6, 12)).astype(np.float32)          # [N][K]
    p_row, s_row = orc.q8_pack_rows(w, 6, 12, contiguous=True)
    p_col, s_col = orc.q8_pack_rows(w.T.copy(), 6, 12, contiguous=False)  # data stored [K][N]
    assert np.array_equal(s_row, s_col)
    q_row = p_row.view(np.int8).reshape(6, 12)
    q_col = p_col.view(np.int8).reshape(12, 6)
    assert np.array_equal(q_row, q_col.T)
    # every code is round(v / scale) within +-127 and the row maximum maps to +-127
    assert np.all(np.abs(q_row).max(axis=1) == 127)
    np.testing.assert_allclose(q_row * s_row[:, None], w, atol=float(s_row.max()) * 0.5 + 1e-7)


def test_q4_packer_codes_and_scale_block(orc):
    w = np.array([[7.0, -7.0, 3.5, -3.5, 0.0, 1.0, -1.0, 2.0],
                  [0.0] * 8], np.float32)
    packed, scales, blk = orc.q4_pack_rows(w, 2, 8)
    assert blk == 8
    assert scales.tolist() == [1.0, 1.0]          # maxAbs 7 -> 1; all-zero row -> 1
    nib = np.array([(int(packed[0]) >> (4 * i)) & 0xF for i in range(8)])
    signed = np.where(nib >= 8, nib - 16, nib)
    assert signed.tolist() == [7, -7, 4, -4, 0, 1, -1, 2]   # 3.5 -> 4, -3.5 -> -4 (ties to even)
    assert int(packed[1]) == 0
    _, _, blk_t = orc.q4_pack_rows(w.T.copy(), 2, 8, contiguous=False)
    assert blk_t == 0


# ---------------------------------------------------------------- dequant

def test_dequant_q8_exhaustive_bytes_all_lanes(orc):
    # every byte value in every lane of a word, against numpy's little-endian int8 view
    b = np.arange(256, dtype=np.uint8)
    rows = []
    for lane in range(4):
        words = np.zeros((256, 4), np.uint8)
        words[:, lane] = b
        rows.append(words.reshape(-1))
    raw = np.concatenate(rows)                       # 1024 words
    words = raw.view(np.uint32)
    n, k = 16, 256
    scales = (2.0 ** np.arange(-8, 8)).astype(np.float32)
    got = orc.dequant_q8(words, scales, n, k)
    want = words.view(np.int8).reshape(n, k).astype(np.float32) * scales[:, None]
    assert np.array_equal(got, want)


def test_dequant_q8_fp16_subnormal_scales_are_not_flushed(orc):
    words = np.full(4, 0x7F81FF01, np.uint32)       # bytes 1, -1, -127, 127
    sc = np.array([1, 0x03FF, 0x0400, 0x3C00], np.uint16).view(np.float16)
    got = orc.dequant_q8(words, sc, 4, 4, scale_dtype=orc.SCALE_F16)
    s = np.array([2.0 ** -24, 1023 * 2.0 ** -24, 2.0 ** -14, 1.0], np.float32)
    want = np.array([1, -1, -127, 127], np.float32)[None, :] * s[:, None]
    assert np.array_equal(got, want)
    assert got[0, 0] > 0


@pytest.mark.parametrize("code", [0, 1])
@pytest.mark.parametrize("block", [16, 32, 64, 0])
def test_dequant_q4_exhaustive_nibbles(orc, code, block):
    # all 16 codes at all 8 positions; the numpy route reads bytes, splits low/high nibbles
    n, k = 4, 128
    rng = np.random.default_rng(block + 10 * code)
    nibbles = np.tile(np.arange(16, dtype=np.uint8), n * k // 16)
    rng.shuffle(nibbles)
    byte = (nibbles[0::2] | (nibbles[1::2] << 4)).astype(np.uint8)
    words = byte.view(np.uint32)
    nscales = n * k // block if block else n
    scales = (rng.integers(1, 64, nscales) / 8.0).astype(np.float32)
    got = orc.dequant_q4(words, scales, n, k, block, nibble_code=code)
    lo = (byte & 0xF).astype(np.int32)
    hi = (byte >> 4).astype(np.int32)
    q = np.empty(n * k, np.int32)
    q[0::2], q[1::2] = lo, hi
    q = (q ^ 8) - 8 if code == 0 else q - 8
    if block:
        sidx = np.arange(n * k) // block
    else:
        sidx = np.repeat(np.arange(n), k)
    want = (q.astype(np.float32) * scales[sidx]).reshape(n, k)
    assert np.array_equal(got, want)


def test_nibble_code_bridge_is_xor_8(orc):
    # (q + 8) & 0xF == (q & 0xF) ^ 8 for every q in [-8, 7]: the two codes differ by one XOR
    rng = np.random.default_rng(5)
    q = rng.integers(-8, 8, 256)
    twos = (q & 0xF).astype(np.uint8)
    off8 = ((q + 8) & 0xF).astype(np.uint8)
    assert np.array_equal(twos ^ 8, off8)
    def pack(nib):
        b = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
        return b.view(np.uint32)
    sc = np.ones(8, np.float32)
    a = orc.dequant_q4(pack(twos), sc, 8, 32, 32, nibble_code=orc.NIBBLE_TWOS)
    b = orc.dequant_q4(pack(off8), sc, 8, 32, 32, nibble_code=orc.NIBBLE_OFFSET8)
    assert np.array_equal(a, b)
    assert np.array_equal(a.ravel(), q.astype(np.float32))


# ---------------------------------------------------------------- gemm

def _dot_dequantized(inp, weights, oc, k):
    """The reference test's own expected-value rule (NcnnInt8WeightOnlyGpuTests.cs:223-237)."""
    row = np.asarray(weights[oc * k:(oc + 1) * k], np.float32)
    max_abs = np.float32(np.abs(row).max())
    scale = np.float32(max_abs / np.float32(127)) if max_abs > 0 else np.float32(1)
    s = np.float32(0)
    for i in range(k):
        q = np.float32(np.clip(np.round(row[i] / scale), -127, 127))  # np.round is ties-to-even
        s = np.float32(s + np.float32(np.float32(inp[i]) * q) * scale)
    return float(s)


def test_gemm_reference_kat_int8(orc):
    kat = KATS["q8_gemm_kernel"]
    n, k = kat["n"], kat["k"]
    packed, scales = orc.q8_pack_rows(kat["weights"], n, k)
    w = orc.dequant_q8(packed, scales, n, k)
    x = np.array([kat["input"]], np.float32)
    got = orc.gemm_gpu_semantics(x, w, 1.0, 1.0, np.array(kat["bias"], np.float32), 4)[0]
    for c in range(n):
        want = kat["bias"][c] + _dot_dequantized(kat["input"], kat["weights"], c, k)
        assert abs(got[c] - want) <= kat["tolerance"]
    # by hand: row 0 = [1, -.5, .25, 2], scale 2/127, codes [64, -32, 16, 127]
    # (63.5 -> 64 ties to even); dot with [1, -1, .5, 2] = 358 codes
    hand0 = 0.1 + (64 + 32 + 16 * 0.5 + 127 * 2) * (2 / 127)
    assert abs(got[0] - hand0) < 1e-5
    # the CPU twin (RunGemmCpu) agrees
    cpu = orc.gemm_cpu(x, w, n, True, 1.0, 1.0, np.array(kat["bias"], np.float32), 4)[0]
    np.testing.assert_allclose(cpu, got, atol=1e-6)


def _create_values(count, scale, period):
    i = np.arange(count)
    return (((i * 7) % period - period // 2) * scale).astype(np.float32)


def test_gemm_reference_linear_projection_golden(orc):
    kat = KATS["linear_projection_fp32"]
    rows, k, n = kat["rows"], kat["k"], kat["n"]
    x = _create_values(rows * k, kat["input"]["scale"], kat["input"]["period"]).reshape(rows, k)
    w = _create_values(n * k, kat["weights"]["scale"], kat["weights"]["period"]).reshape(n, k)
    b = _create_values(n, kat["bias"]["scale"], kat["bias"]["period"])
    # the test's ReferenceLinearProjection: float32, bias first, k ascending
    want = np.zeros((rows, n), np.float32)
    for r in range(rows):
        for c in range(n):
            s = np.float32(b[c])
            for kk in range(k):
                s = np.float32(s + np.float32(x[r, kk] * w[c, kk]))
            want[r, c] = s
    got = orc.gemm_gpu_semantics(x, w, 1.0, 1.0, b, 4)
    assert np.max(np.abs(got - want)) <= kat["tolerance"]
    cpu = orc.gemm_cpu(x, w, n, True, 1.0, 1.0, b, 4)
    assert np.max(np.abs(cpu - want)) <= kat["tolerance"]


@pytest.mark.parametrize("trans_b", [True, False])
@pytest.mark.parametrize("bcast", [-1, 0, 1, 3, 4])
def test_gemm_cpu_against_numpy(orc, trans_b, bcast):
    rng = np.random.default_rng(11 + bcast)
    m, k, n = 3, 37, 19
    a = rng.standard_normal((m, k)).astype(np.float32)
    wt = rng.standard_normal((n, k)).astype(np.float32)
    b = wt if trans_b else wt.T.copy()
    alpha, beta = 0.75, -1.25
    c = {-1: None, 0: rng.standard_normal(1), 1: rng.standard_normal(m),
         3: rng.standard_normal(m * n), 4: rng.standard_normal(n)}[bcast]
    c = None if c is None else c.astype(np.float32)
    got = orc.gemm_cpu(a, b, n, trans_b, alpha, beta, c, bcast)
    prod = a.astype(np.float64) @ wt.astype(np.float64).T
    want = alpha * prod
    if c is not None:
        cc = {0: lambda: np.full((m, n), c[0]), 1: lambda: np.repeat(c[:, None], n, 1),
              3: lambda: c.reshape(m, n), 4: lambda: np.repeat(c[None, :], m, 0)}[bcast]()
        want = want + beta * cc
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    mt = orc.gemm_cpu(a, b, n, trans_b, alpha, beta, c, bcast, threads=4)
    assert np.array_equal(mt.view(np.uint32), got.view(np.uint32))


def test_gemm_gpu_semantics_alpha_scales_bias(orc):
    # Pack4-linear kernel: alpha * (beta*C + sum) (MM:1054-1057,1101); CPU path: alpha*sum + beta*C
    a = np.array([[1.0, 2.0]], np.float32)
    w = np.array([[3.0, 4.0]], np.float32)
    c = np.array([10.0], np.float32)
    gpu = orc.gemm_gpu_semantics(a, w, 2.0, 0.5, c, 4)[0, 0]
    cpu = orc.gemm_cpu(a, w, 1, True, 2.0, 0.5, c, 4)[0, 0]
    assert gpu == 2.0 * (0.5 * 10.0 + 11.0)
    assert cpu == 2.0 * 11.0 + 0.5 * 10.0


# ---------------------------------------------------------------- epilogues

def test_rmsnorm_closed_forms(orc):
    y = orc.rmsnorm(np.array([3.0, 4.0], np.float32), 0.0)[0]
    r = math.sqrt(12.5)
    np.testing.assert_allclose(y, [3 / r, 4 / r], rtol=1e-7)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 1024)).astype(np.float32)
    y = orc.rmsnorm(x, 0.0)
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(1)), 1.0, rtol=1e-6)
    # scale invariance with eps = 0, and gamma multiplies elementwise
    np.testing.assert_allclose(orc.rmsnorm(x * 37.0, 0.0), y, rtol=2e-6, atol=1e-7)
    g = (1.0 + 0.02 * rng.standard_normal(1024)).astype(np.float32)
    np.testing.assert_allclose(orc.rmsnorm(x, 0.0, g), y * g[None, :], rtol=2e-6, atol=1e-7)
    # eps enters inside the root: all-equal row c gives c / sqrt(c^2 + eps)
    c, eps = 0.01, 1e-4
    yc = orc.rmsnorm(np.full(8, c, np.float32), eps)[0]
    np.testing.assert_allclose(yc, c / math.sqrt(c * c + eps), rtol=1e-6)
    # zero row stays zero (the 1e-20 floor prevents inf*0)
    assert np.all(orc.rmsnorm(np.zeros(8, np.float32), 0.0) == 0)
    # gamma index is clamped to the last affine weight
    yg = orc.rmsnorm(np.ones(4, np.float32), 0.0, np.array([2.0, 3.0], np.float32))[0]
    assert yg.tolist() == [2.0, 3.0, 3.0, 3.0]


def test_swish_and_swiglu_closed_forms(orc):
    assert orc.swish(0.0) == 0.0
    assert abs(orc.swish(1.0) - 0.7310585786300049) < 1e-7
    assert abs(orc.swish(-1.0) + 0.2689414213699951) < 1e-7
    assert orc.swish(30.0) == pytest.approx(30.0, rel=1e-12)
    assert abs(orc.swish(-30.0)) < 1e-11
    g = np.array([0.0, 1.0, -1.0, 2.0], np.float32)
    u = np.array([5.0, 2.0, -3.0, 0.0], np.float32)
    out = orc.swiglu(g, u)
    np.testing.assert_allclose(out, [0.0, 2 * 0.7310585786300049, 3 * 0.2689414213699951, 0.0],
                               rtol=1e-6)


# ---------------------------------------------------------------- argmax

def test_argmax_reference_kats(orc):
    kat = KATS["argmax_linear"]
    v = -np.arange(kat["vocabulary"], dtype=np.float32)
    v[kat["expected"]] = 100.0
    assert orc.argmax_rows(v)[0] == kat["expected"]
    kat = KATS["argmax_tiled_pack4"]
    v = -(np.arange(kat["vocabulary"], dtype=np.float32) + 1)
    v[kat["expected"]] = 100.0
    # tiled Pack4 storage of one row is the linear row padded to whole packs
    packs = -(-kat["vocabulary"] // 4)
    tile_rows = -(-packs // kat["tile_width_packs"])
    storage = np.zeros(tile_rows * kat["tile_width_packs"] * 4, np.float32)
    storage[:kat["vocabulary"]] = v
    assert orc.argmax_rows(storage[None, :], width=kat["vocabulary"])[0] == kat["expected"]


def test_argmax_tie_and_nan_rules(orc):
    assert orc.argmax_rows(np.array([1.0, 5.0, 5.0, 2.0], np.float32))[0] == 1
    assert orc.argmax_rows(np.array([5.0, 5.0], np.float32))[0] == 0
    assert orc.argmax_rows(np.array([np.nan, 5.0, 7.0], np.float32))[0] == 0
    assert orc.argmax_rows(np.array([1.0, np.nan, 0.5], np.float32))[0] == 0
    assert orc.argmax_rows(np.array([1.0, np.nan, 3.0], np.float32))[0] == 2
    assert orc.argmax_rows(np.full(5, -np.inf, np.float32))[0] == 0
    # width masks the padded tail
    assert orc.argmax_rows(np.array([[1.0, 2.0, 9.0]], np.float32), width=2)[0] == 1
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 1000)).astype(np.float32)
    x[3, 10] = x[3, 900] = 50.0
    assert np.array_equal(orc.argmax_rows(x), np.argmax(x, axis=1))   # numpy: first occurrence


# ---------------------------------------------------------------- archive

def test_archive_header_round_trip_and_rejects(orc):
    h = orc.archive_header(8, 256, 3, 12345)
    assert len(h) == 32
    assert h[:8] == (0x0038544547535141).to_bytes(8, "little")
    assert orc.archive_parse_header(h) == (0, 8, 256, 3)
    bad = bytearray(h); bad[0] ^= 1
    assert orc.archive_parse_header(bytes(bad))[0] != 0
    bad = bytearray(h); bad[8] = 2
    assert orc.archive_parse_header(bytes(bad))[0] != 0
    bad = bytearray(h); bad[12] = 5
    assert orc.archive_parse_header(bytes(bad))[0] != 0
    assert orc.archive_parse_header(orc.archive_header(0, 16, 0, 0))[:2] == (0, 8)


def test_q8_record_round_trip_reference_bound(orc):
    kat = KATS["q8_record_round_trip"]
    i = np.arange(kat["count"], dtype=np.float64)
    v = (np.sin(i * 0.017).astype(np.float32) * (1 + i % 13).astype(np.float32)).astype(np.float32)
    rec = orc.record_write_q8(v, kat["block"])
    assert int.from_bytes(rec[16:20], "little") == kat["count"] + 33 * 4   # payload
    rc, restored, used = orc.record_read_array(rec, kat["count"])
    assert rc == 0 and used == len(rec)
    assert float(np.abs(restored - v).max()) <= 13 / 127 + 1e-6
    # the packed reader and the GPU unpack agree with the float reader bit for bit
    rc, packed, scales, blk, _ = orc.record_read_q8_packed(rec, kat["count"])
    assert rc == 0 and blk == 256 and scales.size == 33
    codes = packed.view(np.int8)[:kat["count"]].astype(np.float32)
    assert np.array_equal(codes * np.repeat(scales, 256)[:kat["count"]], restored)


def test_raw_record_bit_exact(orc):
    kat = KATS["raw_record_bit_exact"]
    vals = np.array([int(b, 16) for b in kat["values_f32_bits"]], np.uint32).view(np.float32)
    rec = orc.record_write_raw_f32(vals)
    rc, back, _ = orc.record_read_array(rec, vals.size)
    assert rc == 0 and np.array_equal(back.view(np.uint32), vals.view(np.uint32))
    # element count mismatch is rejected
    assert orc.record_read_array(rec, vals.size + 1)[0] != 0


def test_q8_row_wise_packed_one_scale_per_row(orc):
    kat = KATS["q8_row_wise_packed"]
    r, c = np.meshgrid(np.arange(kat["rows"]), np.arange(kat["cols"]), indexing="ij")
    v = ((r + 1) * (c - 3.5)).astype(np.float32)
    rec = orc.record_write_q8(v, kat["cols"])
    rc, packed, scales, blk, _ = orc.record_read_q8_packed(rec, v.size, kat["cols"])
    assert rc == 0 and scales.size == kat["expected_scale_count"]
    assert packed.size == kat["expected_packed_words"]
    # block mismatch is rejected (Q8A:345-346)
    assert orc.record_read_q8_packed(rec, v.size, 4)[0] != 0


@pytest.mark.parametrize("block", [16, 32, 7])
def test_q4_record_round_trip_and_two_decoders_agree(orc, block):
    rng = np.random.default_rng(block)
    n = 16 * 64 + 5
    v = rng.standard_normal(n).astype(np.float32)
    rec = orc.record_write_q4(v, block)
    rc, back, used = orc.record_read_array(rec, n)
    assert rc == 0 and used == len(rec)
    nb = -(-n // block)
    scale = np.array([np.abs(v[b * block:(b + 1) * block]).max() / np.float32(7) for b in range(nb)],
                     np.float32)
    assert np.all(np.abs(back - v) <= np.repeat(scale, block)[:n] * 0.5 + 1e-7)
    rc, packed, scales, blk, _ = orc.record_read_q4_packed(rec, n)
    assert rc == 0 and blk == block
    np.testing.assert_array_equal(scales, scale)
    if n % block == 0 or True:
        # MM:712-720 unpack over the packed words equals the CPU reader (Q8A:329-334)
        k = n  # one "row" of n elements
        gpu = orc.dequant_q4(packed, scales, 1, k, block, orc.NIBBLE_TWOS)[0]
        assert np.array_equal(gpu, back)


def test_q4_from_q8_rows_group16(orc):
    rng = np.random.default_rng(9)
    rows, width = 5, 64
    w = rng.standard_normal((rows, width)).astype(np.float32)
    q8, s8 = orc.q8_pack_rows(w, rows, width)
    rec = orc.record_write_q4_from_q8_rows(q8, s8, rows, width, 16)
    rc, packed, scales, blk, _ = orc.record_read_q4_packed(rec, rows * width, 16)
    assert rc == 0 and blk == 16 and scales.size == rows * width // 16
    q4 = orc.dequant_q4(packed, scales, rows, width, 16)
    q8f = orc.dequant_q8(q8, s8, rows, width)
    # each Q4 value is within half a Q4 step of the Q8 value it came from
    step = np.repeat(scales.reshape(rows, -1), 16, axis=1)
    assert np.all(np.abs(q4 - q8f) <= step * 0.5 + 1e-6)
    with pytest.raises(ValueError):
        orc.record_write_q4_from_q8_rows(q8, s8, rows, width, 24)


# ---------------------------------------------------------------- decode-step oracle functions

def test_rope_table_and_rotation_properties(orc):
    """Rotate-half RoPE (PN:414-473): position 0 is the identity, every (j, j+d/2)
    pair keeps its norm, and <rope(q, a), rope(k, b)> depends only on a - b."""
    d = 128
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, d)).astype(np.float32)
    c0, s0 = orc.rope_table(0, d, 1e6)
    assert np.array_equal(c0, np.ones(d // 2, np.float32)) and np.array_equal(s0, np.zeros(d // 2, np.float32))
    assert np.array_equal(orc.rope_rotate_half(x, c0, s0), x)
    c, s = orc.rope_table(1234, d, 1e6)
    y = orc.rope_rotate_half(x, c, s)
    half = d // 2
    np.testing.assert_allclose(x[:, :half] ** 2 + x[:, half:] ** 2, y[:, :half] ** 2 + y[:, half:] ** 2,
                               rtol=1e-5)
    # frequency of pair j is base^(-2j/d): pair 0 turns by exactly `position` radians
    assert abs(float(c[0]) - np.cos(1234.0)) < 1e-6 and abs(float(s[0]) - np.sin(1234.0)) < 1e-6
    q, k = x[0:1], x[1:2]

    def dot_at(a, b):
        ca, sa = orc.rope_table(a, d, 1e6)
        cb, sb = orc.rope_table(b, d, 1e6)
        return float(np.dot(orc.rope_rotate_half(q, ca, sa)[0].astype(np.float64),
                            orc.rope_rotate_half(k, cb, sb)[0].astype(np.float64)))
    assert abs(dot_at(10, 3) - dot_at(107, 100)) < 1e-3 * abs(dot_at(10, 3)) + 1e-3


def test_rope_rotation_direction_closed_form(orc):
    """PN:414-473 (non-interleaved): first = x0 cos - x1 sin, second = x0 sin +
    x1 cos for the pair (j, j + d/2).  A quarter turn (cos 0, sin 1) sends e_j
    to e_{j+d/2} and e_{j+d/2} to -e_j; a sign flip of either sin term, or the
    pair partner taken as j + 1 (interleaved), fails one of these."""
    d, half = 8, 4
    c = np.zeros(half, np.float32)
    s = np.ones(half, np.float32)
    for j in (0, 1, half - 1):
        e_j = np.zeros((1, d), np.float32)
        e_j[0, j] = 1.0
        want = np.zeros((1, d), np.float32)
        want[0, j + half] = 1.0
        assert np.array_equal(orc.rope_rotate_half(e_j, c, s), want), j
        e_p = np.zeros((1, d), np.float32)
        e_p[0, j + half] = 1.0
        want = np.zeros((1, d), np.float32)
        want[0, j] = -1.0
        assert np.array_equal(orc.rope_rotate_half(e_p, c, s), want), j
    # a half turn negates every element whatever the sin convention
    assert np.array_equal(orc.rope_rotate_half(np.arange(1, d + 1, dtype=np.float32)[None],
                                               -np.ones(half, np.float32), np.zeros(half, np.float32)),
                          -np.arange(1, d + 1, dtype=np.float32)[None])


@pytest.mark.parametrize("head_dim,base", [(128, 1e6), (64, 1e7)])
def test_rope_table_frequency_schedule(orc, head_dim, base):
    """DEC:1660-1675: pair j turns by position / base^(2j/d).  Position 1 gives
    the inverse frequency itself (below pi, so atan2 recovers it); it is
    checked at j = 1, d/4 and d/2 - 1 against exp(-2j/d * ln base) evaluated
    here in float64 (float32 rounding of the reference's steps is within
    2e-6 relative).  A larger position checks that angles scale with it."""
    half = head_dim // 2
    c1, s1 = orc.rope_table(1, head_dim, base)
    for j in (1, head_dim // 4, half - 1):
        want = math.exp(-2.0 * j / head_dim * math.log(base))
        got = math.atan2(float(s1[j]), float(c1[j]))
        assert abs(got - want) <= 2e-6 * want + 1e-9, (j, got, want)
    pos = 1537
    cp, sp = orc.rope_table(pos, head_dim, base)
    for j in (1, head_dim // 4, half - 1):
        ang = pos * math.exp(-2.0 * j / head_dim * math.log(base))
        # the angle is formed in float32: its rounding (<= 2^-24 relative) bounds the error
        tol = abs(ang) * 2.0 ** -22 + 1e-6
        assert abs(float(cp[j]) - math.cos(ang)) <= tol and abs(float(sp[j]) - math.sin(ang)) <= tol, j
    # j = 0 turns by exactly `position` radians (float(position) is exact)
    assert float(cp[0]) == np.float32(math.cos(pos)) and float(sp[0]) == np.float32(math.sin(pos))


def test_sdpa_decode_properties(orc):
    """SDPA (MM:420-544) without retyping it: equal keys give the mean of the
    values, one position gives its value row, a dominant score selects its row,
    adding a constant to every score changes nothing, and query heads of one
    key group with equal queries give equal outputs."""
    rng = np.random.default_rng(6)
    d, L = 8, 5
    v = rng.standard_normal((1, L, d)).astype(np.float32)
    q = rng.standard_normal((2, d)).astype(np.float32)
    k_eq = np.repeat(rng.standard_normal((1, 1, d)).astype(np.float32), L, axis=1)
    out = orc.sdpa_decode(q, k_eq, v, 0.7)
    np.testing.assert_allclose(out, np.repeat(v[0].mean(0, keepdims=True), 2, 0), rtol=1e-6, atol=1e-7)
    out1 = orc.sdpa_decode(q, k_eq[:, :1], v[:, :1], 0.7)
    np.testing.assert_allclose(out1, np.repeat(v[0, :1], 2, 0), rtol=1e-6)
    k = rng.standard_normal((1, L, d)).astype(np.float32) * 0.01
    k[0, 3] = q[0] * 50.0
    sel = orc.sdpa_decode(q[:1], k, v, 1.0)
    np.testing.assert_allclose(sel[0], v[0, 3], rtol=1e-6, atol=1e-6)
    # shift: a key offset orthogonal... use a constant direction e with q.e = c for every key
    e = np.zeros(d, np.float32); e[0] = 1.0
    qq = np.zeros((1, d), np.float32); qq[0, 0] = 2.0; qq[0, 1:] = rng.standard_normal(d - 1)
    kk = rng.standard_normal((1, L, d)).astype(np.float32); kk[0, :, 0] = 0.0
    a = orc.sdpa_decode(qq, kk, v, 0.5)
    b = orc.sdpa_decode(qq, kk + 3.0 * e, v, 0.5)       # every score + 0.5 * 2 * 3
    np.testing.assert_allclose(a, b, rtol=1e-9)
    # GQA: heads 0..3 share key head 0, heads 4..7 key head 1
    q8 = np.repeat(rng.standard_normal((1, d)).astype(np.float32), 8, 0)
    k2 = rng.standard_normal((2, L, d)).astype(np.float32)
    v2 = rng.standard_normal((2, L, d)).astype(np.float32)
    o = orc.sdpa_decode(q8, k2, v2, 0.3)
    assert np.all(o[:4] == o[0]) and np.all(o[4:] == o[4]) and not np.allclose(o[0], o[4])
    np.testing.assert_allclose(o[0], orc.sdpa_decode(q8[:1], k2[:1], v2[:1], 0.3)[0], rtol=1e-12)


@pytest.mark.parametrize("scale", [0.37, 0.23])
def test_sdpa_decode_score_scale_closed_form(orc, scale):
    """MM:477 multiplies each score q.k by the scale before the softmax.  Two
    positions with scores s1, s2 give (v1 e^(a s1) + v2 e^(a s2)) / (e^(a s1) +
    e^(a s2)) with a = scale, computed here in float64 from hand-chosen keys:
    q = (1, 2, 0, 0), k1 = (3, 0, 0, 0) (s1 = 3), k2 = (0, -1, 0, 0) (s2 = -2).
    A dropped, inverted or squared scale moves the output well past the
    tolerance at both scales."""
    q = np.array([[1.0, 2.0, 0.0, 0.0]], np.float32)
    k = np.array([[[3.0, 0.0, 0.0, 0.0], [0.0, -1.0, 0.0, 0.0]]], np.float32)
    v = np.array([[[1.0, -2.0, 0.5, 4.0], [-3.0, 1.0, 2.0, 0.25]]], np.float32)
    s1, s2 = 3.0, -2.0

    def expect(a):
        e1, e2 = math.exp(a * s1), math.exp(a * s2)
        return (v[0, 0].astype(np.float64) * e1 + v[0, 1].astype(np.float64) * e2) / (e1 + e2)

    got = orc.sdpa_decode(q, k, v, scale)[0].astype(np.float64)
    np.testing.assert_allclose(got, expect(scale), rtol=2e-6, atol=2e-6)
    for wrong in (1.0, 1.0 / scale, scale * scale):
        assert np.max(np.abs(expect(wrong) - expect(scale))) > 1e-2, wrong
    assert np.max(np.abs(got - orc.sdpa_decode(q, k, v, 1.0)[0])) > 1e-2


def test_head_packed_layout_positions(orc):
    """The attention head-packed layout against texel positions worked out by
    hand from MM:1192-1318 (texel (dim, row, head / 4), lane head % 4, lanes of
    missing heads 0): 6 heads of 3 dims over 2 rows fill two slices, the second
    holding heads 4 and 5 in lanes 0 and 1."""
    rows, heads, hd = 2, 6, 3
    x = np.arange(1, rows * heads * hd + 1, dtype=np.float32).reshape(rows, heads * hd)
    buf = orc.head_pack(x, heads, hd)
    assert buf.size == 48                      # 2 slices x 2 rows x 3 texels x 4 lanes
    assert buf[0] == x[0, 0]                   # row 0, head 0, d 0: slice 0, texel 0, lane 0
    assert buf[1] == x[0, 3]                   # row 0, head 1, d 0: lane 1 of that texel
    assert buf[11] == x[0, 3 * 3 + 2]          # row 0, head 3, d 2: texel 2, lane 3
    assert buf[18] == x[1, 2 * 3 + 1]          # row 1, head 2, d 1: texel 3 + 1, lane 2
    assert buf[45] == x[1, 5 * 3 + 2]          # row 1, head 5, d 2: slice 1, texel 3 + 2, lane 1
    tail = buf[24:].reshape(rows, hd, 4)
    assert np.all(tail[:, :, 2:] == 0)         # heads 6 and 7 do not exist
    assert np.array_equal(orc.head_unpack(buf, rows, heads, hd), x)
    # four heads exactly fill one slice: every lane is a value
    y = np.arange(1, 3 * 4 * 5 + 1, dtype=np.float32).reshape(3, 20)
    b2 = orc.head_pack(y, 4, 5)
    assert b2.size == 60 and np.all(b2 != 0)
    assert np.array_equal(orc.head_unpack(b2, 3, 4, 5), y)
