"""AQSGET8 record -> device weight (aexq_weight_from_record) against the CPU
oracle's restatement of the archive reader (NcnnQ8Archive.cs).

Bars: the device dequantization of a loaded record is bit-exact with the
reader's float32 values (ReadArray, Q8A:295-339) -- and with the packed-array
readers fed through the direct upload; records of another kind are quantized
per output row exactly as the float overloads do; a matvec through a loaded
record is within 1e-3 normwise of the float64 oracle; malformed records fail
with the reader's exception class (InvalidDataError / ArgumentError).
"""
import struct
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


def _values(n, k, seed):
    rng = np.random.default_rng(seed)
    v = rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.05)
    v[0, :] = 0.0                       # an all-zero block: scale 1 in the writer
    return v


def _same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("n,k,block", [(96, 256, 16), (64, 1024, 32), (33, 245, 5), (8, 64, 64)])
def test_q4_record_direct_bit_exact(ctx, aexq, orc, n, k, block):
    _announce(f"q4 record n={n} k={k} block={block}")
    rec = orc.record_write_q4(_values(n, k, n + k + block), block)
    w, used = ctx.weight_from_record(rec, n, k, bits=4)
    assert used == len(rec)
    info = w.info()
    assert (info.bits, info.block, info.scale_dtype) == (4, block, aexq.DTYPE_F32)
    got = ctx.dequant(w).cpu().numpy()
    rc, ref, _ = orc.record_read_array(rec, n * k)
    assert rc == 0
    assert _same_bits(got, ref.reshape(n, k))
    # the same record through the packed reader and the direct packed upload
    rc, packed, scales, blk, _ = orc.record_read_q4_packed(rec, n * k)
    assert rc == 0 and blk == block
    w2 = ctx.weight(aexq.QuantizedTensor(n * k, block, packed, scales, bits=4,
                                         nibble_code=aexq.NIBBLE_TWOS), n, k)
    assert _same_bits(ctx.dequant(w2).cpu().numpy(), got)


@pytest.mark.parametrize("n,k", [(100, 1024), (7, 37)])
def test_q8_record_direct_bit_exact(ctx, aexq, orc, n, k):
    _announce(f"q8 record n={n} k={k}")
    rec = orc.record_write_q8(_values(n, k, 3 * n + k), k)
    w, used = ctx.weight_from_record(rec, n, k, bits=8)
    assert used == len(rec)
    got = ctx.dequant(w).cpu().numpy()
    rc, ref, _ = orc.record_read_array(rec, n * k)
    assert rc == 0
    assert _same_bits(got, ref.reshape(n, k))


@pytest.mark.parametrize("kind,bits", [("raw", 8), ("raw", 4), ("q8", 4), ("q4", 8)])
def test_other_records_quantized_per_row(ctx, aexq, orc, kind, bits):
    """A record of another kind is read as float32 and quantized per output row
    (GL:60-141): identical to the oracle's packer on ReadArray's values."""
    _announce(f"record {kind} as bits={bits}")
    n, k = 48, 160
    v = _values(n, k, 11 + bits)
    rec = {"raw": lambda: orc.record_write_raw_f32(v),
           "q8": lambda: orc.record_write_q8(v, 32),
           "q4": lambda: orc.record_write_q4(v, 16)}[kind]()
    w, used = ctx.weight_from_record(rec, n, k, bits=bits)
    assert used == len(rec)
    rc, floats, _ = orc.record_read_array(rec, n * k)
    assert rc == 0
    floats = floats.reshape(n, k)
    if bits == 8:
        packed, scales = orc.q8_pack_rows(floats, n, k, True)
        ref = orc.dequant_q8(packed, scales, n, k, scale_dtype=orc.SCALE_F32)
    else:
        packed, scales, blk = orc.q4_pack_rows(floats, n, k, True)
        ref = orc.dequant_q4(packed, scales, n, k, blk, orc.NIBBLE_TWOS, orc.SCALE_F32)
    assert _same_bits(ctx.dequant(w).cpu().numpy(), ref)


def test_shipping_q4_from_q8_rows_matvec(ctx, aexq, orc):
    """The shipping Q4 (group 16, converted from Q8 rows, Q8A:167-207) at the
    q_proj shape: loaded from its record, one matvec against the oracle."""
    _announce("shipping q4 record matvec")
    from aiimage_amd import synth
    n, k = 2048, 1024
    q8p, q8s = orc.q8_pack_rows(_values(n, k, 21), n, k, True)
    rec = orc.record_write_q4_from_q8_rows(q8p, q8s, n, k, 16)
    w, _ = ctx.weight_from_record(rec, n, k, bits=4)
    rc, wf, _ = orc.record_read_array(rec, n * k)
    assert rc == 0
    x16 = synth.activations(1, k, 22)
    y = aexq.new_activation(1, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
    ctx.linear(w, aexq.describe(torch.as_tensor(x16).cuda(), 1, k),
               aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR))
    torch.cuda.synchronize()
    ref = orc.gemm_gpu_semantics(x16.astype(np.float32), wf.reshape(n, k))[0]
    assert normwise(y.cpu().numpy()[:n], ref) <= TOL


def test_archive_walk_consumes_each_record(ctx, aexq, orc):
    """Header + three records in one buffer: each load reports its record's
    size, so a host walks the archive by offsets."""
    _announce("archive walk")
    shapes = [(16, 64, 4, 16), (24, 32, 8, 32), (8, 48, 4, 48)]
    recs = []
    for i, (n, k, bits, blk) in enumerate(shapes):
        v = _values(n, k, 40 + i)
        recs.append(orc.record_write_q4(v, blk) if bits == 4 else orc.record_write_q8(v, blk))
    buf = orc.archive_header(4, 16, len(recs), 12345) + b"".join(recs)
    assert aexq.archive_header(buf[:32]) == (4, 16, 3)
    off = 32
    for (n, k, bits, _), rec in zip(shapes, recs):
        w, used = ctx.weight_from_record(buf[off:], n, k, bits=bits)
        rc, ref, _ = orc.record_read_array(rec, n * k)
        assert _same_bits(ctx.dequant(w).cpu().numpy(), ref.reshape(n, k))
        off += used
    assert off == len(buf)


def test_malformed_records_are_rejected(ctx, aexq, orc):
    _announce("malformed records")
    from aiimage_amd import _abi
    n, k = 8, 64
    v = _values(n, k, 50)
    q4 = orc.record_write_q4(v, 16)
    q8 = orc.record_write_q8(v, 16)
    with pytest.raises(_abi.InvalidDataError):          # Q8 block must equal K
        ctx.weight_from_record(q8, n, k, bits=8)
    with pytest.raises(_abi.InvalidDataError):          # element count mismatch
        ctx.weight_from_record(q4, n, k // 2, bits=4)
    with pytest.raises(_abi.InvalidDataError):          # truncated payload
        ctx.weight_from_record(q4[:-3], n, k, bits=4)
    bad = bytearray(q4)
    bad[0] ^= 0xFF                                       # record magic
    with pytest.raises(_abi.InvalidDataError):
        ctx.weight_from_record(bytes(bad), n, k, bits=4)
    bad = bytearray(q4)
    struct.pack_into("<i", bad, 16, len(q4) - 24 - 1)    # payload field one short
    with pytest.raises(_abi.InvalidDataError):
        ctx.weight_from_record(bytes(bad), n, k, bits=4)
    q4_g24 = orc.record_write_q4(_values(4, 48, 51), 24)
    with pytest.raises(_abi.ArgumentError):             # group must divide K
        ctx.weight_from_record(q4_g24, 6, 32, bits=4)


def test_sharded_archive_into_device_weights(ctx, aexq, orc, tmp_path):
    """A manifest-backed, sharded AQSGET8 archive (MAS:50-158) walked into device
    weights record by record: each dequantises bit-exactly to the oracle's reader."""
    _announce("sharded archive load")
    import hashlib
    import json
    import os
    from aiimage_amd import assets
    shapes = [(64, 256, 4), (40, 128, 8), (32, 64, 4)]
    recs = []
    for i, (n, k, bits) in enumerate(shapes):
        v = _values(n, k, 60 + i)
        recs.append(orc.record_write_q4(v, 32) if bits == 4 else orc.record_write_q8(v, k))
    blob = orc.archive_header(4, 32, len(recs), 777) + b"".join(recs)
    root = str(tmp_path)
    cuts = [0, 100, 5000, len(blob)]
    parts = []
    for j, (a, b) in enumerate(zip(cuts, cuts[1:])):
        rel = "w/shard%d.bin" % j
        os.makedirs(os.path.join(root, "w"), exist_ok=True)
        with open(os.path.join(root, rel), "wb") as f:
            f.write(blob[a:b])
        parts.append({"file": rel, "bytes": b - a, "sha256": hashlib.sha256(blob[a:b]).hexdigest()})
    with open(os.path.join(root, assets.Q4_MANIFEST_FILE), "w") as f:
        json.dump({"schema": assets.Q4_MANIFEST_SCHEMA, "weight_only": True,
                   "logical_files": {"decoder.aqs": {"stored_bytes": len(blob), "parts": parts}}}, f)
    a = assets.MobileAssetSet.try_load(root, verify_hashes=True)
    with a.open_read("decoder.aqs") as s:
        ws, header = assets.load_archive_weights(ctx, s, shapes)
    assert header == (4, 32, 3)
    for (n, k, _), rec, w in zip(shapes, recs, ws):
        rc, ref, _ = orc.record_read_array(rec, n * k)
        assert rc == 0
        assert _same_bits(ctx.dequant(w).cpu().numpy(), ref.reshape(n, k))
        w.release()
