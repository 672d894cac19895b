"""Sharded model assets (aiimage_amd.assets) on the CPU: the manifest reader's
checks and the shard stream, mirroring Qwen35MobileAssetSet (MAS:50-158,
461-558) and its test Qwen35Q8ArchiveTests.ManifestBackedShardStreamSeeksAcrossPartBoundary
(TQ8:199-235); the AQSGET8 walk over a sharded archive with records written by
the oracle's restatement of the archive writer."""
import hashlib
import io
import json
import os

import numpy as np
import pytest

from aiimage_amd import assets


def _part(root, rel, data):
    path = os.path.join(root, rel)
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "wb") as f:
        f.write(data)
    return {"file": rel, "bytes": len(data), "sha256": hashlib.sha256(data).hexdigest()}


def _manifest(root, files, schema=assets.MANIFEST_SCHEMA, name=assets.MANIFEST_FILE, **extra):
    doc = {"schema": schema, "weight_only": True, "logical_files": files}
    doc.update(extra)
    with open(os.path.join(root, name), "w") as f:
        json.dump(doc, f)


def test_shard_stream_seeks_across_part_boundary(tmp_path):
    root = str(tmp_path)
    p0 = _part(root, "weights/p0", bytes([1, 2, 3]))
    p1 = _part(root, "weights/p1", bytes([4, 5, 6, 7]))
    _manifest(root, {"test.bin": {"stored_bytes": 7, "parts": [p0, p1]}})
    a = assets.MobileAssetSet.try_load(root, verify_hashes=True)
    assert a.contains("test.bin") and a.stored_bytes("test.bin") == 7 and a.stored_weight_bytes == 7
    with a.open_read("test.bin") as s:
        s.seek(2)
        assert s.read(4) == bytes([3, 4, 5, 6])
        s.seek(-1, io.SEEK_END)
        assert s.read(5) == bytes([7])
        assert s.read(1) == b""
        with pytest.raises(OSError):
            s.seek(8)


def test_manifest_choice_and_rejections(tmp_path):
    root = str(tmp_path)
    assert assets.MobileAssetSet.try_load(root) is None
    p = _part(root, "a/p0", b"abcd")
    good = {"x.bin": {"stored_bytes": 4, "parts": [p]}}

    def load(files, **kw):
        _manifest(root, files, **kw)
        return assets.MobileAssetSet.try_load(root, verify_hashes=True)

    assert load(good).quantization_bits == 8
    with pytest.raises(assets.InvalidDataError):
        load(good, schema="qwen35.mobile-q8-assets/v2")
    with pytest.raises(assets.InvalidDataError):
        load(good, quantization_bits=6)
    with pytest.raises(assets.InvalidDataError):
        load({"x.bin": {"stored_bytes": 0, "parts": []}})
    with pytest.raises(assets.InvalidDataError):
        load({"x.bin": {"stored_bytes": 4, "parts": [dict(p, bytes=5)]}})
    with pytest.raises(assets.InvalidDataError):
        load({"x.bin": {"stored_bytes": 4, "parts": [dict(p, sha256="ab")]}})
    with pytest.raises(assets.InvalidDataError):
        load({"x.bin": {"stored_bytes": 4, "parts": [dict(p, sha256="0" * 64)]}})
    with pytest.raises(assets.InvalidDataError):
        load({"x.bin": {"stored_bytes": 4, "parts": [dict(p, file="../outside")]}})
    with pytest.raises(assets.InvalidDataError):
        load({"x.bin": {"stored_bytes": 4, "parts": [dict(p, file=os.path.join(root, "a/p0"))]}})
    with pytest.raises(FileNotFoundError):
        load({"x.bin": {"stored_bytes": 4, "parts": [dict(p, file="a/missing")]}})
    with pytest.raises(assets.InvalidDataError):
        load({"x.bin": {"stored_bytes": 5, "parts": [p]}})
    # without hash verification a wrong (well-formed) digest is not read
    _manifest(root, {"x.bin": {"stored_bytes": 4, "parts": [dict(p, sha256="0" * 64)]}})
    assert assets.MobileAssetSet.try_load(root, verify_hashes=False).contains("x.bin")
    # the Q4 manifest wins when both exist (MAS:56-59)
    _manifest(root, good, schema=assets.Q4_MANIFEST_SCHEMA, name=assets.Q4_MANIFEST_FILE)
    a = assets.MobileAssetSet.try_load(root)
    assert a.quantization_bits == 4 and a.manifest_path.endswith(assets.Q4_MANIFEST_FILE)
    with pytest.raises(FileNotFoundError):
        a.open_read("y.bin")


class _RecordCtx:
    """Stands in for the device context: returns each record as loaded."""

    def weight_from_record(self, record, n, k, bits):
        return (bytes(record), n, k, bits), len(record)


def test_sharded_archive_walk(tmp_path, orc):
    """An archive of three records split into shards at boundaries that fall
    inside records: the stream reassembles it and the walk hands each record,
    whole, to the loader in model order."""
    root = str(tmp_path)
    rng = np.random.default_rng(5)
    shapes = [(16, 64, 4), (24, 32, 8), (8, 48, 4)]
    recs = []
    for n, k, bits in shapes:
        v = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
        recs.append(orc.record_write_q4(v, 16) if bits == 4 else orc.record_write_q8(v, k))
    blob = orc.archive_header(4, 16, len(recs), 4242) + b"".join(recs)
    cuts = [0, 7, 40, 41, len(blob) - 3, len(blob)]
    parts = [_part(root, "shards/part%d" % i, blob[a:b]) for i, (a, b) in enumerate(zip(cuts, cuts[1:]))]
    _manifest(root, {"model.aqs": {"stored_bytes": len(blob), "parts": parts}})
    a = assets.MobileAssetSet.try_load(root, verify_hashes=True)
    with a.open_read("model.aqs") as s:
        assert s.read() == blob
    with a.open_read("model.aqs") as s:
        ws, header = assets.load_archive_weights(_RecordCtx(), s, shapes)
    assert header == (4, 16, 3)
    assert [w[0] for w in ws] == recs
    assert [w[1:] for w in ws] == shapes
    with a.open_read("model.aqs") as s:              # more layers than records
        with pytest.raises(assets.InvalidDataError):
            assets.load_archive_weights(_RecordCtx(), s, shapes + [(8, 8, 4)])


def test_sharded_file_random_slices(tmp_path):
    """Every (offset, length) window of a logical file cut into uneven shards,
    some of one byte, reads the same bytes as the concatenation."""
    root = str(tmp_path)
    rng = np.random.default_rng(11)
    blob = rng.integers(0, 256, 97, dtype=np.uint8).tobytes()
    cuts = [0, 1, 2, 30, 31, 64, 96, 97]
    parts = [_part(root, "s/%d" % i, blob[a:b]) for i, (a, b) in enumerate(zip(cuts, cuts[1:]))]
    _manifest(root, {"f": {"stored_bytes": len(blob), "parts": parts}})
    a = assets.MobileAssetSet.try_load(root, verify_hashes=True)
    with a.open_read("f") as s:
        assert len(s) == len(blob)
        for off in range(len(blob) + 1):
            for n in (0, 1, 2, 33, 200):
                s.seek(off)
                assert s.read(n) == blob[off:off + n]
                assert s.tell() == min(off + n, len(blob))
        s.seek(90)
        with pytest.raises(assets.InvalidDataError):
            s.read_exact(8)


def test_load_assets_needs_both_logical_files(tmp_path, orc):
    """decoder.load_assets refuses an asset set without the decoder archive or
    the tied embedding before touching a device."""
    import hashlib
    import json
    import os

    from aiimage_amd import assets, decoder
    blob = orc.archive_header(8, 1024, 0, 0)
    rel = "weights/e.part000"
    os.makedirs(tmp_path / "weights")
    (tmp_path / rel).write_bytes(blob)
    doc = {"schema": assets.Q4_MANIFEST_SCHEMA, "weight_only": True,
           "logical_files": {decoder.EMBED_FILE: {"stored_bytes": len(blob), "parts": [
               {"file": rel, "bytes": len(blob), "sha256": hashlib.sha256(blob).hexdigest()}]}}}
    (tmp_path / assets.Q4_MANIFEST_FILE).write_text(json.dumps(doc))
    with pytest.raises(assets.InvalidDataError, match=decoder.DECODER_FILE):
        decoder.load_assets(None, str(tmp_path), decoder.ModelConfig(layers=1))
    with pytest.raises(assets.InvalidDataError, match="no mobile asset manifest"):
        decoder.load_assets(None, str(tmp_path / "weights"), decoder.ModelConfig(layers=1))


def test_read_float_record_rules(orc):
    """Raw fp32 records read back exactly; a quantized record, a wrong count, a
    bad magic and a short payload are refused (Q8A:295-306, 445-463)."""
    import io
    import struct

    import numpy as np

    from aiimage_amd import assets
    v = np.array([1.5, -2.25, 3e-8, 65504.0, -0.0], np.float32)
    rec = orc.record_write_raw_f32(v)
    got = assets.read_float_record(io.BytesIO(rec), v.size)
    assert np.array_equal(got.view(np.uint32), v.view(np.uint32))
    with pytest.raises(assets.InvalidDataError, match="element count"):
        assets.read_float_record(io.BytesIO(rec), v.size + 1)
    with pytest.raises(assets.InvalidDataError, match="raw FP32"):
        assets.read_float_record(io.BytesIO(orc.record_write_q8(np.ones(8, np.float32), 8)), 8)
    bad = bytearray(rec)
    bad[0] ^= 1
    with pytest.raises(assets.InvalidDataError, match="magic"):
        assets.read_float_record(io.BytesIO(bytes(bad)), v.size)
    with pytest.raises(assets.InvalidDataError):
        assets.read_float_record(io.BytesIO(rec[:-1]), v.size)
    bad = bytearray(rec)
    struct.pack_into("<i", bad, 16, 4 * v.size + 4)
    with pytest.raises(assets.InvalidDataError, match="size mismatch"):
        assets.read_float_record(io.BytesIO(bytes(bad)), v.size)
