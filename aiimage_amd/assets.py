"""Sharded model assets and the archive-to-device loader (host side).

The reference ships its quantized weights as "logical files" (an AQSGET8
archive, for instance) cut into shard files and described by a JSON manifest
(Samples/AIImageApplicationExample/Runtime/Scripts/Qwen35MobileAssetSet.cs,
cited as MAS:line).  What the format fixes is kept here exactly: the two
manifest file names and schema strings (MAS:15-20), the JSON keys
(`schema`, `weight_only`, `quantization_bits`, `logical_files`, and per part
`file`, `bytes`, `sha256`, per logical file `stored_bytes`), the preference of
the Q4 manifest over the Q8 one (MAS:56-59), the rule that shard paths are
relative and stay inside the model directory (MAS:173-181), and the size,
digest and stored-byte checks (MAS:76-138).

The reader is this module's own design:

* `read_manifest` turns the document into an immutable `AssetManifest` of
  `LogicalFile`s, each a tuple of `Shard(path, size, sha256)`; every rule is a
  small checker that raises `InvalidDataError` with a message naming the
  manifest, the logical file and the rule.
* `ShardedFile` reads a logical file with positional reads (`os.preadv`) on
  a table of shard descriptors opened on first use: a read is cut into
  per-shard spans (`_spans`), so there is no per-shard cursor to keep in step
  and `seek` is a plain assignment.

`load_archive_weights` then walks an AQSGET8 archive from such a stream, record
by record, into device weights (`aexq_weight_from_record`), in the model order
the Gemm layers read their weights.

Not provided: the reference's on-disk cache of verified digests (MAS:195-296),
which only saves re-hashing between runs.
"""
from __future__ import annotations

import bisect
import hashlib
import io
import json
import os
import struct
from typing import Dict, Iterator, NamedTuple, Optional, Sequence, Tuple

from . import _abi

MANIFEST_FILE = "qwen3.5_mobile_q8_assets.json"       # MAS:15
MANIFEST_SCHEMA = "qwen35.mobile-q8-assets/v1"        # MAS:16
Q4_MANIFEST_FILE = "qwen3.5_mobile_q4_assets.json"    # MAS:19
Q4_MANIFEST_SCHEMA = "qwen35.mobile-q4-assets/v1"     # MAS:20
_DEFAULT_BITS = {MANIFEST_SCHEMA: 8, Q4_MANIFEST_SCHEMA: 4}

ARCHIVE_HEADER_BYTES = 32   # AQSGET8 archive header (Q8A:26-33)
RECORD_HEADER_BYTES = 24    # record header; payload byte count at offset 16 (Q8A:60-65)
RECORD_MAGIC = 0x31523851   # "Q8R1" (Q8A:28)
RECORD_RAW = 2              # raw fp32 record kind (Q8A:32)

_HASH_BLOCK = 8 << 20


class InvalidDataError(_abi.InvalidDataError):
    """A manifest or archive that breaks the format (the reference raises
    InvalidDataException for the same conditions)."""

    def __init__(self, message: str):
        super().__init__(_abi.ERR_FORMAT, message)


class Shard(NamedTuple):
    path: str       # absolute path, inside the model directory
    size: int       # bytes, as the manifest declares and the file holds
    sha256: str     # lower-case hex digest


class LogicalFile(NamedTuple):
    name: str
    shards: Tuple[Shard, ...]

    @property
    def size(self) -> int:
        return sum(s.size for s in self.shards)


class AssetManifest(NamedTuple):
    path: str
    schema: str
    weight_only: bool
    quantization_bits: int
    files: Dict[str, LogicalFile]


# ----------------------------------------------------------------- checks


def _fail(manifest: str, where: str, what: str) -> InvalidDataError:
    return InvalidDataError("asset manifest %s: %s: %s" % (os.path.basename(manifest), where, what))


def _resolve_inside(root: str, rel: str, manifest: str, where: str) -> str:
    """Shard paths are relative and resolve inside the model directory (MAS:173-181)."""
    if os.path.isabs(rel):
        raise _fail(manifest, where, "shard path %r is absolute; paths are relative to %s" % (rel, root))
    full = os.path.normpath(os.path.join(root, rel))
    if os.path.commonpath([root.lower(), full.lower()]) != root.lower() or full == root:
        raise _fail(manifest, where, "shard path %r leaves the model directory %s" % (rel, root))
    return full


def _digest(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb", buffering=0) as f:
        buf = bytearray(_HASH_BLOCK)
        view = memoryview(buf)
        while True:
            n = f.readinto(buf)
            if not n:
                return h.hexdigest()
            h.update(view[:n])


def _shard(root: str, manifest: str, where: str, spec, verify: bool) -> Shard:
    if not isinstance(spec, dict):
        raise _fail(manifest, where, "a part is %s, not an object" % type(spec).__name__)
    rel = spec.get("file")
    if not isinstance(rel, str) or rel.strip() == "":
        raise _fail(manifest, where, "a part has no file name")
    path = _resolve_inside(root, rel, manifest, where)
    if not os.path.isfile(path):
        raise FileNotFoundError("asset manifest %s: %s: shard file not found"
                                % (os.path.basename(manifest), where), path)
    declared = spec.get("bytes")
    on_disk = os.path.getsize(path)
    if declared != on_disk:
        raise _fail(manifest, where, "shard %s holds %d bytes, the manifest says %r" % (rel, on_disk, declared))
    digest = str(spec.get("sha256") or "").lower()
    if len(digest) != 64:
        raise _fail(manifest, where, "shard %s has no 64-digit sha256" % rel)
    if verify:
        actual = _digest(path)
        if actual != digest:
            raise _fail(manifest, where, "shard %s hashes to %s, the manifest says %s" % (rel, actual, digest))
    return Shard(path, on_disk, digest)


def _logical_file(root: str, manifest: str, name: str, item, verify: bool) -> LogicalFile:
    where = "logical file %r" % name
    if not isinstance(item, dict):
        raise _fail(manifest, where, "entry is %s, not an object" % type(item).__name__)
    parts = item.get("parts")
    if not isinstance(parts, list) or len(parts) == 0:
        raise _fail(manifest, where, "needs a non-empty 'parts' list")
    lf = LogicalFile(name, tuple(_shard(root, manifest, where, p, verify) for p in parts))
    if item.get("stored_bytes") != lf.size:
        raise _fail(manifest, where, "its shards hold %d bytes, 'stored_bytes' says %r"
                    % (lf.size, item.get("stored_bytes")))
    return lf


def read_manifest(path: str, root: Optional[str] = None, verify_hashes: bool = False) -> AssetManifest:
    """Parse and check one manifest; shard paths resolve against `root`
    (default: the manifest's directory)."""
    root = os.path.normpath(os.path.abspath(root or os.path.dirname(path)))
    with open(path, "r", encoding="utf-8") as f:
        doc = json.load(f)
    if not isinstance(doc, dict):
        raise _fail(path, "document", "top level is not an object")
    schema = doc.get("schema")
    if schema not in _DEFAULT_BITS:
        raise _fail(path, "schema", "%r is neither %s nor %s" % (schema, MANIFEST_SCHEMA, Q4_MANIFEST_SCHEMA))
    bits = doc.get("quantization_bits")
    bits = _DEFAULT_BITS[schema] if bits is None else int(bits)
    if bits not in (4, 8):
        raise _fail(path, "quantization_bits", "%d is not 4 or 8" % bits)
    listing = doc.get("logical_files")
    if not isinstance(listing, dict):
        raise _fail(path, "logical_files", "missing, or not an object")
    files = {name: _logical_file(root, path, name, item, verify_hashes) for name, item in listing.items()}
    return AssetManifest(path, schema, bool(doc.get("weight_only", False)), bits, files)


# ----------------------------------------------------------------- the asset set


class MobileAssetSet:
    """The model directory's sharded assets, the role of the reference's
    Qwen35MobileAssetSet (MAS:13-158): `try_load`, `contains`, `open_read`,
    `stored_bytes` and the manifest's properties."""

    def __init__(self, model_directory: str, manifest: AssetManifest):
        self.model_directory = model_directory
        self._manifest = manifest

    manifest_path = property(lambda self: self._manifest.path)
    weight_only = property(lambda self: self._manifest.weight_only)
    quantization_bits = property(lambda self: self._manifest.quantization_bits)
    stored_weight_bytes = property(lambda self: sum(f.size for f in self._manifest.files.values()))

    @classmethod
    def try_load(cls, model_directory: str, verify_hashes: bool = False) -> Optional["MobileAssetSet"]:
        """The Q4 manifest when the directory has one, else the Q8 manifest,
        else None (MAS:50-66)."""
        root = os.path.normpath(os.path.abspath(model_directory or ""))
        for name in (Q4_MANIFEST_FILE, MANIFEST_FILE):
            candidate = os.path.join(root, name)
            if os.path.exists(candidate):
                return cls(root, read_manifest(candidate, root, verify_hashes))
        return None

    def contains(self, logical_name: str) -> bool:
        return bool(logical_name) and logical_name in self._manifest.files

    def logical_file(self, logical_name: str) -> LogicalFile:
        lf = self._manifest.files.get(logical_name)
        if lf is None:
            raise FileNotFoundError("%s lists no logical file %r" % (os.path.basename(self.manifest_path),
                                                                     logical_name), logical_name)
        return lf

    def open_read(self, logical_name: str) -> "ShardedFile":
        return ShardedFile(self.logical_file(logical_name).shards)

    def stored_bytes(self, logical_name: str) -> int:
        lf = self._manifest.files.get(logical_name)
        return lf.size if lf is not None else 0


class ShardedFile(io.RawIOBase):
    """A read-only, seekable view of one logical file across its shards
    (the role of MAS:461-558).  Reads are positional: a request is cut into
    per-shard spans and each span is one `os.preadv` into the caller's buffer."""

    def __init__(self, shards: Sequence[Shard]):
        super().__init__()
        if len(shards) == 0:
            raise ValueError("a logical file needs at least one shard")
        self._shards = tuple(shards)
        ends, total = [], 0
        for s in self._shards:
            total += s.size
            ends.append(total)
        self._ends = ends          # exclusive end offset of each shard
        self._size = total
        self._pos = 0
        self._fds: Dict[int, int] = {}

    def readable(self) -> bool:
        return True

    def seekable(self) -> bool:
        return True

    def __len__(self) -> int:
        return self._size

    def tell(self) -> int:
        return self._pos

    def seek(self, offset: int, whence: int = io.SEEK_SET) -> int:
        base = {io.SEEK_SET: 0, io.SEEK_CUR: self._pos, io.SEEK_END: self._size}[whence]
        target = base + offset
        if not 0 <= target <= self._size:
            raise OSError("seek to %d is outside the logical file (0..%d)" % (target, self._size))
        self._pos = target
        return target

    def _spans(self, pos: int, count: int) -> Iterator[Tuple[int, int, int]]:
        """(shard index, offset inside that shard, bytes) covering [pos, pos+count)."""
        i = bisect.bisect_right(self._ends, pos)
        while count > 0 and i < len(self._shards):
            start = self._ends[i] - self._shards[i].size
            take = min(count, self._ends[i] - pos)
            yield i, pos - start, take
            pos += take
            count -= take
            i += 1

    def _fd(self, i: int) -> int:
        fd = self._fds.get(i)
        if fd is None:
            fd = self._fds[i] = os.open(self._shards[i].path, os.O_RDONLY)
        return fd

    def readinto(self, buf) -> int:
        out = memoryview(buf).cast("B")
        done = 0
        for i, local, n in self._spans(self._pos, min(len(out), self._size - self._pos)):
            got = os.preadv(self._fd(i), [out[done:done + n]], local)
            if got != n:
                raise InvalidDataError("shard %s is shorter than its manifest entry (read %d of %d bytes at %d)"
                                       % (self._shards[i].path, got, n, local))
            done += n
        self._pos += done
        return done

    def read_exact(self, n: int) -> bytes:
        data = self.read(n)
        if data is None or len(data) != n:
            raise InvalidDataError("archive stream ended %d bytes short of a record"
                                   % (n - len(data or b"")))
        return data

    def close(self) -> None:
        for fd in self._fds.values():
            os.close(fd)
        self._fds.clear()
        super().close()


# The stream's name in the reference's vocabulary.
ShardReadStream = ShardedFile


# ----------------------------------------------------------------- archive walk


def read_archive_header(stream) -> Tuple[int, int, int]:
    """The 32-byte AQSGET8 header at the stream's position, checked as the
    reader's constructor does (Q8A:277-293): (quant_bits, default_block,
    record_count)."""
    from .aexq import archive_header
    read = stream.read_exact if hasattr(stream, "read_exact") else stream.read
    return archive_header(read(ARCHIVE_HEADER_BYTES))


def read_float_record(stream, count: int):
    """One raw fp32 record (kind 2, written by WriteFloat32Array, Q8A:216-223)
    of `count` values, as ReadArray reads it with requireRaw (Q8A:295-306): the
    RMSNorm weights and other small constants of an archive.  Returns a
    float32 numpy array."""
    import numpy as np
    read = stream.read_exact if hasattr(stream, "read_exact") else stream.read
    rh = read(RECORD_HEADER_BYTES)
    if len(rh) != RECORD_HEADER_BYTES:
        raise InvalidDataError("archive stream ends inside a record header")
    magic, kind, elements, block, payload = struct.unpack_from("<Iiiii", rh, 0)
    if magic != RECORD_MAGIC:
        raise InvalidDataError("Invalid Q8 record magic.")
    if elements != count:
        raise InvalidDataError("Q8 record element count mismatch. expected=%d actual=%d."
                               % (count, elements))
    if block <= 0 or payload < 0:
        raise InvalidDataError("Invalid Q8 record header.")
    if kind != RECORD_RAW:
        raise InvalidDataError("Expected a raw FP32 quantized archive record.")
    if payload != count * 4:
        raise InvalidDataError("Q8 raw float record size mismatch.")
    body = read(payload)
    if len(body) != payload:
        raise InvalidDataError("archive stream ends inside a record payload")
    return np.frombuffer(body, "<f4").astype(np.float32)


def load_archive_weights(ctx, stream, shapes: Sequence[Tuple[int, int, int]]):
    """Walk an AQSGET8 archive (header, then one record per Gemm weight in model
    order) from `stream` into device weights: `shapes` gives (n, k, bits) of
    each record's layer (Q8A:277-293 header, GL:60-141 per record).  Returns
    (weights, (quant_bits, default_block, record_count))."""
    header = read_archive_header(stream)
    if len(shapes) > header[2]:
        raise InvalidDataError("archive holds %d records, %d layers asked for"
                               % (header[2], len(shapes)))
    return read_weight_records(ctx, stream, shapes), header


def read_weight_records(ctx, stream, shapes: Sequence[Tuple[int, int, int]]):
    """The next len(shapes) Gemm weight records of an archive stream into
    device weights, (n, k, bits) per record (GL:60-141).  On failure the
    weights made so far are released."""
    read = stream.read_exact if hasattr(stream, "read_exact") else stream.read
    weights = []
    try:
        for n, k, bits in shapes:
            rh = read(RECORD_HEADER_BYTES)
            if len(rh) != RECORD_HEADER_BYTES:
                raise InvalidDataError("archive stream ends inside a record header")
            payload = struct.unpack_from("<i", rh, 16)[0]
            if payload < 0:
                raise InvalidDataError("record payload size %d is negative" % payload)
            body = read(payload)
            w, used = ctx.weight_from_record(rh + body, n, k, bits)
            weights.append(w)
            if used != RECORD_HEADER_BYTES + payload:
                raise InvalidDataError("record consumed %d bytes, its header says %d"
                                       % (used, RECORD_HEADER_BYTES + payload))
    except BaseException:
        for w in weights:
            if hasattr(w, "release"):
                w.release()
        raise
    return weights
