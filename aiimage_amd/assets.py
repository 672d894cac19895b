"""Sharded model assets and the archive-to-device loader (host side).

Mirrors the reference's `Qwen35MobileAssetSet` / `Qwen35ShardReadStream`
(Samples/AIImageApplicationExample/Runtime/Scripts/Qwen35MobileAssetSet.cs,
cited as MAS:line): a JSON manifest (`qwen35.mobile-q8-assets/v1` or
`qwen35.mobile-q4-assets/v1`) maps each logical file -- an AQSGET8 archive, for
instance -- to an ordered list of shard files with their byte counts and
SHA-256 digests, and a logical file is read as one seekable stream across its
shards.  `load_archive_weights` then walks an AQSGET8 archive from such a
stream record by record into device weights (`aexq_weight_from_record`), the
way the Gemm layers read their weights in model order.

Not mirrored: the on-disk cache of verified hashes (MAS:195-296), which only
saves re-hashing between runs.
"""
from __future__ import annotations

import hashlib
import io
import json
import os
import struct
from typing import List, Optional, Sequence, Tuple

from . import _abi

MANIFEST_FILE = "qwen3.5_mobile_q8_assets.json"       # MAS:15
MANIFEST_SCHEMA = "qwen35.mobile-q8-assets/v1"        # MAS:16
Q4_MANIFEST_FILE = "qwen3.5_mobile_q4_assets.json"    # MAS:19
Q4_MANIFEST_SCHEMA = "qwen35.mobile-q4-assets/v1"     # MAS:20

ARCHIVE_HEADER_BYTES = 32   # AQSGET8 archive header (Q8A:26-33)
RECORD_HEADER_BYTES = 24    # record header; payload byte count at offset 16 (Q8A:60-65)


class InvalidDataError(_abi.InvalidDataError):
    """InvalidDataException of the reference manifest reader."""

    def __init__(self, message: str):
        super().__init__(_abi.ERR_FORMAT, message)


def _contained_path(root: str, relative: str) -> str:
    """ResolveContainedPath (MAS:173-181): relative, and inside the model directory."""
    if os.path.isabs(relative):
        raise InvalidDataError("Qwen3.5 shard paths must be relative: " + relative)
    full = os.path.abspath(os.path.join(root, relative))
    prefix = root.rstrip(os.sep) + os.sep
    if not full.lower().startswith(prefix.lower()):
        raise InvalidDataError("Qwen3.5 shard path escapes the model directory: " + relative)
    return full


def _sha256(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            block = f.read(4 << 20)
            if not block:
                break
            h.update(block)
    return h.hexdigest()


class Part:
    __slots__ = ("path", "bytes", "sha256")

    def __init__(self, path: str, nbytes: int, sha256: str):
        self.path, self.bytes, self.sha256 = path, nbytes, sha256


class MobileAssetSet:
    """Qwen35MobileAssetSet (MAS:13-158)."""

    def __init__(self, model_directory: str, manifest_path: str):
        self.model_directory = model_directory
        self.manifest_path = manifest_path
        self.stored_weight_bytes = 0
        self.weight_only = False
        self.quantization_bits = 8
        self._entries = {}

    @staticmethod
    def try_load(model_directory: str, verify_hashes: bool = False) -> Optional["MobileAssetSet"]:
        """TryLoad (MAS:50-138): the Q4 manifest if present, else the Q8 one, else None."""
        root = os.path.abspath(model_directory or "")
        q4 = os.path.join(root, Q4_MANIFEST_FILE)
        q8 = os.path.join(root, MANIFEST_FILE)
        path = q4 if os.path.exists(q4) else q8
        if not os.path.exists(path):
            return None
        with open(path, "r", encoding="utf-8") as f:
            doc = json.load(f)
        schema = doc.get("schema")
        if schema not in (MANIFEST_SCHEMA, Q4_MANIFEST_SCHEMA):
            raise InvalidDataError("Unsupported Qwen3.5 mobile asset manifest: " + path)
        res = MobileAssetSet(root, path)
        res.weight_only = bool(doc.get("weight_only", False))
        bits = doc.get("quantization_bits")
        res.quantization_bits = int(bits) if bits is not None else (4 if schema == Q4_MANIFEST_SCHEMA else 8)
        if res.quantization_bits not in (4, 8):
            raise InvalidDataError("Unsupported Qwen3.5 mobile quantization bit width: %d"
                                   % res.quantization_bits)
        files = doc.get("logical_files")
        if not isinstance(files, dict):
            raise InvalidDataError("Qwen3.5 mobile asset manifest has no logical_files object: " + path)
        for name, item in files.items():
            if not isinstance(item, dict):
                raise InvalidDataError("Invalid logical asset entry: " + name)
            parts = item.get("parts")
            if not isinstance(parts, list):
                raise InvalidDataError("Logical asset has no parts: " + name)
            if not parts:
                raise InvalidDataError("Logical asset has an empty part list: " + name)
            entry: List[Part] = []
            stored = 0
            for part in parts:
                if not isinstance(part, dict):
                    raise InvalidDataError("Invalid shard entry: " + name)
                rel = part.get("file")
                if not isinstance(rel, str) or not rel.strip():
                    raise InvalidDataError("Shard file name is empty: " + name)
                full = _contained_path(root, rel)
                if not os.path.exists(full):
                    raise FileNotFoundError("Qwen3.5 mobile shard is missing.", full)
                actual = os.path.getsize(full)
                expected = part.get("bytes", -1)
                if actual != expected:
                    raise InvalidDataError("Qwen3.5 mobile shard size mismatch: %s expected=%s actual=%d"
                                           % (rel, expected, actual))
                digest = str(part.get("sha256") or "").lower()
                if len(digest) != 64:
                    raise InvalidDataError("Qwen3.5 shard SHA-256 is missing: " + rel)
                if verify_hashes and _sha256(full) != digest:
                    raise InvalidDataError("Qwen3.5 mobile shard SHA-256 mismatch: " + rel)
                entry.append(Part(full, actual, digest))
                stored += actual
            if item.get("stored_bytes", -1) != stored:
                raise InvalidDataError("Qwen3.5 logical stored byte count mismatch: " + name)
            res._entries[name] = entry
            res.stored_weight_bytes += stored
        return res

    def contains(self, logical_name: str) -> bool:
        return bool(logical_name) and logical_name in self._entries

    def open_read(self, logical_name: str) -> "ShardReadStream":
        if logical_name not in self._entries:
            raise FileNotFoundError("Qwen3.5 logical mobile asset is missing from the manifest.",
                                    logical_name)
        return ShardReadStream(self._entries[logical_name])

    def stored_bytes(self, logical_name: str) -> int:
        return sum(p.bytes for p in self._entries.get(logical_name, []))


class ShardReadStream(io.RawIOBase):
    """Qwen35ShardReadStream (MAS:461-558): one read-only, seekable stream over
    the concatenated shards of a logical file."""

    def __init__(self, parts: Sequence[Part]):
        super().__init__()
        if not parts:
            raise ValueError("At least one shard is required.")
        self._parts = list(parts)
        self._offsets = [0]
        for p in self._parts:
            self._offsets.append(self._offsets[-1] + p.bytes)
        self._length = self._offsets[-1]
        self._pos = 0
        self._file = None
        self._index = -1

    def readable(self) -> bool:
        return True

    def seekable(self) -> bool:
        return True

    def __len__(self) -> int:
        return self._length

    def tell(self) -> int:
        return self._pos

    def seek(self, offset: int, whence: int = io.SEEK_SET) -> int:
        target = {io.SEEK_SET: offset, io.SEEK_CUR: self._pos + offset,
                  io.SEEK_END: self._length + offset}[whence]
        if target < 0 or target > self._length:
            raise OSError("Seek target is outside the Qwen3.5 logical asset.")
        self._pos = target
        return target

    def _part_at(self, pos: int) -> int:
        lo, hi = 0, len(self._parts) - 1
        while lo <= hi:
            mid = (lo + hi) >> 1
            if pos < self._offsets[mid]:
                hi = mid - 1
            elif pos >= self._offsets[mid + 1]:
                lo = mid + 1
            else:
                return mid
        raise OSError("Could not map Qwen3.5 logical stream position to a shard.")

    def readinto(self, buf) -> int:
        view = memoryview(buf).cast("B")
        total = 0
        while total < len(view) and self._pos < self._length:
            i = self._part_at(self._pos)
            if i != self._index:
                if self._file:
                    self._file.close()
                self._file = open(self._parts[i].path, "rb")
                self._index = i
            local = self._pos - self._offsets[i]
            self._file.seek(local)
            want = min(len(view) - total, self._parts[i].bytes - local)
            got = self._file.readinto(view[total:total + want])
            if not got:
                raise EOFError("Unexpected end of Qwen3.5 mobile shard: " + self._parts[i].path)
            total += got
            self._pos += got
        return total

    def read_exact(self, n: int) -> bytes:
        data = self.read(n)
        if data is None or len(data) != n:
            raise InvalidDataError("AQSGET8 stream ends inside a record")
        return data

    def close(self) -> None:
        if self._file:
            self._file.close()
            self._file = None
        super().close()


def load_archive_weights(ctx, stream, shapes: Sequence[Tuple[int, int, int]]):
    """Walk an AQSGET8 archive (header, then one record per Gemm weight in model
    order) from `stream` into device weights: `shapes` gives (n, k, bits) of
    each record's layer (Q8A:277-293 header, GL:60-141 per record).  Returns
    (weights, (quant_bits, default_block, record_count))."""
    from .aexq import archive_header
    read = stream.read_exact if hasattr(stream, "read_exact") else stream.read
    header = archive_header(read(ARCHIVE_HEADER_BYTES))
    if len(shapes) > header[2]:
        raise InvalidDataError("archive holds %d records, %d layers asked for"
                               % (header[2], len(shapes)))
    weights = []
    for n, k, bits in shapes:
        rh = read(RECORD_HEADER_BYTES)
        if len(rh) != RECORD_HEADER_BYTES:
            raise InvalidDataError("AQSGET8 stream ends inside a record header")
        payload = struct.unpack_from("<i", rh, 16)[0]
        if payload < 0:
            raise InvalidDataError("AQSGET8 record payload size is negative")
        body = read(payload)
        w, used = ctx.weight_from_record(rh + body, n, k, bits)
        if used != RECORD_HEADER_BYTES + payload:
            w.release()
            raise InvalidDataError("AQSGET8 record size disagrees with its header")
        weights.append(w)
    return weights, header
