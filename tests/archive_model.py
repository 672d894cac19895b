"""Writes a model directory in the reference's mobile-asset form with the
oracle's record writers (test helper; the oracle is the checker, never the
product path).

The layout follows Qwen35MobileQ4AssetBuilder (Packages/com.aexis/Samples/
AIImageApplicationExample/Editor/Qwen35MobileQ4AssetBuilder.cs, B4 below):

  * qwen3.5_embed_token.ncnn.bin -- the tied token embedding / LM head, one Q8
    record with a scale per row of `hidden` (B4:185-198, "row-int8");
  * qwen3.5_decoder.ncnn.bin -- an AQSGET8 archive whose Gemm records are Q4
    groups of 16 written from Q8 rows (WriteQ4FromQ8Rows, Q8A:167-207; the
    builder's default block 16, B4:25) or, for a Q8 asset set, Q8 records with
    one scale per row (WriteQ8FromFloat32Rows, Q8A:141-165), and whose RMSNorm
    weights are raw fp32 records (WriteFloat32Array, Q8A:216-223), in the
    order aiimage_amd.decoder.archive_records gives;
  * each logical file cut into shard files listed with size and SHA-256 under
    the qwen35.mobile-q4-assets/v1 (or -q8-) manifest (B4:236-283, MAS:50-138).

Returns the oracle's view of the same model: dequantised float32 weights
(through the oracle's record readers) for OracleDecoder.from_weights.
"""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np


def _rows_q8(orc, values, n, k):
    """Float rows [n][k] -> (Q8 words, fp32 row scales) as the Q8 source archive holds them."""
    words, scales = orc.q8_pack_rows(values, n, k)
    return words, scales


def write_model(orc, cfg, root: str, seed: int, shard_bytes: int = 3 << 20):
    """Writes the asset set of `cfg` (cfg.layer_bits 4 or 8) under root and
    returns {"layers": [(W, g_attn, g_mlp)], "lm": float32 [vocab][hidden],
    "g_final": float32}."""
    from aiimage_amd import assets, decoder
    rng = np.random.default_rng(seed)
    os.makedirs(os.path.join(root, "weights"), exist_ok=True)

    # tied embedding / LM head: one Q8 record, one scale per row
    emb = (rng.standard_normal((cfg.vocab, cfg.hidden)) * 0.05).astype(np.float32)
    emb_rec = orc.record_write_q8(emb.reshape(-1), cfg.hidden)
    rc, ew, es, blk, _ = orc.record_read_q8_packed(emb_rec, cfg.vocab * cfg.hidden, cfg.hidden)
    assert rc == 0 and blk == cfg.hidden
    lm = orc.dequant_q8(ew, es, cfg.vocab, cfg.hidden, scale_dtype=orc.SCALE_F32)
    emb_blob = orc.archive_header(8, cfg.hidden, 1, emb.nbytes) + emb_rec

    recs, norms, weights = [], [], []
    for item in decoder.archive_records(cfg):
        if item[0] == "norm":
            g = (1.0 + 0.02 * rng.standard_normal(item[1])).astype(np.float32)
            recs.append(orc.record_write_raw_f32(g))
            norms.append(g)
            continue
        name, n, k = item
        v = (rng.standard_normal((n, k)) * 0.03).astype(np.float32)
        words, scales = _rows_q8(orc, v, n, k)
        if cfg.layer_bits == 8:
            rec = orc.record_write_q8(v.reshape(-1), k)
            rc, w8, s8, blk, _ = orc.record_read_q8_packed(rec, n * k, k)
            assert rc == 0 and blk == k
            W = orc.dequant_q8(w8, s8, n, k, scale_dtype=orc.SCALE_F32)
        else:
            rec = orc.record_write_q4_from_q8_rows(words, scales, n, k, cfg.group)
            rc, w4, s4, blk, _ = orc.record_read_q4_packed(rec, n * k, cfg.group)
            assert rc == 0 and blk == cfg.group
            W = orc.dequant_q4(w4, s4, n, k, cfg.group, orc.NIBBLE_TWOS, orc.SCALE_F32)
        recs.append(rec)
        weights.append((name, W))
    dec_blob = orc.archive_header(cfg.layer_bits, cfg.group if cfg.layer_bits == 4 else cfg.hidden,
                                  len(recs), 0) + b"".join(recs)

    logical = {}
    for name, blob in ((decoder.EMBED_FILE, emb_blob), (decoder.DECODER_FILE, dec_blob)):
        parts = []
        for j, a in enumerate(range(0, len(blob), shard_bytes)):
            chunk = blob[a:a + shard_bytes]
            rel = f"weights/{name}.part{j:03d}"
            with open(os.path.join(root, rel), "wb") as f:
                f.write(chunk)
            parts.append({"file": rel, "bytes": len(chunk),
                          "sha256": hashlib.sha256(chunk).hexdigest()})
        logical[name] = {"stored_bytes": len(blob), "parts": parts}
    q4 = cfg.layer_bits == 4
    manifest = {"schema": assets.Q4_MANIFEST_SCHEMA if q4 else assets.MANIFEST_SCHEMA,
                "model_id": "qwen3.5_synthetic", "quantization_bits": cfg.layer_bits,
                "weight_only": True, "tied_embedding_quantization_bits": 8,
                "logical_files": logical}
    with open(os.path.join(root, assets.Q4_MANIFEST_FILE if q4 else assets.MANIFEST_FILE), "w") as f:
        json.dump(manifest, f)

    layers = []
    it = iter(weights)
    for l in range(cfg.layers):
        W = dict(next(it) for _ in range(7))
        layers.append((W, norms[2 * l], norms[2 * l + 1]))
    return {"layers": layers, "lm": lm, "g_final": norms[-1]}
