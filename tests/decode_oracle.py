"""The synthetic decode step composed from CPU oracle functions (test helper).

Follows aiimage_amd.decoder's model (EmbedTokens -> per layer RMSNorm-in,
q/k/v, RoPE, K/V append, GQA attention, o_proj + residual, RMSNorm-in,
gate/up + SwiGLU, down + residual -> final RMSNorm -> LM head logits), every
operator an oracle restatement of the reference (oracle/aexq_oracle.c), and
rounds to fp16 wherever the device stores an fp16 tensor.  Dequantised weights
are built once per layer and kept.
"""
from __future__ import annotations

import numpy as np


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


class OracleDecoder:
    def __init__(self, orc, cfg):
        from aiimage_amd import decoder, synth
        self.orc, self.cfg = orc, cfg
        lw, ls, _ = decoder.host_lm_head(cfg)
        self.lm = orc.dequant_q8(lw, ls, cfg.vocab, cfg.hidden, scale_dtype=orc.SCALE_F16)
        self.g_final = decoder.host_final_gamma(cfg)
        self.layers = []
        for l in range(cfg.layers):
            ws, g_attn, g_mlp = decoder.host_weights(cfg, l)
            W = {}
            sd = orc.SCALE_F32 if cfg.scales_f32 else orc.SCALE_F16
            for name, n, k in cfg.linears():
                words, scales, _ = ws[name]
                if getattr(cfg, "layer_bits", 4) == 8:
                    W[name] = orc.dequant_q8(words, scales, n, k, scale_dtype=sd)
                else:
                    W[name] = orc.dequant_q4(words, scales, n, k, cfg.group,
                                             getattr(cfg, "nibble_code", synth.NIBBLE_OFFSET8), sd)
            self.layers.append((W, g_attn, g_mlp))
        self.caches = []
        for l in range(cfg.layers):
            kc, vc = decoder.host_kv_cache(cfg, l)
            self.caches.append((kc.astype(np.float32), vc.astype(np.float32)))

    @classmethod
    def from_weights(cls, orc, cfg, model):
        """The same composition over given dequantised weights (the oracle's
        reading of an archive): model = {"layers": [(W, g_attn, g_mlp)],
        "lm": [vocab][hidden], "g_final": [hidden]}; the caches are the seeded
        synthetic ones DecodeSession fills."""
        from aiimage_amd import decoder
        self = cls.__new__(cls)
        self.orc, self.cfg = orc, cfg
        self.lm = np.asarray(model["lm"], np.float32)
        self.g_final = np.asarray(model["g_final"], np.float32)
        self.layers = list(model["layers"])
        self.caches = []
        for l in range(cfg.layers):
            kc, vc = decoder.host_kv_cache(cfg, l)
            self.caches.append((kc.astype(np.float32), vc.astype(np.float32)))
        return self

    def step(self, tok: int, pos: int):
        """(final hidden state, logits) of one step; appends this position's
        K/V rows to the oracle's caches."""
        orc, cfg = self.orc, self.cfg
        x = f16(self.lm[tok])
        cos_t, sin_t = orc.rope_table(pos, cfg.head_dim, cfg.rope_base)
        scale = np.float32(1.0 / np.sqrt(cfg.head_dim))
        for (W, g_attn, g_mlp), (kc, vc) in zip(self.layers, self.caches):
            xn = f16(orc.rmsnorm(x[None, :], cfg.eps, g_attn))
            q = f16(orc.gemm_gpu_semantics(xn, W["q_proj"]))[0]
            k = f16(orc.gemm_gpu_semantics(xn, W["k_proj"]))[0]
            v = f16(orc.gemm_gpu_semantics(xn, W["v_proj"]))[0]
            q = f16(orc.rope_rotate_half(q.reshape(cfg.heads_q, cfg.head_dim), cos_t, sin_t))
            k = f16(orc.rope_rotate_half(k.reshape(cfg.heads_kv, cfg.head_dim), cos_t, sin_t))
            kc[:, pos] = k
            vc[:, pos] = v.reshape(cfg.heads_kv, cfg.head_dim)
            att = f16(orc.sdpa_decode(q, kc[:, :pos + 1], vc[:, :pos + 1], scale)).reshape(1, -1)
            xb = f16(orc.gemm_gpu_semantics(att, W["o_proj"])[0] + x)
            xn2 = f16(orc.rmsnorm(xb[None, :], cfg.eps, g_mlp))
            g = orc.gemm_gpu_semantics(xn2, W["gate_proj"])[0]
            u = orc.gemm_gpu_semantics(xn2, W["up_proj"])[0]
            h = f16(orc.swiglu(g.astype(np.float32), u.astype(np.float32)))[None, :]
            x = f16(orc.gemm_gpu_semantics(h, W["down_proj"])[0] + xb)
        xf = f16(orc.rmsnorm(x[None, :], cfg.eps, self.g_final))
        logits = orc.gemm_gpu_semantics(xf, self.lm)[0]
        return x, logits


def top2_gap(logits) -> float:
    s = np.sort(np.asarray(logits, np.float64))
    return float(s[-1] - s[-2])
