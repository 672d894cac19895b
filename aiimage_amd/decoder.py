"""Synthetic Qwen3.5-0.8B-shaped decode step over the aexq C ABI (benchmark config 3).

Mirrors the per-token work of Qwen35DecoderSession (paths relative to the
reference root, DEC = Packages/com.aexis/Samples/AIImageApplicationExample/
Runtime/Scripts/Qwen35DecoderSession.cs): EmbedTokens (DEC:402-428) from the
tied Q8 table, the decoder layers (DecodeCore, DEC:463-585), and the final
norm fused into SelectNextToken's LM head + greedy argmax (DEC:734-809).  Each
layer:

    x  -> RMSNorm-in + q/k/v (one grouped launch)
       -> RoPE on q, k; k/v appended to the fp16 cache; GQA decode attention
          over the cache (one fused pass + the split combine)
       -> o_proj + residual
       -> RMSNorm-in + gate/up + SwiGLU-out
       -> down + residual

The model is random-init with the benchmark's shapes: hidden 1024, 16 query
heads of 128, 4 key/value heads (k/v_proj 1024 -> 512), SwiGLU 3584, 24
layers, Q4 offset-8 linears with fp16 scales per 32, RMSNorm eps 1e-6 with
weights 1 + N(0, 0.02), RoPE base 1e6, a Q8 per-row LM head 1024 -> 151936
with fp16 scales (also the embedding), and an fp16 KV cache filled with N(0, 1).

The decode position lives in device memory: the attention launches read it
and take their RoPE row from [capacity][head_dim/2] tables built once, and a
step that advances ends by writing the argmax into the input token and moving
the position on (Generate, DEC:1160-1237), so one captured step replays token
after token.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _abi, aexq, synth


@dataclass
class ModelConfig:
    layers: int = 24
    hidden: int = 1024
    heads_q: int = 16
    heads_kv: int = 4
    head_dim: int = 128
    intermediate: int = 3584
    vocab: int = synth.VOCAB
    rope_base: float = 1e6
    eps: float = 1e-6
    capacity: int = 2048     # KV cache positions
    group: int = 32          # Q4 scale group
    seed: int = synth.SEED_BASE + 3
    scales_f32: bool = False  # layer scales fp32 (the reference archives' dtype) instead of fp16
    layer_bits: int = 4       # 8: Q8 layer weights with one scale per row (Q8A:94-114)
    nibble_code: int = synth.NIBBLE_OFFSET8  # Q4 code; the reference's archives: NIBBLE_TWOS

    @classmethod
    def reference_q4(cls, **kw) -> "ModelConfig":
        """The reference's shipping Q4 layers: two's-complement nibbles, one fp32
        scale per 16 codes (Qwen35MobileQ4AssetBuilder.cs:22-25, Q8A:116-139)."""
        return cls(group=16, scales_f32=True, nibble_code=synth.NIBBLE_TWOS, **kw)

    @classmethod
    def reference_q8(cls, **kw) -> "ModelConfig":
        """Q8 layers with one fp32 scale per output row (Q8A:94-114, GL:65-67)."""
        return cls(layer_bits=8, scales_f32=True, **kw)

    @property
    def format_name(self) -> str:
        if self.layer_bits == 8:
            return "q8_row_" + ("f32" if self.scales_f32 else "f16")
        return f"q4_g{self.group}_" + ("f32" if self.scales_f32 else "f16")

    def weight_block(self, k: int) -> int:
        """Scale block of a layer weight with reduction length k."""
        return k if self.layer_bits == 8 else self.group

    @property
    def q_width(self):
        return self.heads_q * self.head_dim

    @property
    def kv_width(self):
        return self.heads_kv * self.head_dim

    def linears(self):
        h, i = self.hidden, self.intermediate
        return (("q_proj", self.q_width, h), ("k_proj", self.kv_width, h),
                ("v_proj", self.kv_width, h), ("o_proj", h, self.q_width),
                ("gate_proj", i, h), ("up_proj", i, h), ("down_proj", h, i))

    def bytes_per_token(self, length: int) -> dict:
        """Algorithmic HBM bytes of one decode step attending over `length`
        positions: every weight code and scale once, each cached K and V row
        once, and the activations each launch reads and writes."""
        sb = 4 if self.scales_f32 else 2
        if self.layer_bits == 8:
            weights = sum(n * k + n * sb for _, n, k in self.linears())
        else:
            weights = sum(n * k // 2 + n * (k // self.group) * sb for _, n, k in self.linears())
        kv_read = 2 * self.heads_kv * length * self.head_dim * 2
        h, qw, kw, i = self.hidden, self.q_width, self.kv_width, self.intermediate
        act = 2 * (h + qw + 2 * kw          # q/k/v: x in, q/k/v out
                   + qw + 2 * kw + qw + 2 * kw  # RoPE: q in/out, k/v in, k/v appended
                   + qw + qw                # attention: q in, out
                   + qw + 2 * h             # o_proj: attention in, residual in, x out
                   + h + i                  # gate/up: x in, h out
                   + i + 2 * h)             # down: h in, residual in, x out
        lm = self.vocab * self.hidden + self.vocab * 2
        total = self.layers * (weights + kv_read + act) + lm + 2 * h * 3 + 4
        return {"linear_weights": self.layers * weights, "kv_read": self.layers * kv_read,
                "activations": self.layers * act + 2 * h * 3 + 4, "lm_head": lm, "total": total}


def host_weights(cfg: ModelConfig, layer: int):
    """Seeded numpy weights of one layer: {name: (words, scales, codes)} and the two norms."""
    out = {}
    sdt = np.float32 if cfg.scales_f32 else np.float16
    for i, (name, n, k) in enumerate(cfg.linears()):
        if cfg.layer_bits == 8:
            out[name] = synth.q8_weights(n, k, cfg.seed + 97 * layer + i, scale_dtype=sdt)
        else:
            out[name] = synth.q4_weights(n, k, cfg.seed + 97 * layer + i, group=cfg.group,
                                         code=cfg.nibble_code, scale_dtype=sdt)
    g_attn = synth.rms_gamma(cfg.hidden, cfg.seed + 97 * layer + 50)
    g_mlp = synth.rms_gamma(cfg.hidden, cfg.seed + 97 * layer + 51)
    return out, g_attn, g_mlp


def rope_tables(capacity: int, head_dim: int, base: float):
    """(cos, sin) float32 [capacity][head_dim/2]: row p is CreateRopeTextures'
    row for position p (DEC:1660-1675), evaluated in the reference's float32
    steps: e = j * (2f / (half * 2f)), p = (float)pow(theta, e), inverse = 1f /
    p, angle = position * inverse, then (float)cos / sin of the float angle
    (UnityEngine's Mathf.Pow/Cos/Sin round System.Math's double results)."""
    half = head_dim // 2
    theta = np.float32(base)
    step = np.float32(2.0) / (np.float32(half) * np.float32(2.0))
    e = (np.arange(half, dtype=np.float32) * step).astype(np.float32)
    pw = np.power(np.float64(theta), e.astype(np.float64)).astype(np.float32)
    inverse = (np.float32(1.0) / pw).astype(np.float32)
    pos = np.arange(capacity, dtype=np.float32)[:, None]
    angle = (pos * inverse[None, :]).astype(np.float32)
    a64 = angle.astype(np.float64)
    return np.cos(a64).astype(np.float32), np.sin(a64).astype(np.float32)


def host_lm_head(cfg: ModelConfig):
    return synth.q8_weights(cfg.vocab, cfg.hidden, cfg.seed + 7)


def host_final_gamma(cfg: ModelConfig):
    return synth.rms_gamma(cfg.hidden, cfg.seed + 8)


def host_kv_cache(cfg: ModelConfig, layer: int):
    """fp16 N(0, 1) K and V caches [heads_kv][capacity][head_dim] of one layer."""
    g = synth.rng(cfg.seed + 1000 + layer)
    shape = (cfg.heads_kv, cfg.capacity, cfg.head_dim)
    return (g.standard_normal(shape).astype(np.float16), g.standard_normal(shape).astype(np.float16))


# ----------------------------------------------------------------- model assets

# Logical files of a mobile asset set (Qwen35MobileQ4AssetBuilder.cs:29, 189):
# the decoder layers' archive and the tied token embedding, which stays Q8 with
# one scale per row whatever the layers' format (B4:21-25).
DECODER_FILE = "qwen3.5_decoder.ncnn.bin"
EMBED_FILE = "qwen3.5_embed_token.ncnn.bin"


@dataclass
class ModelWeights:
    """Device weights of the model: per layer the seven linears and the two
    RMSNorm gammas (host float32), the tied Q8 embedding / LM head and the
    final norm's gamma."""
    layers: list          # [{"w": {name: QuantWeight}, "g_attn": np, "g_mlp": np}]
    lm: object            # QuantWeight, Q8 per row [vocab][hidden]
    g_final: np.ndarray


def archive_records(cfg: ModelConfig) -> list:
    """The decoder archive's record order for this model: per layer the
    attention RMSNorm weights (a raw fp32 record), q/k/v/o, the MLP RMSNorm
    weights, gate/up/down, then the final norm -- the order in which the
    graph's layers read their weights (GL:15-162 per Gemm, RMS:24-46 per
    RMSNorm).  Entries: ("norm", count) or (name, n, k)."""
    out = []
    lin = cfg.linears()
    for _ in range(cfg.layers):
        out.append(("norm", cfg.hidden))
        out.extend(lin[:4])
        out.append(("norm", cfg.hidden))
        out.extend(lin[4:])
    out.append(("norm", cfg.hidden))
    return out


def load_assets(ctx: aexq.Context, model_directory: str, cfg: ModelConfig,
                verify_hashes: bool = True) -> ModelWeights:
    """A mobile asset set (MAS:50-138: the Q4 manifest preferred over the Q8
    one) into device weights: the decoder archive walked record by record
    (Gemm weights through aexq_weight_from_record, GL:60-141; RMSNorm weights
    as raw fp32 records, Q8A:295-306) and the tied Q8 embedding, whose device
    copy is also the LM head (EMB:95-120).  The layers' Gemm records are read
    as cfg.layer_bits weights: Q4 records for a Q4 model, Q8 records with a
    block of K for a Q8 one; any other record is quantized per row."""
    from . import assets
    aset = assets.MobileAssetSet.try_load(model_directory, verify_hashes=verify_hashes)
    if aset is None:
        raise assets.InvalidDataError("no mobile asset manifest in " + model_directory)
    for name in (DECODER_FILE, EMBED_FILE):
        if not aset.contains(name):
            raise assets.InvalidDataError(f"the asset set has no logical file {name}")
    made = []
    try:
        with aset.open_read(EMBED_FILE) as s:
            (lm,), _ = assets.load_archive_weights(ctx, s, [(cfg.vocab, cfg.hidden, 8)])
        made.append(lm)
        info = lm.info()
        if info.block != cfg.hidden:
            raise assets.InvalidDataError(
                f"{EMBED_FILE}: the tied embedding has scale blocks of {info.block}, not one "
                f"per row of {cfg.hidden}")
        plan = archive_records(cfg)
        layers, cur, norms = [], None, []
        with aset.open_read(DECODER_FILE) as s:
            header = assets.read_archive_header(s)
            if header[2] != len(plan):
                raise assets.InvalidDataError(
                    f"{DECODER_FILE} holds {header[2]} records, the model reads {len(plan)}")
            for item in plan:
                if item[0] == "norm":
                    norms.append(assets.read_float_record(s, item[1]))
                    continue
                name, n, k = item
                if name == "q_proj":
                    cur = {}
                    layers.append(cur)
                (w,) = assets.read_weight_records(ctx, s, [(n, k, cfg.layer_bits)])
                made.append(w)
                cur[name] = w
        out = [{"w": w, "g_attn": norms[2 * l], "g_mlp": norms[2 * l + 1]}
               for l, w in enumerate(layers)]
        return ModelWeights(out, lm, norms[-1])
    except BaseException:
        for w in made:
            w.release()
        raise


class DecodeSession:
    """Device state of the model and one decode step (eager or graph)."""

    def __init__(self, ctx: aexq.Context, cfg: ModelConfig, device: str = "cuda",
                 fused: bool = False, workgroups: int = 0, weights: ModelWeights = None):
        """fused: the layers run as one launch (aexq_decoder_run) instead of
        five launches per layer.  weights: the model's device weights (from
        load_assets); None builds the seeded synthetic model of cfg."""
        self.ctx, self.cfg, self.device = ctx, cfg, device
        P4 = aexq.LAYOUT_PACK4_LINEAR
        c = cfg
        self.layers = []
        for l in range(c.layers):
            if weights is not None:
                dev_w = weights.layers[l]["w"]
                g_attn, g_mlp = weights.layers[l]["g_attn"], weights.layers[l]["g_mlp"]
            else:
                ws, g_attn, g_mlp = host_weights(c, l)
                dev_w = {}
                for name, n, k in c.linears():
                    words, scales, _ = ws[name]
                    dev_w[name] = ctx.weight(
                        aexq.QuantizedTensor(n * k, c.weight_block(k), words, scales,
                                             bits=c.layer_bits, nibble_code=c.nibble_code), n, k)
            kc, vc = host_kv_cache(c, l)
            self.layers.append({
                "w": dev_w,
                "g_attn": torch.as_tensor(g_attn).to(device),
                "g_mlp": torch.as_tensor(g_mlp).to(device),
                "k_cache": torch.as_tensor(kc).to(device).reshape(-1),
                "v_cache": torch.as_tensor(vc).to(device).reshape(-1),
            })
        if weights is not None:
            self.lm = weights.lm
            g_final = weights.g_final
        else:
            words, scales, _ = host_lm_head(c)
            self.lm = ctx.weight(aexq.QuantizedTensor(c.vocab * c.hidden, c.hidden, words, scales,
                                                      bits=8), c.vocab, c.hidden)
            g_final = host_final_gamma(c)
        # the embedding reads the LM head's device copy through a non-owning
        # alias (Qwen35SharedTokenEmbeddingWeights, EMB:95-120; GL:91-111)
        self.embed = self.lm.alias()
        self.g_final = torch.as_tensor(g_final).to(device)
        f16 = torch.float16
        z = lambda n, dt=f16: torch.zeros(n, dtype=dt, device=device)
        self.token = torch.zeros(1, dtype=torch.int32, device=device)
        self.next_token = torch.zeros(1, dtype=torch.int32, device=device)
        # the decode position (device), and the token generated at each position
        self.pos = torch.zeros(1, dtype=torch.int32, device=device)
        self.history = torch.full((c.capacity,), -1, dtype=torch.int32, device=device)
        self.xa, self.xb = z(c.hidden), z(c.hidden)
        self.q, self.k, self.v = z(c.q_width), z(c.kv_width), z(c.kv_width)
        self.attn = z(c.q_width)
        self.h = z(c.intermediate)
        ct, st = rope_tables(c.capacity, c.head_dim, c.rope_base)
        self.cos = torch.as_tensor(ct).to(device).reshape(-1)
        self.sin = torch.as_tensor(st).to(device).reshape(-1)
        d = aexq.describe
        self.d = {
            "xa": d(self.xa, 1, c.hidden, P4), "xb": d(self.xb, 1, c.hidden, P4),
            "q": d(self.q, 1, c.q_width, P4), "k": d(self.k, 1, c.kv_width, P4),
            "v": d(self.v, 1, c.kv_width, P4), "attn": d(self.attn, 1, c.q_width, P4),
            "h": d(self.h, 1, c.intermediate, P4),
        }
        self.position = None
        self.scale = 1.0 / math.sqrt(c.head_dim)
        self.fused = None
        if fused:
            layers = [dict(L["w"], attn_norm=L["g_attn"], mlp_norm=L["g_mlp"],
                           k_cache=L["k_cache"], v_cache=L["v_cache"]) for L in self.layers]
            self.fused = ctx.decoder(layers, self.embed, c.heads_q, c.heads_kv, c.head_dim,
                                     c.capacity, c.eps, self.scale, self.cos, self.sin,
                                     workgroups)

    def set_position(self, position: int):
        """Sets the device decode position (the new token's cache row)."""
        if not 0 <= position < self.cfg.capacity:
            raise ValueError(f"position {position} outside the cache capacity {self.cfg.capacity}")
        self.pos.fill_(position)
        self.position = position

    def check_fused(self):
        """Raises when a fused run since the last check gave up a bounded wait
        (its outputs are then invalid).  Synchronizes the stream."""
        if self.fused is not None and self.fused.error():
            raise _abi.DeviceError(
                _abi.ERR_DEVICE,
                "aexq_decoder_run gave up a bounded wait: the step's outputs are invalid")

    def step(self, advance: bool = False, check: bool = True):
        """One decode step for self.token at the device position ->
        self.next_token.  With `advance` the step also stores the argmax as the
        next input token (and in self.history) and moves the position on.  On
        the fused path `check` synchronizes and raises if the run gave up a
        bounded wait; hot loops and graph capture pass False and call
        check_fused() once afterwards."""
        c, ctx, d = self.cfg, self.ctx, self.d
        if self.fused is not None:
            self.fused.run(self.token, self.pos, self.xa)
            ctx.lmhead_argmax(self.lm, d["xa"], None, self.next_token, rmsnorm=True,
                              rms_gamma=self.g_final, rms_eps=c.eps)
            if advance:
                ctx.decode_advance(self.pos, self.token, self.next_token, self.history)
            if check:
                self.check_fused()
            return
        ctx.embed_q8(self.embed, self.token, self.xa)
        for L in self.layers:
            w = L["w"]
            ctx.linear_group([w["q_proj"], w["k_proj"], w["v_proj"]], d["xa"],
                             [d["q"], d["k"], d["v"]], rmsnorm=True, rms_gamma=L["g_attn"],
                             rms_eps=c.eps)
            ctx.attention_decode_rope_at(self.q, self.k, self.v, L["k_cache"], L["v_cache"],
                                         c.heads_q, c.heads_kv, c.head_dim, c.capacity, self.pos,
                                         self.cos, self.sin, self.scale, self.attn)
            ctx.linear(w["o_proj"], d["attn"], d["xb"], residual=d["xa"])
            ctx.linear(w["gate_proj"], d["xb"], d["h"], rmsnorm=True, rms_gamma=L["g_mlp"],
                       rms_eps=c.eps, up=w["up_proj"])
            ctx.linear(w["down_proj"], d["h"], d["xa"], residual=d["xb"])
        ctx.lmhead_argmax(self.lm, d["xa"], None, self.next_token, rmsnorm=True,
                          rms_gamma=self.g_final, rms_eps=c.eps)
        if advance:
            ctx.decode_advance(self.pos, self.token, self.next_token, self.history)

    def capture(self, warmup: int = 2, advance: bool = False, steps: int = 1) -> torch.cuda.CUDAGraph:
        """Captures `steps` consecutive step(advance) calls into one HIP graph on
        a side stream (with `advance` each step feeds its argmax to the next on
        the device, so a replay decodes `steps` tokens; a graph launch costs the
        device about 8 us of idle time between replays, which this spreads over
        the steps).  The warm-up steps (which do not advance) size the context's
        scratch first, so nothing allocates while capturing."""
        if steps < 1:
            raise ValueError(f"steps={steps}")
        stream = torch.cuda.Stream()
        old = self.ctx.stream
        self.ctx.set_stream(stream)
        try:
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                for _ in range(warmup):
                    self.step(check=False)
            stream.synchronize()
            self.check_fused()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
                for _ in range(steps):
                    self.step(advance=advance, check=False)
        finally:
            self.ctx.set_stream(old)
        torch.cuda.synchronize()
        # what generate() needs to know about a replay
        g.aexq_steps = steps
        g.aexq_advance = advance
        return g

    def generate(self, start_token: int, position: int, count: int,
                 graph: torch.cuda.CUDAGraph = None, graph_steps: int = None) -> list:
        """Greedy decoding of `count` tokens from `start_token` at `position`
        (Qwen35DecoderSession.Generate, DEC:1160-1237): each step's argmax is the
        next step's input.  With `graph` (from capture(advance=True, steps=K))
        each replay decodes K tokens and the remainder of count runs as eager
        steps; otherwise every token is an eager step.  graph_steps defaults to
        the graph's K and must equal it; a graph captured without advance (its
        replays do not move the position) is refused.  Returns the generated
        token ids."""
        if graph is not None:
            captured = getattr(graph, "aexq_steps", None)
            if getattr(graph, "aexq_advance", True) is False:
                raise ValueError("the graph was captured without advance=True: its replays "
                                 "do not move the position")
            if graph_steps is None:
                graph_steps = captured if captured is not None else 1
            elif captured is not None and graph_steps != captured:
                raise ValueError(f"graph_steps={graph_steps} for a graph of {captured} steps")
        elif graph_steps is None:
            graph_steps = 1
        if graph_steps < 1:
            raise ValueError(f"graph_steps={graph_steps}")
        if count < 0 or position + count > self.cfg.capacity:
            raise ValueError(f"{count} tokens from position {position} exceed the cache "
                             f"capacity {self.cfg.capacity}")
        self.token.fill_(start_token)
        self.set_position(position)
        replays = count // graph_steps if graph is not None else 0
        for _ in range(replays):
            graph.replay()
        for _ in range(count - replays * graph_steps):
            self.step(advance=True, check=False)
        torch.cuda.synchronize()
        self.check_fused()
        self.position = position + count
        return [int(t) for t in self.history[position:position + count].cpu().tolist()]
