#!/usr/bin/env python3
"""Benchmark of the quantized decode-linear path on one MI355X.

Workload (benchmark config 2, the metric's configuration): one decoder layer's
seven Q4 linears at M=1 (q 1024->2048, k/v 1024->512, o 2048->1024,
gate/up 1024->3584, down 3584->1024), symmetric 4-bit offset-8 codes with one
fp16 scale per 32 K, fp16 activations, fp32 accumulation, fp16 outputs.

"Cold" follows the sustained protocol of the benchmark: COPIES distinct
device copies of the layer's weights are processed in every step, enough that
each of the step's launches cycles through >= 1 GiB of distinct weights (the
smallest launch, o_proj, sets the count: about 900 copies, 8.3 GB), far above
the 256 MB Infinity Cache and the L2s, so no weight byte is re-read from a
cache.  One step = the layer's linears over all copies in four
launches: RMSNorm-in + q/k/v (one grouped launch), RMSNorm-in + gate/up with
the SwiGLU-out epilogue, o_proj (input: that copy's q output), down (input:
that copy's SwiGLU output).

value = COPIES * algorithmic bytes of one layer / wall time of one step, where
the algorithmic bytes count every code, scale, activation and output once
(9,142,272 + 46,080 = 9,188,352 B per layer).  The JSON line also carries the
roofline of the dominant launch (HIP events on the launch stream) and the
reference CPU path (RunGemmCpu restated in C) timed on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

METRIC = ("cold-HBM GB/s (% of peak) per quant matvec; decode tokens/s, 0.8B-shape, 1 GPU")
HBM_PEAK_GBS = 8000.0
ROOT = os.path.dirname(os.path.abspath(__file__))
# HBM bytes per dispatch of the dominant kernel, from two rocprofv3 --pmc runs of
# this bench (FETCH_SIZE, WRITE_SIZE) scaled by the calibration kernel's counts
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "qmv_q4_layer_config2_traffic.json")
# the sources the dominant launch's kernel is compiled from: the traffic record
# holds their hash, and a record of other sources is not this build's traffic
KERNEL_SOURCES = ("include/aexq.h", "aiimage_amd/csrc/aexq_internal.hpp",
                  "aiimage_amd/csrc/aexq_device.hpp", "aiimage_amd/csrc/aexq_qmv.hpp",
                  "aiimage_amd/csrc/aexq_qmv_q4.hip")
LAYER_WEIGHT_BYTES = 9_142_272
LAYER_ACT_BYTES = 46_080
LAYER_BYTES = LAYER_WEIGHT_BYTES + LAYER_ACT_BYTES
GIB = 1 << 30


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--copies", type=int, default=0,
                    help="layer copies per step (default: every launch streams >= 1 GiB)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the per-config extras")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the config-3 decode step timing and print its JSON (for "
                         "profiling that step); not the benchmark line")
    ap.add_argument("--decode-phases", action="store_true",
                    help="per-phase times of the fused decode step from the phase-stamped "
                         "library (aiimage_amd/libaexq_stamps.so; built if missing)")
    ap.add_argument("--lmhead-only", action="store_true",
                    help="config 5 only (the LM head with the fused argmax, M = 1 and 8) and "
                         "the logits-only matvec of the same head")
    ap.add_argument("--config4-only", action="store_true",
                    help="run only the config-4 timings (M in {16, 64, 512}, Q4 and Q8; batched "
                         "copies and single layers) and print their JSON (for profiling those "
                         "kernels); not the benchmark line")
    ap.add_argument("--calib", action="store_true",
                    help="also run one 256 MiB fp32 neg kernel (known HBM traffic) to scale "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def kernel_source_hash() -> str:
    """sha256 over KERNEL_SOURCES (path, then contents, in order): names the
    build of the streaming matvec whose traffic a record describes."""
    import hashlib
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        h.update(rel.encode() + b"\0")
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def measured_traffic(launch: str, copies: int):
    """(HBM bytes per dispatch, note) from the committed counter record, or
    (None, why not) when the record is of another launch, copy count or build."""
    if not os.path.exists(TRAFFIC_FILE):
        return None, "no counter record"
    rec = json.load(open(TRAFFIC_FILE))
    if rec.get("launch") != launch or rec.get("copies") != copies:
        return None, f"counter record is of {rec.get('launch')} x {rec.get('copies')} copies"
    if rec.get("source_sha256") != kernel_source_hash():
        return None, "counter record is of another build of the kernel sources"
    return rec.get("hbm_bytes_per_dispatch"), rec.get("source")


class Layer:
    """One stacked copy set of the seven Q4 linears plus the activation buffers."""

    def __init__(self, ctx, aexq, synth, torch, copies: int, seed: int):
        self.copies = copies
        self.aexq = aexq
        self.ctx = ctx
        dims = {name: (n, k) for name, n, k in synth.LAYER_LINEARS}
        self.dims = dims
        self.w = {}
        for i, (name, n, k) in enumerate(synth.LAYER_LINEARS):
            words, scales, _ = synth.q4_weights(n, k, seed + i, group=32, code=synth.NIBBLE_OFFSET8)
            base = ctx.weight(aexq.QuantizedTensor(n * k, 32, words, scales, bits=4,
                                                   nibble_code=synth.NIBBLE_OFFSET8), n, k)
            self.w[name] = base.replicate(copies)
            base.release()
        dev = "cuda"
        x = torch.as_tensor(synth.activations(1, 1024, seed + 100)).to(dev)
        self.x = x.reshape(-1)
        self.gamma = torch.as_tensor(synth.rms_gamma(1024, seed + 101)).to(dev)
        P4 = aexq.LAYOUT_PACK4_LINEAR
        self.out = {}
        for name in ("q_proj", "k_proj", "v_proj", "o_proj", "down_proj"):
            n = dims[name][0]
            self.out[name] = torch.zeros(copies * n, dtype=torch.float16, device=dev)
        self.h = torch.zeros(copies * 3584, dtype=torch.float16, device=dev)
        d = aexq.describe
        self.xd = d(self.x, 1, 1024)
        self.yd = {name: d(t, 1, dims[name][0], P4, batch=copies, batch_stride=dims[name][0])
                   for name, t in self.out.items()}
        self.hd = d(self.h, 1, 3584, P4, batch=copies, batch_stride=3584)
        # o_proj reads that copy's q output (2048 wide); down reads the SwiGLU output
        self.o_in = d(self.out["q_proj"], 1, 2048, P4, batch=copies, batch_stride=2048)
        self.down_in = d(self.h, 1, 3584, P4, batch=copies, batch_stride=3584)
        self.eps = 1e-6

    def launch(self, i: int):
        c, w = self.ctx, self.w
        if i == 0:
            c.linear_group([w["q_proj"], w["k_proj"], w["v_proj"]], self.xd,
                           [self.yd["q_proj"], self.yd["k_proj"], self.yd["v_proj"]],
                           rmsnorm=True, rms_gamma=self.gamma, rms_eps=self.eps)
        elif i == 1:
            c.linear(w["gate_proj"], self.xd, self.hd, rmsnorm=True, rms_gamma=self.gamma,
                     rms_eps=self.eps, up=w["up_proj"])
        elif i == 2:
            c.linear(w["o_proj"], self.o_in, self.yd["o_proj"])
        else:
            c.linear(w["down_proj"], self.down_in, self.yd["down_proj"])

    # algorithmic bytes of each launch for ONE copy (codes + scales + activations)
    def launch_bytes(self, i: int) -> int:
        def wb(n, k):
            return n * k // 2 + n * (k // 32) * 2
        d = self.dims
        if i == 0:
            return sum(wb(*d[nm]) + (d[nm][1] + d[nm][0]) * 2 for nm in ("q_proj", "k_proj", "v_proj"))
        if i == 1:
            return sum(wb(*d[nm]) + (d[nm][1] + d[nm][0]) * 2 for nm in ("gate_proj", "up_proj"))
        if i == 2:
            return wb(*d["o_proj"]) + (2048 + 1024) * 2
        return wb(*d["down_proj"]) + (3584 + 1024) * 2

    def step(self):
        for i in range(4):
            self.launch(i)


def time_launches(torch, fn, reps: int):
    """Average duration (ms) of fn() measured with HIP events on the current stream."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(reps)]
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    ts = sorted(a.elapsed_time(b) for a, b in evs)
    return sum(ts) / len(ts), ts[len(ts) // 2]


def per_call_cold(torch, aexq, synth, ctx, calls: int = 20):
    """BASELINE's per-call figure: before each timed call a 512 MiB scratch
    buffer is written (past the 256 MB Infinity Cache and every L2), then the
    call alone is bracketed by events.  Config 1 (one Q8 matvec) and config 2
    (one layer: its four launches, and each launch alone); medians."""
    scratch = torch.empty(128 << 20, dtype=torch.float32, device="cuda")   # 512 MiB
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(calls)]

    def cold(fn):
        for i, (a, b) in enumerate(evs):
            scratch.fill_(float(i))
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        ts = sorted(a.elapsed_time(b) for a, b in evs)
        return ts[len(ts) // 2]

    out = {}
    n, k = 3584, 1024
    words, scales, _ = synth.q8_weights(n, k, synth.SEED_BASE + 1)
    w = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    x = torch.as_tensor(synth.activations(1, k, 7)).cuda().reshape(-1)
    y = torch.zeros(n, dtype=torch.float16, device="cuda")
    xd, yd = aexq.describe(x, 1, k), aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR)
    for _ in range(3):
        ctx.linear(w, xd, yd)
    ms = cold(lambda: ctx.linear(w, xd, yd))
    b1 = n * k + n * 2 + k * 2 + n * 2
    out["config1_q8_m1_per_call"] = {"us": round(ms * 1e3, 2), "bytes": b1,
                                     "GBps": round(b1 / (ms * 1e-3) / 1e9, 1)}
    w.release()
    layer = Layer(ctx, aexq, synth, torch, 1, synth.SEED_BASE + 2)
    for _ in range(3):
        layer.step()
    ms = cold(layer.step)
    lb = sum(layer.launch_bytes(i) for i in range(4))
    per = {}
    for i, name in enumerate(("qkv_rms", "gate_up_swiglu_rms", "o_proj", "down_proj")):
        t = cold(lambda i=i: layer.launch(i))
        per[name] = {"us": round(t * 1e3, 2), "GBps": round(layer.launch_bytes(i) / (t * 1e-3) / 1e9, 1)}
    out["config2_layer_per_call"] = {"us": round(ms * 1e3, 2), "bytes": lb,
                                     "GBps": round(lb / (ms * 1e-3) / 1e9, 1), "launches": per,
                                     "note": "four dependent launches; each pays launch latency "
                                             "and a cold HBM round trip"}
    del scratch, layer
    torch.cuda.empty_cache()
    return out


def extras(torch, aexq, synth, ctx):
    """Per-config kernel measurements (sustained cold via rotating copies)."""
    out = {}
    # config 1: Q8 M=1 K=1024 N=3584, copies rotated so each launch is cold
    n, k = 3584, 1024
    words, scales, _ = synth.q8_weights(n, k, synth.SEED_BASE + 1)
    base = ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
    copies = 320
    stack = base.replicate(copies)
    base.release()
    x = torch.as_tensor(synth.activations(1, k, 7)).cuda().reshape(-1)
    y = torch.zeros(copies * n, dtype=torch.float16, device="cuda")
    xd = aexq.describe(x, 1, k)
    yd = aexq.describe(y, 1, n, aexq.LAYOUT_PACK4_LINEAR, batch=copies, batch_stride=n)
    bytes1 = n * k + n * 2 + k * 2 + n * 2
    for _ in range(3):
        ctx.linear(stack, xd, yd)
    avg, med = time_launches(torch, lambda: ctx.linear(stack, xd, yd), 20)
    out["config1_q8_m1_sustained"] = {"copies_per_launch": copies, "bytes_per_matvec": bytes1,
                                      "ms_per_launch": avg,
                                      "GBps": copies * bytes1 / (avg * 1e-3) / 1e9}
    stack.release()
    del y
    out.update(config5(torch, aexq, synth, ctx))
    return out


def config5(torch, aexq, synth, ctx, plain: bool = False):
    """Config 5: the LM head (Q8 per-row, K=1024, N=151,936) with the argmax
    fused, M = 1 and 8, eight rotated copies so every call is cold; each call
    between its own events and the same calls back to back.  plain: also the
    logits-only matvec of the same head (fp16 logits, no argmax) for
    comparison."""
    out = {}
    n, k = synth.VOCAB, synth.HIDDEN
    words, scales, _ = synth.q8_weights(n, k, synth.SEED_BASE + 5)
    heads = [ctx.weight(aexq.QuantizedTensor(n * k, k, words, scales, bits=8), n, k)
             for _ in range(8)]         # 8 x 156 MB rotated: each call is cold
    for m in (1, 8):
        xm = torch.as_tensor(synth.activations(m, k, 9)).cuda()
        xmd = aexq.describe(xm, m, k)
        lay = aexq.LAYOUT_PACK4_TILED
        logits = aexq.new_activation(m, n, torch.float32, lay)
        ld = aexq.describe(logits, m, n, lay)
        am = torch.zeros(m, dtype=torch.int32, device="cuda")
        it = [0]

        def call():
            ctx.lmhead_argmax(heads[it[0] % 8], xmd, ld, am)
            it[0] += 1
        for _ in range(8):
            call()
        avg, med = time_launches(torch, call, 24)
        # the same calls back to back between one pair of events (as a decode
        # loop issues the LM head behind the layer kernel): no per-call event gap
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(24):
            call()
        e1.record()
        torch.cuda.synchronize()
        stream_ms = e0.elapsed_time(e1) / 24
        b = n * k + n * 2 + m * k * 2 + m * n * 4
        out[f"config5_lmhead_m{m}"] = {"bytes": b, "ms_per_call": avg,
                                       "GBps": b / (avg * 1e-3) / 1e9,
                                       "ms_per_call_back_to_back": stream_ms,
                                       "GBps_back_to_back": b / (stream_ms * 1e-3) / 1e9,
                                       "note": ("one launch: " + ("streaming matvec" if m == 1
                                                                  else "MFMA matvec") +
                                                ", logits and argmax, the tagged partials "
                                                "merged by the last workgroup")}
    if plain:
        for m in (1, 8):
            xm = torch.as_tensor(synth.activations(m, k, 9)).cuda()
            xmd = aexq.describe(xm, m, k)
            y16 = aexq.new_activation(m, n, torch.float16, aexq.LAYOUT_PACK4_LINEAR)
            yd = aexq.describe(y16, m, n, aexq.LAYOUT_PACK4_LINEAR)
            it = [0]

            def lin():
                ctx.linear(heads[it[0] % 8], xmd, yd)
                it[0] += 1
            for _ in range(8):
                lin()
            avg, _ = time_launches(torch, lin, 24)
            b = n * k + n * 2 + m * k * 2 + m * n * 2
            out[f"config5_plain_matvec_m{m}"] = {"bytes": b, "ms_per_call": avg,
                                                 "GBps": b / (avg * 1e-3) / 1e9,
                                                 "note": "logits only (fp16), no argmax"}
    for h in heads:
        h.release()
    return out


def config4(torch, aexq, synth, ctx, copies: int = 120):
    """Benchmark config 4: the layer's linears at M in {16, 64, 512} rows, Q4 and Q8,
    on the MFMA path.  Each of the 120 copies (1.1 GB of Q4 weights) has its own
    activation rows and outputs, so every byte counted (weights, scales, x in,
    y out) streams from or to HBM once per step."""
    out = {}
    P4 = aexq.LAYOUT_PACK4_LINEAR
    for bits in (4, 8):
        ws = {}
        for i, (name, n, k) in enumerate(synth.LAYER_LINEARS):
            if bits == 4:
                words, scales, _ = synth.q4_weights(n, k, 700 + i, group=32, code=synth.NIBBLE_OFFSET8)
                qt = aexq.QuantizedTensor(n * k, 32, words, scales, bits=4, nibble_code=synth.NIBBLE_OFFSET8)
            else:
                words, scales, _ = synth.q8_weights(n, k, 700 + i)
                qt = aexq.QuantizedTensor(n * k, k, words, scales, bits=8)
            base = ctx.weight(qt, n, k)
            ws[name] = base.replicate(copies)
            base.release()
        wbytes = 9_142_272 if bits == 4 else 16_277_504
        for m in (16, 64, 512):
            # one copy of each activation per weight copy (the same values)
            xs = {k: torch.as_tensor(synth.activations(m, k, 800 + k)).cuda().reshape(1, -1)
                  .repeat(copies, 1).reshape(-1) for k in (1024, 2048, 3584)}
            gamma = torch.as_tensor(synth.rms_gamma(1024, 801)).cuda()
            ystride = {name: m * aexq.storage_elements(P4, m, n) for name, n, _ in synth.LAYER_LINEARS}
            ys = {name: torch.zeros(copies * ystride[name], dtype=torch.float16, device="cuda")
                  for name, n, _ in synth.LAYER_LINEARS}
            d = aexq.describe
            yd = {name: d(ys[name], m, n, P4, batch=copies, batch_stride=ystride[name])
                  for name, n, _ in synth.LAYER_LINEARS}
            xd = {k: d(v, m, k, batch=copies, batch_stride=m * k) for k, v in xs.items()}

            def step():
                ctx.linear_group([ws["q_proj"], ws["k_proj"], ws["v_proj"]], xd[1024],
                                 [yd["q_proj"], yd["k_proj"], yd["v_proj"]],
                                 rmsnorm=True, rms_gamma=gamma, rms_eps=1e-6)
                ctx.linear(ws["gate_proj"], xd[1024], yd["gate_proj"], rmsnorm=True,
                           rms_gamma=gamma, rms_eps=1e-6, up=ws["up_proj"])
                ctx.linear(ws["o_proj"], xd[2048], yd["o_proj"])
                ctx.linear(ws["down_proj"], xd[3584], yd["down_proj"])
            reps = 3 if m == 512 else 10
            avg, med = time_launches(torch, step, reps)
            b = copies * (wbytes + m * 46_080)
            fl = copies * 2 * m * 16_252_928
            out[f"config4_q{bits}_m{m}"] = {"copies": copies, "ms_per_step": round(med, 4),
                                            "GBps": round(b / (med * 1e-3) / 1e9, 1),
                                            "TFLOPs": round(fl / (med * 1e-3) / 1e12, 1)}
            log(f"config4 q{bits} m={m}: {out[f'config4_q{bits}_m{m}']}")
            del xs, ys
        for w in ws.values():
            w.release()
    return out


def config4_single(torch, aexq, synth, ctx, copies: int = 24):
    """Config 4 as a short prefill meets it: one layer's four launches (q/k/v
    group and gate/up pair with RMSNorm-in, o_proj, down) on ONE copy of the
    weights per launch, in Q4 (group 32, fp16 scales), Q8 and the reference's
    shipping Q4 (group 16, fp32 scales).  `copies` separate layers rotate so
    the weights come cold from HBM (24 Q4 layers: 220 MB); the calls are
    captured in a HIP graph and replayed, so the figure is GPU time per layer
    (the MFMA kernels split K across workgroups here: a single layer has too
    few output tiles to fill the part)."""
    import numpy as np
    out = {}
    P4 = aexq.LAYOUT_PACK4_LINEAR
    for tag, bits, group in (("q4", 4, 32), ("q8", 8, 0), ("q4g16", 4, 16)):
        layers = []
        wbytes = 0
        for c in range(copies):
            ws = {}
            for i, (name, n, k) in enumerate(synth.LAYER_LINEARS):
                if bits == 4:
                    sdt = np.float32 if group == 16 else np.float16
                    words, scales, _ = synth.q4_weights(n, k, 900 + i, group=group,
                                                        code=synth.NIBBLE_OFFSET8, scale_dtype=sdt)
                    qt = aexq.QuantizedTensor(n * k, group, words, scales, bits=4,
                                              nibble_code=synth.NIBBLE_OFFSET8)
                    if c == 0:
                        wbytes += n * k // 2 + scales.nbytes
                else:
                    words, scales, _ = synth.q8_weights(n, k, 900 + i)
                    qt = aexq.QuantizedTensor(n * k, k, words, scales, bits=8)
                    if c == 0:
                        wbytes += n * k + scales.nbytes
                ws[name] = ctx.weight(qt, n, k)
            layers.append(ws)
        gamma = torch.as_tensor(synth.rms_gamma(1024, 801)).cuda()
        for m in (16, 64, 512):
            xs = {k: torch.as_tensor(synth.activations(m, k, 800 + k)).cuda() for k in (1024, 2048, 3584)}
            ys = {name: torch.zeros(m * n, dtype=torch.float16, device="cuda")
                  for name, n, _ in synth.LAYER_LINEARS}
            d = aexq.describe
            yd = {name: d(ys[name], m, n, P4) for name, n, _ in synth.LAYER_LINEARS}
            xd = {k: d(v, m, k) for k, v in xs.items()}
            it = [0]

            def step():
                ws = layers[it[0] % copies]
                it[0] += 1
                ctx.linear_group([ws["q_proj"], ws["k_proj"], ws["v_proj"]], xd[1024],
                                 [yd["q_proj"], yd["k_proj"], yd["v_proj"]],
                                 rmsnorm=True, rms_gamma=gamma, rms_eps=1e-6)
                ctx.linear(ws["gate_proj"], xd[1024], yd["gate_proj"], rmsnorm=True,
                           rms_gamma=gamma, rms_eps=1e-6, up=ws["up_proj"])
                ctx.linear(ws["o_proj"], xd[2048], yd["o_proj"])
                ctx.linear(ws["down_proj"], xd[3584], yd["down_proj"])
            for _ in range(copies):
                step()   # plans and scratch sized before the capture
            torch.cuda.synchronize()
            stream = torch.cuda.Stream()
            ctx.set_stream(stream)
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                step()
            stream.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for _ in range(copies):
                    step()
            ctx.set_stream(torch.cuda.current_stream())
            g.replay()
            torch.cuda.synchronize()
            avg, med = time_launches(torch, g.replay, 10)
            us = med * 1e3 / copies
            b = wbytes + m * 46_080
            out[f"config4_single_{tag}_m{m}"] = {
                "us_per_layer": round(us, 2), "GBps": round(b / us / 1e3, 1),
                "TFLOPs": round(2 * m * 16_252_928 / us / 1e6, 1), "copies_rotated": copies}
            log(f"config4 single {tag} m={m}: {out[f'config4_single_{tag}_m{m}']}")
            del g, xs, ys
        for ws in layers:
            for w in ws.values():
                w.release()
    return out


def config3(torch, aexq, ctx, steps: int = 30):
    """Benchmark config 3: one full synthetic Qwen3.5-0.8B-shaped decode step
    (24 layers, 2048 cached positions, Q8 LM head with argmax); tokens/s
    against the step's algorithmic bytes.  Two forms of the step: the fused
    one (every decoder layer in one persistent launch, aexq_decoder_run) and
    the per-operator one (five launches per layer); each eager, as a replayed
    HIP graph, and as the Generate loop (one graph per token that feeds the
    argmax back and advances the device position).  The fused form also as
    graphs of 8 steps (a graph launch leaves the device idle for about 8 us
    between replays): the same step replayed, and the Generate loop decoding 8
    tokens per replay."""
    from aiimage_amd import decoder
    cfg = decoder.ModelConfig()
    t0 = time.time()
    sess = decoder.DecodeSession(ctx, cfg, fused=True)
    log(f"config3 model built in {time.time() - t0:.1f} s ({sess.fused.info()})")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn):
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    def measure(multi=False):
        sess.token.fill_(1)
        sess.set_position(cfg.capacity - 1)     # attends over all 2048 positions
        for _ in range(2):
            sess.step(check=False)
        torch.cuda.synchronize()
        eager_ms = timed(lambda: sess.step(check=False))
        g = sess.capture()
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        graph_ms = timed(g.replay)
        ga = sess.capture(advance=True)
        start = cfg.capacity - steps
        sess.generate(1, start - 3, 3, graph=ga)          # warm replays
        sess.token.fill_(1)
        sess.set_position(start)
        torch.cuda.synchronize()
        gen_ms = timed(ga.replay)
        assert int(sess.pos.item()) == cfg.capacity
        del g, ga
        if not multi:
            return eager_ms, graph_ms, gen_ms, start, None, None
        # 8 steps per graph: the same step (4 replays, 32 steps), and 8 tokens
        # per replay of the Generate loop over the same last 24 positions
        g8 = sess.capture(steps=8)
        sess.token.fill_(1)
        sess.set_position(cfg.capacity - 1)
        g8.replay()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(4):
            g8.replay()
        e1.record()
        torch.cuda.synchronize()
        graph8_ms = e0.elapsed_time(e1) / 32
        ga8 = sess.capture(advance=True, steps=8)
        sess.generate(1, cfg.capacity - 48, 16, graph=ga8, graph_steps=8)   # warm replays
        sess.token.fill_(1)
        sess.set_position(cfg.capacity - 24)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(3):
            ga8.replay()
        e1.record()
        torch.cuda.synchronize()
        gen8_ms = e0.elapsed_time(e1) / 24
        assert int(sess.pos.item()) == cfg.capacity
        del g8, ga8
        return eager_ms, graph_ms, gen_ms, start, graph8_ms, gen8_ms

    eager_ms, graph_ms, gen_ms, start, graph8_ms, gen8_ms = measure(multi=True)
    err = sess.fused.error()
    assert err == 0, "the fused step gave up a bounded wait"
    keep, sess.fused = sess.fused, None
    p_eager, p_graph, p_gen, _, _, _ = measure()
    sess.fused = keep
    b = cfg.bytes_per_token(cfg.capacity)
    roof = HBM_PEAK_GBS * 1e9 / b["total"]
    # BASELINE.json's "8 kv heads" reading: twice the cached K/V bytes
    roof8 = HBM_PEAK_GBS * 1e9 / (b["total"] + b["kv_read"])
    mean_len = start + (steps + 1) / 2.0
    b_gen = cfg.bytes_per_token(int(round(mean_len)))["total"]
    tps = lambda ms: round(1000.0 / ms, 1)
    out = {"config3_decode": {
        "step": "fused decoder layers (one launch) + LM head with the final RMSNorm and argmax",
        "tokens_per_s_graph": tps(graph_ms), "ms_per_token_graph": round(graph_ms, 4),
        "tokens_per_s_eager": tps(eager_ms), "ms_per_token_eager": round(eager_ms, 4),
        "tokens_per_s_generate": tps(gen_ms), "ms_per_token_generate": round(gen_ms, 4),
        "generate_positions": [start, cfg.capacity - 1],
        "tokens_per_s_graph8": tps(graph8_ms), "ms_per_token_graph8": round(graph8_ms, 4),
        "tokens_per_s_generate8": tps(gen8_ms), "ms_per_token_generate8": round(gen8_ms, 4),
        "generate8_positions": [cfg.capacity - 24, cfg.capacity - 1],
        "generate_frac_of_roofline": round(b_gen / (gen_ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
        "bytes_per_token": b, "roofline_tokens_per_s": round(roof, 1),
        "roofline_tokens_per_s_8kv_heads": round(roof8, 1),
        "frac_of_roofline": round(1000.0 / graph_ms / roof, 4),
        "frac_of_roofline_8kv_heads": round(1000.0 / graph_ms / roof8, 4),
        "GBps_graph": round(b["total"] / (graph_ms * 1e-3) / 1e9, 1),
        "kv_heads": cfg.heads_kv, "positions": cfg.capacity, "layers": cfg.layers,
        "fused_grid": sess.fused.info(),
        # the fused layers and the LM head (RMSNorm-in, in-kernel argmax merge);
        # the Generate loop adds the advance
        "launches_per_token": 2,
        "per_operator": {
            "tokens_per_s_graph": tps(p_graph), "ms_per_token_graph": round(p_graph, 4),
            "tokens_per_s_eager": tps(p_eager), "ms_per_token_eager": round(p_eager, 4),
            "tokens_per_s_generate": tps(p_gen), "ms_per_token_generate": round(p_gen, 4),
            # embedding; per layer q/k/v, attention, o_proj, gate/up, down;
            # the LM head
            "launches_per_token": 1 + cfg.layers * 5 + 1}}}
    log(f"config3: {out['config3_decode']}")
    del sess
    torch.cuda.empty_cache()
    # the same step on the reference's own layer formats (its shipping Q4
    # archives: two's-complement nibbles with an fp32 scale per 16 codes; Q8
    # layers with an fp32 scale per row), fused and per operator, as graphs
    formats = {}
    for mk in (decoder.ModelConfig.reference_q4, decoder.ModelConfig.reference_q8):
        fc = mk()
        fs = decoder.DecodeSession(ctx, fc, fused=True)
        fs.token.fill_(1)
        fs.set_position(fc.capacity - 1)
        res = {}
        for form in ("fused", "per_operator"):
            keep = fs.fused
            if form == "per_operator":
                fs.fused = None
            g = fs.capture()
            for _ in range(3):
                g.replay()
            torch.cuda.synchronize()
            res[form] = timed(g.replay)
            del g
            fs.fused = keep
        fs.check_fused()
        fb = fc.bytes_per_token(fc.capacity)
        froof = HBM_PEAK_GBS * 1e9 / fb["total"]
        formats[fc.format_name] = {
            "tokens_per_s_graph": tps(res["fused"]), "ms_per_token_graph": round(res["fused"], 4),
            "per_operator_tokens_per_s_graph": tps(res["per_operator"]),
            "bytes_per_token": fb["total"], "roofline_tokens_per_s": round(froof, 1),
            "frac_of_roofline": round(1000.0 / res["fused"] / froof, 4),
            "fused_grid": fs.fused.info()}
        log(f"config3 {fc.format_name}: {formats[fc.format_name]}")
        del fs
        torch.cuda.empty_cache()
    out["config3_decode"]["formats"] = formats
    return out


def host_cpu() -> dict:
    """The host's CPU: model, logical CPUs, the CPUs this process may run on,
    and the threads the all-cores runs use (the job's CPU share: the smaller of
    the affinity set and OMP_NUM_THREADS where that is set)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    nproc = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = nproc
    share = avail
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        share = min(share, int(env))
    return {"cpu_model": model, "nproc": nproc, "affinity_cpus": avail, "threads_used": share}


def cpu_baseline(seconds: float):
    """RunGemmCpu (GS:13328-13381) restated in C, timed on this host: the seven
    linears of one layer on dequantized fp32 weights (dequant untimed, as at
    reference load time), float64 accumulation, single thread -- the reported
    baseline.  Beside it, bounded samples of the same loop split over output
    columns on the host's cores (identical results) and of configs 1 and 5,
    and the linear part of config 3 derived from them."""
    import numpy as np

    import oracle
    from aiimage_amd import synth
    host = host_cpu()
    threads = host["threads_used"]

    def timed(fn, budget, min_runs=10):
        """Median seconds per run over at least min_runs runs and `budget` s."""
        runs, t0 = [], time.perf_counter()
        while len(runs) < min_runs or time.perf_counter() - t0 < budget:
            a = time.perf_counter()
            fn()
            runs.append(time.perf_counter() - a)
        runs.sort()
        return runs[len(runs) // 2], len(runs), time.perf_counter() - t0

    lin = []
    for i, (name, n, k) in enumerate(synth.LAYER_LINEARS):
        words, scales, _ = synth.q4_weights(n, k, 1000 + i, group=32, code=synth.NIBBLE_OFFSET8)
        wf = oracle.dequant_q4(words, scales, n, k, 32, oracle.NIBBLE_OFFSET8, oracle.SCALE_F16)
        x = synth.activations(1, k, 2000 + i).astype(np.float32)
        lin.append((x, wf, n))

    def layer(th):
        for x, wf, n in lin:
            oracle.gemm_cpu(x, wf, n, True, threads=th)

    per_layer, layers, el = timed(lambda: layer(1), seconds)
    out = {"value": LAYER_BYTES / per_layer / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": f"median of {layers} passes of one layer's 7 Q4 linears (M=1) through the C "
                     f"restatement of RunGemmCpu on dequantized fp32 weights ({el:.1f} s), "
                     f"{per_layer * 1e3:.2f} ms per layer; rate in algorithmic quantized bytes",
           "host": host}
    budget = max(1.0, seconds / 5)
    per_layer_mt, _, _ = timed(lambda: layer(threads), budget)
    cfg = {"config2_all_cores": {"GBps": LAYER_BYTES / per_layer_mt / 1e9, "cores": threads}}
    # config 1: Q8 1024 -> 3584
    w8, s8, _ = synth.q8_weights(3584, 1024, 3000)
    wf8 = oracle.dequant_q8(w8, s8, 3584, 1024, scale_dtype=oracle.SCALE_F16)
    x1 = synth.activations(1, 1024, 3001).astype(np.float32)
    for th, key in ((1, "config1_single"), (threads, "config1_all_cores")):
        t, _, _ = timed(lambda th=th: oracle.gemm_cpu(x1, wf8, 3584, True, threads=th), budget)
        cfg[key] = {"GBps": 3_686_400 / t / 1e9, "cores": th}
    del wf8
    # config 5: the Q8 LM head, M = 1
    wl, sl, _ = synth.q8_weights(synth.VOCAB, synth.HIDDEN, 3002)
    wfl = oracle.dequant_q8(wl, sl, synth.VOCAB, synth.HIDDEN, scale_dtype=oracle.SCALE_F16)
    del wl
    xl = synth.activations(1, synth.HIDDEN, 3003).astype(np.float32)
    lm = {}
    for th, key in ((1, "config5_m1_single"), (threads, "config5_m1_all_cores")):
        t, _, _ = timed(lambda th=th: oracle.gemm_cpu(xl, wfl, synth.VOCAB, True, threads=th), budget)
        lm[th] = t
        cfg[key] = {"GBps": 156_496_128 / t / 1e9, "ms": t * 1e3, "cores": th}
    del wfl
    # config 3, linear part only (24 layers + LM head; no attention on the CPU path)
    for th, key, pl in ((1, "config3_linears_single", per_layer),
                        (threads, "config3_linears_all_cores", per_layer_mt)):
        step = 24 * pl + lm[th]
        cfg[key] = {"tokens_per_s": 1.0 / step, "ms_per_token": step * 1e3, "cores": th}
    out["configs"] = {k: {a: (round(b, 4) if isinstance(b, float) else b) for a, b in v.items()}
                      for k, v in cfg.items()}
    return out


def decode_phases(torch, steps: int = 10):
    """Per-phase times of the fused decode step (config 3 shapes, 2048 cached
    positions) for the benchmark's Q4 and the reference's Q4-g16 and Q8
    formats, from the phase-stamped build of the library: per workgroup and
    layer, the compute time of each phase (barrier to the compute waves' last
    output) and its hand-over (to the next workgroup barrier, which waits for
    the grid's outputs the next phase polls); medians over workgroups and
    layers 1..L-1 (layer 0 includes the launch prologue)."""
    import ctypes
    import numpy as np
    from aiimage_amd import _abi, build as hip_build
    if not os.path.exists(hip_build.LIB_STAMPS):
        hip_build.build(stamps=True)
    lib = _abi.load(hip_build.LIB_STAMPS)
    lib.aexq_step_stamps.argtypes = [ctypes.c_void_p, ctypes.c_longlong]
    from aiimage_amd import aexq, decoder
    ctx = aexq.Context(0)
    names = ["P1 q/k/v", "P2 attention splits + split merge", "P3 o_proj + residual",
             "P4 gate/up + SwiGLU", "P5 down + residual"]
    out = {"library": os.path.basename(hip_build.LIB_STAMPS), "formats": {}}
    for mk in (decoder.ModelConfig, decoder.ModelConfig.reference_q4,
               decoder.ModelConfig.reference_q8):
        cfg = mk()
        sess = decoder.DecodeSession(ctx, cfg, fused=True)
        grid = sess.fused.info()["workgroups"]
        sess.token.fill_(1)
        sess.set_position(cfg.capacity - 1)
        for _ in range(3):
            sess.step(check=False)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            sess.step(check=False)
        e1.record()
        torch.cuda.synchronize()
        sess.check_fused()
        n = cfg.layers * 10 * grid
        buf = (ctypes.c_ulonglong * n)()
        if lib.aexq_step_stamps(buf, n) != 0:
            raise RuntimeError("aexq_step_stamps failed")
        st = np.frombuffer(buf, dtype=np.uint64).astype(np.int64).reshape(cfg.layers, 10, grid) * 10
        rows = []
        for ph in range(5):
            prev = st[:-1, 9, :] if ph == 0 else st[1:, 2 * ph - 1, :]
            comp = (st[1:, 2 * ph, :] - prev) / 1e3
            hand = (st[1:, 2 * ph + 1, :] - st[1:, 2 * ph, :]) / 1e3
            rows.append({"phase": names[ph], "compute_us": round(float(np.median(comp)), 2),
                         "compute_us_p90": round(float(np.percentile(comp, 90)), 2),
                         "handover_us": round(float(np.median(hand)), 2),
                         "handover_us_p90": round(float(np.percentile(hand, 90)), 2)})
        layer = np.diff(st[:, 9, :], axis=0) / 1e3
        out["formats"][cfg.format_name] = {
            "ms_per_step_eager": round(e0.elapsed_time(e1) / steps, 4), "workgroups": grid,
            "layers": cfg.layers, "layer_us": round(float(np.median(layer)), 2), "phases": rows}
        del sess
        torch.cuda.synchronize()
    return out


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the matvec would shard by output rows, one slice of the weight rows "
              "per GPU)", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.decode_phases:
        if not torch.cuda.is_available():
            print("bench.py needs a GPU", file=sys.stderr)
            sys.exit(2)
        print(json.dumps(decode_phases(torch)), flush=True)
        return
    from aiimage_amd import aexq, synth
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    ctx = aexq.Context(0)
    if args.decode_only:
        print(json.dumps(config3(torch, aexq, ctx, steps=max(args.steps, 10))), flush=True)
        return
    if args.lmhead_only:
        print(json.dumps(config5(torch, aexq, synth, ctx, plain=True)), flush=True)
        return
    if args.config4_only:
        res = config4(torch, aexq, synth, ctx)
        res.update(config4_single(torch, aexq, synth, ctx))
        print(json.dumps(res), flush=True)
        return
    if args.calib:
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)       # reads 256 MiB, writes 256 MiB
        torch.cuda.synchronize()
        del src, dst
    # the smallest launch (o_proj: 1024 x 2048 Q4 codes + fp16 group scales)
    o_proj_bytes = 1024 * 2048 // 2 + 1024 * (2048 // 32) * 2
    copies = args.copies or -(-GIB // o_proj_bytes)
    log(f"building {copies} cold copies of the layer ({copies * LAYER_WEIGHT_BYTES / 1e9:.2f} GB)")
    layer = Layer(ctx, aexq, synth, torch, copies, synth.SEED_BASE + 2)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        layer.step()
    torch.cuda.synchronize()
    log(f"warmup done; timing {args.steps} steps")
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for _ in range(args.steps):
        layer.step()
    t1.record()
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    value = copies * LAYER_BYTES / (ms_per_step * 1e-3) / 1e9
    log(f"{ms_per_step:.4f} ms/step -> {value:.1f} GB/s")

    # per-launch durations; the dominant launch carries the roofline
    per = {}
    for i, name in enumerate(("qkv_rms", "gate_up_swiglu_rms", "o_proj", "down_proj")):
        avg, med = time_launches(torch, lambda i=i: layer.launch(i), max(10, args.steps))
        b = copies * layer.launch_bytes(i)
        per[name] = {"ms": avg, "ms_median": med, "bytes": b, "GBps": b / (avg * 1e-3) / 1e9}
    dom = max(per, key=lambda k: per[k]["ms"])
    ach = per[dom]["GBps"]
    traffic, traffic_note = measured_traffic(dom, copies)
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
                "traffic_source": traffic_note, "kernel_source_sha256": kernel_source_hash(),
                "algorithmic_bytes": per[dom]["bytes"]}
    result = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "config2: one decoder layer's 7 Q4 linears, M=1, cold (sustained)",
                   "copies_per_step": copies, "algorithmic_bytes_per_layer": LAYER_BYTES,
                   "q4": "offset-8, fp16 scale per 32 K", "accumulate": "f32",
                   "epilogues": "RMSNorm-in (q/k/v, gate/up), SwiGLU-out (gate/up)",
                   "launches_per_step": 4,
                   "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
        "launches": per,
    }
    if not args.no_extra:
        del layer
        torch.cuda.empty_cache()
        log("extras: config 1 and config 5")
        result["extra"] = extras(torch, aexq, synth, ctx)
        result["extra"].update(per_call_cold(torch, aexq, synth, ctx))
        result["extra"].update(config3(torch, aexq, ctx))
        result["extra"].update(config4(torch, aexq, synth, ctx))
        result["extra"].update(config4_single(torch, aexq, synth, ctx))
    if not args.no_cpu:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
