#!/usr/bin/env python3
"""Benchmark of the MI355X Q8_0 / Q4_K FC hot path (one JSON line on stdout).

Workload (the headline configuration, cfg2): one MaskGIT transformer
layer's four Q8_0 FC GEMMs at M = 1025 tokens (32x32 grid + class token), fp32 activations:
    QKV   768 -> 2304  (+bias)            (q/k/v stacked: Q8_0 blocks are row-local)
    out   768 -> 768   (+bias +residual)
    up    768 -> 3072  (+bias, GELU)
    down 3072 -> 768   (+bias +residual)
A step runs each FC of the chosen path, all inputs already resident in HBM, the weights
prepared once at upload (outside the timed region, as the reference uploads each weight once):
  --path dq (default, the headline): the dequantize-fused path on the quantized bytes --
    k_gemm_fc<..., WQ=8> reads the Q8_0 blocks on every call (regrouped once at upload into
    MFMA fragment order, 1.0625 bytes per weight, the GGUF size) and decodes each weight to
    fp16 inside the K loop, as the reference's k_mul_mat_q8_0_t2_h does; the fp32 activations
    are rounded to fp16 as they are read; fp16 MFMA, fp32 accumulation, fused
    bias/GELU/residual epilogue. It meets the 1e-3 * max|y| bar against the reference's
    dequantize-then-F32 product;
  --path h16: the same product on fp16 weight copies made at upload (k_gemm_fc<..., WQ=0>,
    2 bytes per weight read, no decoding in the K loop; identical outputs);
  --path packed (the int8-dot path, bit-exact int32 block dots of the reference's int8
    kernels): per-32 int8 activation quantization (k_quantize_act_q8, codes as fp16), then
    k_gemm_qp on the packed codes with per-block scales applied in fp32;
  --path raw: the int8-dot path on one-byte operands: int8 activation codes and the GGUF blocks
    as stored, on int8 MFMA (k_gemm_q_i8).
Every path is measured on every GEMM workload of the metric (Q8_0 and Q4_K at M = 1025 and
4097) and reported under extra.<wtype>_m<M> with its TOPS and fraction of the HBM roofline.
The step's kernels are enqueued one by one on the context's stream (--graphs instead captures
each buffer set's step once as a HIP graph and replays it; for these few-kernel steps the
graph launch measured slower). Buffers rotate over >= --rotate-gb of distinct sets so the 256 MB
MALL and the L2s do not serve the timed reads. Before the W warmup steps the step runs untimed
for 0.25 s, so the timed K steps see steady-state GPU clocks. extra.cfg2_hot_cache repeats the
step on two buffer sets (warm caches) for comparison. Synthetic data: x ~ N(0,1), W ~ N(0,0.02)
quantized to Q8_0, biases ~ N(0,0.01), residuals ~ N(0,1), seeded.

value = 2*M*K*N summed over the four GEMMs / step time, in TOPS.
roofline = the dominant kernel (k_gemm_fc on the dq / h16 paths, k_gemm_qp / k_gemm_q_i8 on the
int8 paths), HBM-bound: algorithmic bytes of its launches (quantized weights once + the
activations it reads: fp32 on the dq / h16 paths, int8 codes + block scales on the int8 paths +
fp32 output + bias + residual) divided by its average launch duration, timed with HIP events
on the stream it runs on; traffic = the measured HBM bytes of those launches (rocprofv3
FETCH_SIZE + WRITE_SIZE, calibrated on a plain copy), from profiles/traffic_*.json, reported only
when that file was measured on the same kernel sources (SHA-256 of edge_maskgit_amd/csrc, also
in config.csrc_sha256_16), else null with the reason in roofline.traffic_source.
cpu_baseline = the reference's own CPU executor (mg-cpu k_mul_mat, single thread, built
from the reference sources into oracle/_ref) on the dequantized weights, timed on this
host over the same four GEMMs; if that library is absent, the C oracle's int8 path.
extra.vqgan_decode = the production VQGAN decoder graph (256 tokens -> 256 x 256 image, 128
filters, multipliers 1,1,2,2,4) on random-init weights through mgr_decode_images, for one image
and a batch of 8: wall ms per decode with the ids already prepared and the image left in HBM,
the per-op device profile, the conv kernels' fraction of the fp32 MFMA peak, and a bounded
sample of the reference's CPU conv (--no-vqgan skips it; --only-vqgan measures only it).
extra.generate_images = the reference's whole generate() (8 device-resident decode steps of a
24-layer Q4_K transformer, then the VQGAN decode) for 1 and 8 images, wall clock per call.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import edge_maskgit_amd as ema  # noqa: E402

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0    # MI355X dense int8 MFMA, published

LAYER = [  # name, N, K, act, residual
    ("qkv", 2304, 768, ema.ACT_NONE, False),
    ("out", 768, 768, ema.ACT_NONE, True),
    ("up", 3072, 768, ema.ACT_GELU, False),
    ("down", 768, 3072, ema.ACT_NONE, True),
]
CFG1 = [("cfg1", 3072, 768, ema.ACT_NONE, False)]   # configs[0]: one Q8_0 FC GEMM at M=257


KERNEL = {"packed": "k_gemm_qp", "raw": "k_gemm_q_i8", "h16": "k_gemm_fc<..., WQ=0>",
          "dq": "k_gemm_fc<..., WQ=8|12>"}
# profiles/traffic_<name>_cfg2_q8_m1025.json: the counter-measured HBM bytes of each path's step
TRAFFIC_FILE = {"dq": "k_gemm_fc_dq", "h16": "k_gemm_fc_f16", "packed": "k_gemm_qp", "raw": "k_gemm_q_i8"}
# bytes each path's GEMM kernel reads per weight, Q8_0 / Q4_K
WEIGHT_BYTES = {"dq": {8: 1.0625, 12: 0.5625}, "raw": {8: 1.0625, 12: 0.5625},
                "h16": {8: 2.0, 12: 2.0}, "packed": {8: 2.125, 12: 2.25}}
PATH_NAME = {"packed": "int8_dot", "raw": "int8_dot_raw", "h16": "dequant_f16", "dq": "dequant_q"}
WORKLOAD_PATH = {
    "h16": "dequantize-fused path (weights dequantized once to fp16 at upload; per FC one GEMM "
           "launch: fp32 activations rounded to fp16 as they are read, fp16 MFMA with fp32 "
           "accumulation, fused epilogue)",
    "packed": "int8-dot path (per FC: per-32 int8 activation quantization + exact block dots with "
              "per-block scales applied in fp32)",
    "raw": "int8-dot path on GGUF blocks as stored",
    "dq": "dequantize-fused path on the quantized bytes (per FC one GEMM launch reading the Q8_0 / "
          "Q4_K blocks, regrouped once at upload into MFMA fragment order at the GGUF byte count, "
          "decoded to fp16 in registers inside the K loop; fp32 activations rounded to fp16 as they "
          "are read; fp16 MFMA with fp32 accumulation; fused epilogue)"}
ALGO = {"packed": 1, "raw": 1, "h16": 2, "dq": 2}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def row_bytes(wtype, K):
    return (K // 32) * 34 if wtype == ema.WTYPE_Q8_0 else (K // 256) * 144


class LayerSet:
    """One set of device buffers for the four FC GEMMs of a layer.

    path "packed" (int8-dot production path): weights rewritten once at upload into the
    device-native layout (mgh_pack_weights, outside the timed region, as the reference uploads
    each weight once), then per FC: quantizer (fp16 codes) + mgh_gemm_q_packed.
    path "h16" (dequantize-fused production path): weights dequantized once at upload into
    fp16 (mgh_pack_weights_f16), then per FC one mgh_gemm_h16_f32in (the fp32 activations are
    rounded to fp16 inside the GEMM).
    path "raw": GGUF blocks as stored, per FC: int8 quantizer + mgh_gemm_q (the int8-MFMA
    raw-block kernel)."""

    def __init__(self, ctx, host, M, wtype, path="packed", layer=LAYER):
        self.ctx = ctx
        self.M = M
        self.wtype = wtype
        self.path = path
        self.g = []
        for (name, N, K, act, res), h in zip(layer, host):
            nb = K // 32
            w = ctx.upload(h["wq"])
            if path == "h16":
                wp = ctx.alloc(ema.packed_weight_bytes_f16(N, K))
                ctx.pack_weights_f16(wtype, w, N, K, wp)
                ctx.sync()
                ctx.free(w)
                w = wp
            elif path == "dq":
                wp = ctx.alloc(ema.packed_weight_bytes_dq(wtype, N, K))
                ctx.pack_weights_dq(wtype, w, N, K, wp)
                ctx.sync()
                ctx.free(w)
                w = wp
            elif path == "packed":
                wp = ctx.alloc(ema.packed_weight_bytes(wtype, N, K))
                ctx.pack_weights(wtype, w, N, K, wp)
                ctx.sync()
                ctx.free(w)
                w = wp
            d = dict(name=name, N=N, K=K, act=act,
                     w=w, x=ctx.upload(h["x"]), b=ctx.upload(h["bias"]),
                     r=ctx.upload(h["resid"]) if res else None, y=ctx.alloc(M * N * 4),
                     qx=ctx.alloc(M * K * 2), dx=ctx.alloc(M * nb * 4), sx=ctx.alloc(M * nb * 4))
            self.g.append(d)

    def _gemm(self, d):
        c = self.ctx
        if self.path == "h16":
            c.gemm_h16(d["w"], d["N"], d["K"], d["qx"], self.M, d["b"], d["act"], d["r"], d["y"])
            return
        f = c.gemm_q_packed if self.path == "packed" else c.gemm_q
        f(self.wtype, d["w"], d["N"], d["K"], d["qx"], d["dx"], d["sx"], self.M,
          d["b"], d["act"], d["r"], d["y"])

    def step(self):
        c = self.ctx
        for d in self.g:
            if self.path == "h16":         # fp32 activations rounded to fp16 inside the GEMM
                c.gemm_h16_f32in(d["w"], d["N"], d["K"], d["x"], self.M, d["b"], d["act"], d["r"], d["y"])
                continue
            if self.path == "dq":
                c.gemm_dq_f32in(self.wtype, d["w"], d["N"], d["K"], d["x"], self.M, d["b"], d["act"], d["r"],
                                d["y"])
                continue
            if self.path == "packed":
                c.quantize_act_q8_codes16(d["x"], self.M, d["K"], d["qx"], d["dx"], d["sx"])
            else:
                c.quantize_act_q8(d["x"], self.M, d["K"], d["qx"], d["dx"], d["sx"])
            self._gemm(d)

    def gemms_only(self):
        if self.path in ("h16", "dq"):     # the GEMM launches are the whole step
            self.step()
            return
        for d in self.g:
            self._gemm(d)


def csrc_digest():
    """First 16 hex digits of the SHA-256 of the kernel library's sources (edge_maskgit_amd/csrc,
    file names and contents in name order): the key that ties a committed rocprofv3 traffic file
    to the kernels it was measured on."""
    import hashlib
    h = hashlib.sha256()
    d = os.path.join(ROOT, "edge_maskgit_amd", "csrc")
    for f in sorted(os.listdir(d)):
        if f.endswith((".hip", ".cpp", ".h")):
            h.update(f.encode())
            with open(os.path.join(d, f), "rb") as fh:
                h.update(fh.read())
    return h.hexdigest()[:16]


def measured_traffic(path, digest):
    """HBM bytes per step of the headline launches from a committed rocprofv3 summary (FETCH_SIZE +
    WRITE_SIZE, scaled on a plain copy): (bytes, provenance) when the file was measured on kernel
    sources with this digest, (None, provenance with the reason) when it was not, (None, None)
    when there is no file."""
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        tj = json.load(f)
    src = {"file": os.path.relpath(path, ROOT), "git_head": tj.get("git_head"),
           "csrc_sha256_16": tj.get("csrc_sha256_16"), "command": tj.get("command")}
    if tj.get("csrc_sha256_16") == digest:
        return tj.get("traffic_bytes_per_step"), src
    src["stale"] = f"measured on kernel sources {tj.get('csrc_sha256_16')}, this run's are {digest}: not used"
    return None, src


def synth_q8_0(w):
    """Synthetic-data encoder: ggml Q8_0 blocks (fp16 d = amax/127, int8 q = rint(w/d))."""
    N, K = w.shape
    b = w.reshape(N, K // 32, 32)
    d = (np.abs(b).max(-1) / np.float32(127)).astype(np.float32)
    q = np.clip(np.rint(b / np.where(d > 0, d, 1)[..., None]), -127, 127).astype(np.int8)
    out = np.empty((N, K // 32, 34), np.uint8)
    out[..., 0:2] = d.astype(np.float16)[..., None].view(np.uint8)
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(N, -1)


def synth_q4_k(w):
    """Synthetic-data encoder: ggml Q4_K super-blocks (min/max sub-block scales)."""
    N, K = w.shape
    x = w.reshape(-1, 8, 32)
    mn = np.minimum(x.min(-1), 0)
    sc = (x.max(-1) - mn) / 15.0
    d = sc.max(-1) / 63.0
    dm = (-mn).max(-1) / 63.0
    scq = np.clip(np.rint(sc / np.where(d > 0, d, 1)[:, None]), 0, 63).astype(np.uint8)
    mq = np.clip(np.rint(-mn / np.where(dm > 0, dm, 1)[:, None]), 0, 63).astype(np.uint8)
    step = np.where(d[:, None] * scq > 0, d[:, None] * scq, 1.0)
    q = np.clip(np.rint((x + (dm[:, None] * mq)[..., None]) / step[..., None]), 0, 15).astype(np.uint8)
    out = np.zeros((x.shape[0], 144), np.uint8)
    out[:, 0:2] = d.astype(np.float16)[:, None].view(np.uint8)
    out[:, 2:4] = dm.astype(np.float16)[:, None].view(np.uint8)
    out[:, 4:8] = (scq[:, :4] & 63) | ((scq[:, 4:] >> 4) << 6)
    out[:, 8:12] = (mq[:, :4] & 63) | ((mq[:, 4:] >> 4) << 6)
    out[:, 12:16] = (scq[:, 4:] & 0xF) | ((mq[:, 4:] & 0xF) << 4)
    for g in range(4):
        out[:, 16 + 32 * g:48 + 32 * g] = q[:, 2 * g] | (q[:, 2 * g + 1] << 4)
    return out.reshape(N, -1)


def host_layer(M, wtype, seed=0, layer=LAYER):
    rng = np.random.default_rng(seed)
    out = []
    enc = synth_q8_0 if wtype == ema.WTYPE_Q8_0 else synth_q4_k
    for name, N, K, act, res in layer:
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        out.append(dict(w=w, wq=enc(w),
                        x=rng.standard_normal((M, K)).astype(np.float32),
                        bias=(rng.standard_normal(N) * 0.01).astype(np.float32),
                        resid=rng.standard_normal((M, N)).astype(np.float32) if res else None))
    return out


def layer_ops(M, layer=LAYER):
    return sum(2.0 * M * N * K for _, N, K, _, _ in layer)


def gemm_alg_bytes(M, wtype, path="h16", layer=LAYER):
    """Algorithmic HBM bytes of the four GEMM launches of one step: the quantized weights
    once, the activations the launch reads (h16 path: the fp32 rows, rounded in the kernel;
    int8-dot paths: fp16-held or one-byte codes + fp32 block scales (+ block sums for Q4_K)), the fp32 output,
    bias and residual."""
    tot = 0
    for _, N, K, act, res in layer:
        nb = K // 32
        if path in ("h16", "dq"):          # fp32 activations read by the GEMM itself
            tot += N * row_bytes(wtype, K) + M * K * 4 + M * N * 4 + N * 4
        else:                              # int8 codes: fp16-held (packed) or one byte (raw)
            tot += N * row_bytes(wtype, K) + M * K * (2 if path == "packed" else 1) + M * N * 4 + N * 4
            tot += M * nb * 4 * (2 if wtype == ema.WTYPE_Q4_K else 1)
        if res:
            tot += M * N * 4
    return tot


def step_alg_bytes(M, wtype, layer=LAYER):
    """Algorithmic bytes of the whole FC op: weights once, fp32 x once, fp32 y once, bias,
    residual once."""
    tot = 0
    for _, N, K, act, res in layer:
        tot += N * row_bytes(wtype, K) + M * K * 4 + M * N * 4 + N * 4 + (M * N * 4 if res else 0)
    return tot


def _capture(ctx, fn):
    ctx.graph_begin()
    try:
        fn()
    finally:
        g = ctx.graph_end()
    return g


RAMP_S = 0.25   # untimed clock ramp before the warmup steps, seconds


def ramp(ctx, run, seconds=RAMP_S):
    """Untimed: repeat the step over the buffer sets until `seconds` of wall time have passed,
    so the GPU clocks, TLBs and caches are in steady state when the warmup steps begin (ten
    warmup steps take under a millisecond; on one box the cfg2 step then measured 223-224
    against 233-234 TOPS after a long warmup)."""
    t0, i = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(32):
            run[i % len(run)]()
            i += 1
        ctx.sync()


def measure(ctx, M, wtype, steps, warmup, rotate_gb, use_graphs=True, path="packed", layer=LAYER):
    host = host_layer(M, wtype, layer=layer)
    set_bytes = sum(h["wq"].nbytes + h["x"].nbytes + h["bias"].nbytes + M * len(h["bias"]) * 4 * 2
                    + (h["resid"].nbytes if h["resid"] is not None else 0) + h["x"].nbytes // 2
                    for h in host)
    nsets = max(2, int(np.ceil(rotate_gb * 1e9 / set_bytes)))
    log(f"[bench] M={M} wtype={wtype}: {nsets} buffer sets x {set_bytes/1e6:.1f} MB")
    sets = [LayerSet(ctx, host, M, wtype, path, layer) for _ in range(nsets)]
    for s in sets:                      # first run outside any graph
        s.step()
    ctx.sync()
    if use_graphs:                      # one graph per buffer set: the step, and the GEMMs alone
        g_step = [_capture(ctx, s.step) for s in sets]
        g_gemm = [_capture(ctx, s.gemms_only) for s in sets]
        run_step = [g.launch for g in g_step]
        run_gemm = [g.launch for g in g_gemm]
    else:
        run_step = [s.step for s in sets]
        run_gemm = [s.gemms_only for s in sets]
    ramp(ctx, run_step)
    for i in range(warmup):
        run_step[i % nsets]()
    ctx.sync()
    ctx.timer_start()
    for i in range(steps):
        run_step[i % nsets]()
    ms_step = ctx.timer_stop() / steps
    # dominant kernel alone: the four GEMM launches per step, same rotation
    for i in range(min(warmup, nsets)):
        run_gemm[i]()
    ctx.sync()
    ctx.timer_start()
    for i in range(steps):
        run_gemm[i % nsets]()
    ms_gemms = ctx.timer_stop() / steps
    if use_graphs:
        for g in g_step + g_gemm:
            g.destroy()
    for s in sets:
        for d in s.g:
            for k in ("w", "x", "b", "r", "y", "qx", "dx", "sx"):
                if d[k] is not None:
                    ctx.free(d[k])
    return ms_step, ms_gemms, host


def write_synthetic_model(path, n_layer, wtype, seed=0, write=True):
    """Random-init MaskGIT transformer GGUF (the cfg4/cfg5 recipe): FC weights ~N(0,0.02)
    in Q8_0 / Q4_K blocks (bench-local encoders), embeddings ~N(0,0.02), biases ~N(0,0.01),
    LN gamma ~1+N(0,0.02), beta ~N(0,0.01); hidden 768, 16 heads, MLP 3072, vocab 2025."""
    from edge_maskgit_amd.gguf import GGML_F32, GGML_Q4_K, GGML_Q8_0, write_gguf
    rng = np.random.default_rng(seed)
    E, F, V, P = 768, 3072, 2025, 257
    enc, gt = (synth_q8_0, GGML_Q8_0) if wtype == ema.WTYPE_Q8_0 else (synth_q4_k, GGML_Q4_K)
    out = []

    def f32(name, a):
        out.append((name, a.shape, GGML_F32, np.ascontiguousarray(a, np.float32).tobytes()))

    def nrm(shape, s):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(s)).astype(np.float32)

    def fcw(name, n_out, n_in):
        w = nrm((n_out, n_in), 0.02)
        out.append((name, (n_out, n_in), gt, enc(w).tobytes()))

    f32("token_embd.weight", nrm((V, E), 0.02))
    f32("pos_embd.weight", nrm((P, E), 0.02))
    f32("token_embd_norm.weight", 1 + nrm(E, 0.02))
    f32("token_embd_norm.bias", nrm(E, 0.01))
    for l in range(n_layer):
        p = f"blk.{l}."
        for nm, no, ni in (("attn_q", E, E), ("attn_k", E, E), ("attn_v", E, E), ("attn_o", E, E),
                           ("ffn_up", F, E), ("ffn_down", E, F)):
            fcw(p + nm + ".weight", no, ni)
            f32(p + nm + ".bias", nrm(no, 0.01))
        for nm in ("attn_norm", "ffn_norm"):
            f32(p + nm + ".weight", 1 + nrm(E, 0.02))
            f32(p + nm + ".bias", nrm(E, 0.01))
    fcw("output_proj.weight", E, E)
    f32("output_proj.bias", nrm(E, 0.01))
    f32("output_norm.weight", 1 + nrm(E, 0.02))
    f32("output_norm.bias", nrm(E, 0.01))
    f32("output.bias", nrm(V, 0.01))
    meta = [("general.architecture", "str", "maskgit"), ("general.alignment", "u32", 32),
            ("maskgit.n_layer", "u32", n_layer), ("maskgit.n_head", "u32", 16),
            ("maskgit.n_embd", "u32", E), ("maskgit.n_ffn", "u32", F), ("maskgit.head_dim", "u32", 48),
            ("maskgit.vocab_size", "u32", V), ("maskgit.n_tokens", "u32", P - 1),
            ("maskgit.n_positions", "u32", P), ("maskgit.mask_token_id", "i32", V - 1),
            ("maskgit.layernorm_eps", "f32", 1e-12), ("maskgit.vqgan.codebook_size", "u32", 1024),
            ("maskgit.sampling.choice_temperature", "f32", 4.5)]
    if not write:
        return meta, out
    write_gguf(path, meta, out)


def synth_tokens(rng, B, S=257):
    """cfg4 token ids: position 0 = class token 1024 + U[0,999]; positions 1..256 codebook ids
    U[0,1023] with half replaced by the mask id 2024 (the reference's convention)."""
    t = rng.integers(0, 1024, (B, S)).astype(np.int32)
    t[:, 0] = 1024 + rng.integers(0, 1000, B)
    t[:, 1:][rng.random((B, S - 1)) < 0.5] = 2024
    return t


def measure_forward(path, B, steps, warmup, algo=1, profile=False):
    """Full transformer forward through the C++ HipRuntime (graph build + kernels + logits
    readback), wall clock per call; and the same without the logits readback."""
    from edge_maskgit_amd.runtime import TransformerRuntime
    rng = np.random.default_rng(1)
    tok = synth_tokens(rng, B)
    with TransformerRuntime(path, algo=algo) as m:
        for _ in range(max(1, warmup)):
            m.forward(tok)                       # first call packs and uploads the weights
        t0 = time.perf_counter()
        for _ in range(steps):
            m.forward(tok)
        ms = (time.perf_counter() - t0) / steps * 1e3
        t0 = time.perf_counter()
        for _ in range(steps):
            m.forward(tok, readback=False)
        ms_nr = (time.perf_counter() - t0) / steps * 1e3
        prof = None
        if profile:
            m.profile(True)
            m.forward(tok, readback=False)
            prof = {n: {"count": c, "ms": round(t, 3)} for n, c, t in m.profile_report()}
            m.profile(False)
    return ms, ms_nr, prof


def measure_generate(path, B, n_steps=8, reps=2, algo=1):
    """cfg5: B images, n_steps device-resident decode steps (transformer forward in HBM ->
    on-device sampling / confidence / re-mask), wall clock per generate; token grids only come
    back at the end."""
    from edge_maskgit_amd.runtime import TransformerRuntime
    cls = (np.arange(B) * 37) % 1000
    seeds = np.arange(B, dtype=np.uint64) + 42
    with TransformerRuntime(path, algo=algo) as m:
        m.generate(cls, seeds, n_steps)          # packs and uploads the weights
        t0 = time.perf_counter()
        for _ in range(reps):
            m.generate(cls, seeds, n_steps)
        return (time.perf_counter() - t0) / reps * 1e3


def measure_decode_step(ctx, B, S=257, V=2025, reps=20):
    """Device time of one mgh_decode_step (engine draws + sampling + re-mask) for B images on
    logits already in HBM."""
    rng = np.random.default_rng(2)
    logits = ctx.upload((rng.standard_normal((B, S, V)) * 2).astype(np.float32))
    tok = np.full((B, S), 2024, np.int32)
    tok[:, 0] = 1024
    d_tok, d_res = ctx.upload(tok), ctx.alloc(tok.nbytes)
    state, work = ctx.alloc(ema.decode_state_bytes(B)), ctx.alloc(ema.decode_work_bytes(B, S))
    ctx.decode_init(list(range(B)), state)
    ctx.decode_step(state, work, logits, B, S, V, 1024, 2024, 256, 0, 8, 4.5, d_tok, d_res)
    ctx.timer_start()
    for _ in range(reps):
        ctx.decode_step(state, work, logits, B, S, V, 1024, 2024, 256, 0, 8, 4.5, d_tok, d_res)
    ms = ctx.timer_stop() / reps
    for b in (logits, d_tok, d_res, state, work):
        ctx.free(b)
    return ms


# ---- VQGAN decoder (the production configuration of the reference's decoder graph) ----
VQ = dict(n_tokens=256, E=256, codebook=1024, filters=128, mult=(1, 1, 2, 2, 4), R=2)


def vqgan_convs(n_tokens, E, filters, mult, R, **_):
    """(side, IC, OC, k) of every convolution of build_vqgan_decoder, in graph order"""
    L = int(round(n_tokens ** 0.5))
    out, side, w = [], L, filters * mult[-1]
    out.append((side, E, w, 3))
    for _ in range(R):
        out += [(side, w, w, 3), (side, w, w, 3)]
    for i in range(len(mult) - 1, -1, -1):
        o = filters * mult[i]
        for _ in range(R):
            out += [(side, w, o, 3), (side, o, o, 3)] + ([(side, o, o, 1)] if w != o else [])
            w = o
        if i > 0:
            side *= 2
            out.append((side, w, w, 3))
    out.append((side, w, 3, 3))
    return out


def write_vqgan_model(path, seed=11, write=True):
    """random-init decoder weights under the converter's names (conv ~N(0, 1/fan_in), GroupNorm
    gamma ~1 + N(0, 0.1), beta / biases ~N(0, 0.1) / N(0, 0.05), codebook ~N(0, 1))"""
    from edge_maskgit_amd.gguf import write_gguf
    rng = np.random.default_rng(seed)
    E, F, mult, R = VQ["E"], VQ["filters"], VQ["mult"], VQ["R"]
    out = []

    def f32(name, a):
        out.append((name, a.shape, 0, np.ascontiguousarray(a, np.float32).tobytes()))

    def conv(name, oc, ic, k, bias):
        f32(name + ".weight", rng.standard_normal((oc, ic, k, k), np.float32) / np.float32(np.sqrt(ic * k * k)))
        if bias:
            f32(name + ".bias", 0.05 * rng.standard_normal(oc, np.float32))

    def gn(name, c):
        f32(name + ".weight", 1 + 0.1 * rng.standard_normal(c, np.float32))
        f32(name + ".bias", 0.1 * rng.standard_normal(c, np.float32))

    def block(p, ci, co):
        gn(p + "norm0", ci)
        conv(p + "conv0", co, ci, 3, False)
        gn(p + "norm1", co)
        conv(p + "conv1", co, co, 3, False)
        if ci != co:
            conv(p + "conv_res", co, co, 1, False)

    f32("vqgan.quantizer.codebook.weight", rng.standard_normal((VQ["codebook"], E), np.float32))
    w = F * mult[-1]
    conv("vqgan.decoder.conv_in", w, E, 3, True)
    for l in range(R):
        block(f"vqgan.decoder.res_blocks.0.{l}.", w, w)
    for i in range(len(mult) - 1, -1, -1):
        j, o = len(mult) - i, F * mult[i]
        for l in range(R):
            block(f"vqgan.decoder.res_blocks.{j}.{l}.", w, o)
            w = o
        if i > 0:
            conv(f"vqgan.decoder.res_blocks.{j}.{R + 1}", w, w, 3, True)
    gn("vqgan.decoder.norm_out", w)
    conv("vqgan.decoder.conv_out", 3, w, 3, True)
    meta = [("general.architecture", "str", "maskgit"), ("general.alignment", "u32", 32),
            ("maskgit.n_tokens", "u32", VQ["n_tokens"]), ("maskgit.resolution", "u32", 256),
            ("maskgit.vqgan.codebook_size", "u32", VQ["codebook"]), ("maskgit.vqgan.embedding_dim", "u32", E),
            ("maskgit.vqgan.filters", "u32", F), ("maskgit.vqgan.num_res_blocks", "u32", R),
            ("maskgit.vqgan.group_norm_groups", "u32", 32),
            ("maskgit.vqgan.channel_multipliers", "i32_array", list(mult))]
    if not write:
        return meta, out
    write_gguf(path, meta, out)


def write_maskgit_model(path, wtype, seed=5):
    """transformer (24 layers) and VQGAN decoder in one GGUF, as a converted model holds them"""
    from edge_maskgit_amd.gguf import write_gguf
    mt, tt = write_synthetic_model(path, 24, wtype, seed=seed, write=False)
    mv, tv = write_vqgan_model(path, write=False)
    keys = {k for k, _, _ in mt}
    write_gguf(path, mt + [e for e in mv if e[0] not in keys], tt + tv)


def measure_generate_images(path, B, n_steps=8, reps=2, algo=2):
    """generate() end to end: B images, n_steps device-resident decode steps, then the VQGAN
    decode of the grids (mgr_generate_images); wall clock per call, images read back"""
    from edge_maskgit_amd.runtime import TransformerRuntime
    cls = (np.arange(B) * 37) % 1000
    seeds = np.arange(B, dtype=np.uint64) + 42
    with TransformerRuntime(path, algo=algo) as m:
        m.generate_images(cls, seeds, n_steps)          # packs and uploads the weights
        t0 = time.perf_counter()
        for _ in range(reps):
            m.generate_images(cls, seeds, n_steps)
        return (time.perf_counter() - t0) / reps * 1e3


def measure_vqgan(path, steps=5, cpu=True, int8=True):
    """The production decoder graph (mgr_decode_images: mg::build_vqgan_decoder on HipRuntime)
    for one image and for a batch of 8: wall clock per decode (ids in, image left in HBM), the
    per-op device profile of one B=1 decode, and the conv kernels' fp32-MFMA roofline."""
    from edge_maskgit_amd.runtime import TransformerRuntime
    convs = vqgan_convs(**VQ)
    conv_flop = sum(2.0 * s * s * ic * oc * k * k for s, ic, oc, k in convs)
    res = {"model": "VQGAN decoder, 256 tokens -> 256 x 256 x 3, 128 filters, multipliers 1,1,2,2,4, "
                    "2 res blocks per level, GroupNorm 32 (random-init weights)",
           "conv_gflop_per_image": round(conv_flop / 1e9, 2)}
    rng = np.random.default_rng(3)
    with TransformerRuntime(path) as m:
        for B in (1, 8):
            g = rng.integers(0, VQ["codebook"], (B, VQ["n_tokens"])).astype(np.int32)
            for _ in range(2):
                m.decode_images(g, readback=False)       # the first call packs and uploads weights
            t0 = time.perf_counter()
            for _ in range(steps):
                m.decode_images(g, readback=False)
            ms = (time.perf_counter() - t0) / steps * 1e3
            res[f"b{B}"] = {"ms_per_decode": round(ms, 3), "ms_per_image": round(ms / B, 3),
                            "tflops": round(conv_flop * B / (ms * 1e-3) / 1e12, 2)}
        m.profile(True)
        m.decode_images(rng.integers(0, VQ["codebook"], (1, VQ["n_tokens"])).astype(np.int32), readback=False)
        prof = {n: {"count": c, "ms": round(t, 4)} for n, c, t in m.profile_report()}
        m.profile(False)
    if int8:
        # the reference's int8 conv (its default on integer-dot devices) under the int8 algorithm
        with TransformerRuntime(path, algo=1) as m:
            for B in (1, 8):
                g = rng.integers(0, VQ["codebook"], (B, VQ["n_tokens"])).astype(np.int32)
                for _ in range(2):
                    m.decode_images(g, readback=False)
                t0 = time.perf_counter()
                for _ in range(steps):
                    m.decode_images(g, readback=False)
                ms = (time.perf_counter() - t0) / steps * 1e3
                res.setdefault("int8_conv", {})[f"b{B}"] = {"ms_per_decode": round(ms, 3),
                                                            "ms_per_image": round(ms / B, 3),
                                                            "tops": round(conv_flop * B / (ms * 1e-3) / 1e12, 2)}
    res["per_op_device_ms_b1"] = prof
    conv_ms = prof.get("Conv2D", {}).get("ms")
    if conv_ms:
        a = conv_flop / (conv_ms * 1e-3) / 1e12
        res["roofline_conv_b1"] = {"bound": "mfma", "achieved": round(a, 2), "peak": 157.3, "unit": "TFLOP/s",
                                   "frac": round(a / 157.3, 4), "kernel": "k_conv2d_pk (+ _pkn, split reduce)",
                                   "note": "fp32 MFMA (the reference's conv arithmetic is fp32); all Conv2D "
                                           "nodes of one decode, device time per node"}
    if cpu:
        from oracle import ref
        if ref.available():
            xs = [(16, 256, 512), (16, 512, 512)]
            fl, t0 = 0.0, time.perf_counter()
            for side, ic, oc in xs:
                x = rng.standard_normal((1, ic, side, side), np.float32)
                k = rng.standard_normal((oc, ic, 3, 3), np.float32) * np.float32(0.02)
                ref.conv2d(x, k, 1, 1)
                fl += 2.0 * side * side * ic * oc * 9
            dt = time.perf_counter() - t0
            res["cpu_baseline"] = {"value": round(fl / dt / 1e9, 3), "unit": "GFLOP/s", "cores": 1,
                                   "kind": "reference",
                                   "sample": f"reference mg-cpu k_conv_2d on the decoder's two 16x16 3x3 convs "
                                             f"(256->512, 512->512: {fl/1e9:.2f} GFLOP in {dt:.1f} s); "
                                             f"a whole decode at this rate: {conv_flop / (fl / dt) :.0f} s"}
    return res


def host_cpu():
    """nproc, the CPU model name and OMP_NUM_THREADS of the host the CPU baseline runs on"""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model, "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cpu_baseline(host, M, wtype, budget_s=15.0):
    """The reference CPU executor (libmgref) on dequantized weights, single thread, over the
    same four GEMMs; rows are processed in chunks until the budget is spent."""
    import oracle
    from oracle import ref
    if ref.available():
        ops = 0.0
        t0 = time.perf_counter()
        rows_done = 0
        chunk = 64
        wdeq = [oracle.dequant(wtype, h["wq"], h["wq"].shape[0], h["x"].shape[1]) for h in host]
        while rows_done < M and time.perf_counter() - t0 < budget_s:
            r0, r1 = rows_done, min(M, rows_done + chunk)
            for (name, N, K, act, res), h, w in zip(LAYER, host, wdeq):
                ref.mul_mat(w, h["x"][r0:r1], bias=h["bias"], act=act,
                            resid=None if h["resid"] is None else h["resid"][r0:r1])
                ops += 2.0 * (r1 - r0) * N * K
            rows_done = r1
        dt = time.perf_counter() - t0
        return {"value": round(ops / dt / 1e12, 6), "unit": "TOPS", "cores": 1, "kind": "reference", **host_cpu(),
                "sample": f"reference mg-cpu k_mul_mat (F32, dequantized Q8_0 weights), the same four "
                          f"GEMMs on rows 0..{rows_done - 1} of M={M} ({ops/1e9:.2f} Gop in {dt:.1f} s)"}
    return cpu_oracle_int8(host, M, wtype)


def cpu_oracle_int8(host, M, wtype, rows=None):
    """The C oracle's int8-dot path (the reference's int8 kernel semantics, OpenMP over all
    host threads, scalar C) over the same four GEMMs (all rows unless a sample is given)."""
    import oracle
    rows = M if rows is None else rows
    nth = int(os.environ.get("OMP_NUM_THREADS", 0)) or os.cpu_count() or 1
    ops = 0.0
    t0 = time.perf_counter()
    for (name, N, K, act, res), h in zip(LAYER, host):
        qx, dx, _ = oracle.quantize_act_q8(h["x"][:rows])
        oracle.gemm_q_i8(wtype, h["wq"], N, K, qx, dx, bias=h["bias"], act=act)
        ops += 2.0 * rows * N * K
    dt = time.perf_counter() - t0
    return {"value": round(ops / dt / 1e12, 6), "unit": "TOPS", "cores": nth, "kind": "port", **host_cpu(),
            "sample": f"C oracle int8-dot path (OpenMP), four GEMMs on {rows} of {M} rows ({ops/1e9:.2f} Gop in {dt:.1f} s)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--rotate-gb", type=float, default=3.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--graphs", action="store_true",
                    help="replay a captured HIP graph per step instead of enqueuing the kernels one by one")
    ap.add_argument("--path", choices=["packed", "h16", "raw", "dq"], default="dq",
                    help="packed: int8-dot path on the device-native weight layout; h16: "
                         "dequantize-fused fp16 path; raw: int8-dot on GGUF blocks as stored")
    ap.add_argument("--no-fwd", action="store_true", help="skip the transformer forward (cfg4)")
    ap.add_argument("--only-config", choices=["cfg1", "m4097", "q4k_m1025", "q4k_m4097"], default=None,
                    help="measure only this workload of --path (cfg1: one Q8_0 FC at M=257; m4097: "
                         "the four Q8_0 FCs at M=4097) and print its timing: the run a kernel "
                         "profile of that workload wraps")
    ap.add_argument("--only-main", action="store_true",
                    help="measure only the cfg2 step of --path (no other path, no cfg1, no forward, "
                         "no CPU baseline): the run a kernel profile wraps")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run 10 plain device copies of BYTES (k_copy4d), to calibrate the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters, and exit")
    ap.add_argument("--no-vqgan", action="store_true", help="skip the VQGAN decoder measurement")
    ap.add_argument("--only-vqgan", action="store_true",
                    help="measure only the VQGAN decoder and print its record: the run a kernel profile wraps")
    ap.add_argument("--extra", action="store_true",
                    help="also measure the cfg5 forward (Q4_K, 64 images) and the 64-image generate loop")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {a.gpus}); "
              "the path shards by data parallelism over images with no per-layer exchange, "
              "but multi-GPU runs are not part of this build.", file=sys.stderr)
        sys.exit(2)

    ctx = ema.Context(0)
    log(f"[bench] device: {ctx.device_name}")
    if a.copy_probe:
        n = a.copy_probe // 4
        src, dst = ctx.alloc(n * 4), ctx.alloc(n * 4)
        ctx.fill_u32(src, 0x3F800000, n)
        for _ in range(10):
            ctx.copy_strided(src, (n, 1, 1, 1), (1, n, n, n), dst)
        ctx.sync()
        print(json.dumps({"copy_probe_bytes": n * 4, "launches": 10}), flush=True)
        ctx.close()
        return
    if a.only_vqgan:
        import tempfile
        with tempfile.TemporaryDirectory() as d:
            pv = os.path.join(d, "vqgan.gguf")
            write_vqgan_model(pv)
            print(json.dumps({"vqgan_decode": measure_vqgan(pv, a.steps, cpu=not a.no_cpu)}), flush=True)
        ctx.close()
        return
    if a.only_config:
        M1, lay = (257, CFG1) if a.only_config == "cfg1" else (1025 if "m1025" in a.only_config else 4097, LAYER)
        wt1 = ema.WTYPE_Q4_K if a.only_config.startswith("q4k") else ema.WTYPE_Q8_0
        s1, g1, _ = measure(ctx, M1, wt1, a.steps, a.warmup, a.rotate_gb, use_graphs=a.graphs,
                            path=a.path, layer=lay)
        ab = step_alg_bytes(M1, wt1, lay)
        print(json.dumps({"config": a.only_config, "path": PATH_NAME[a.path], "M": M1, "ms_per_step": round(s1, 5),
                          "tops": round(layer_ops(M1, lay) / (s1 * 1e-3) / 1e12, 2),
                          "alg_bytes_per_step": ab, "alg_gbs": round(ab / (s1 * 1e-3) / 1e9, 1)}), flush=True)
        ctx.close()
        return
    M, wtype = 1025, ema.WTYPE_Q8_0
    ms_step, ms_gemms, host = measure(ctx, M, wtype, a.steps, a.warmup, a.rotate_gb,
                                      use_graphs=a.graphs, path=a.path)
    ops = layer_ops(M)
    value = ops / (ms_step * 1e-3) / 1e12
    gb = gemm_alg_bytes(M, wtype, a.path)
    achieved = gb / (ms_gemms * 1e-3) / 1e9
    extra = {"gemm_only_ms_per_step": round(ms_gemms, 5),
             "gemm_tops": round(ops / (ms_gemms * 1e-3) / 1e12, 2),
             "step_alg_bytes": step_alg_bytes(M, wtype),
             "step_hbm_roofline_us": round(step_alg_bytes(M, wtype) / (HBM_PEAK_GBS * 1e9) * 1e6, 2),
             "step_frac_of_hbm_roofline": round(step_alg_bytes(M, wtype) / (HBM_PEAK_GBS * 1e9)
                                                / (ms_step * 1e-3), 4)}
    if a.only_main:
        a.no_fwd, a.no_cpu = True, True
    else:
        # the same step with warm caches: two buffer sets, so weights and activations stay in
        # the MALL (and largely in the L2s) between steps; reported beside the cold headline
        hs, hg, _ = measure(ctx, M, wtype, a.steps, a.warmup, 0.0, use_graphs=a.graphs, path=a.path)
        extra["cfg2_hot_cache"] = {"ms_per_step": round(hs, 5), "tops": round(ops / (hs * 1e-3) / 1e12, 2),
                                   "buffer_sets": 2}
        # every path on every GEMM workload of the metric (configs[1], [2]): Q8_0 at M = 1025 and
        # 4097, Q4_K at M = 1025 and 4097; per path the step time, TOPS and the fraction of the
        # HBM roofline on the metric's algorithmic bytes (quantized weights once, fp32 activations
        # and outputs once), plus the bytes the path's kernels actually read per weight
        paths = [p for p in ("dq", "h16", "packed", "raw") if p != a.path]
        for (mm, wt) in ((1025, ema.WTYPE_Q8_0), (4097, ema.WTYPE_Q8_0), (1025, ema.WTYPE_Q4_K),
                         (4097, ema.WTYPE_Q4_K)):
            key = f"{'q8_0' if wt == ema.WTYPE_Q8_0 else 'q4_k'}_m{mm}"
            ab = step_alg_bytes(mm, wt)
            ent = {"alg_bytes_per_step": ab,
                   "hbm_roofline_us": round(ab / (HBM_PEAK_GBS * 1e9) * 1e6, 2)}
            for pth in ([a.path] if (mm, wt) != (M, wtype) else []) + paths:
                if wt == ema.WTYPE_Q4_K and pth == "raw" and mm > 1025:
                    continue
                st = max(10, a.steps // 2) if mm > 1025 else a.steps
                sm, sg, _ = measure(ctx, mm, wt, st, a.warmup, a.rotate_gb, use_graphs=a.graphs, path=pth)
                ent[PATH_NAME[pth]] = {
                    "kernel": KERNEL[pth], "weight_bytes_read": WEIGHT_BYTES[pth][wt],
                    "ms_per_step": round(sm, 5), "tops": round(layer_ops(mm) / (sm * 1e-3) / 1e12, 2),
                    "gemm_tops": round(layer_ops(mm) / (sg * 1e-3) / 1e12, 2),
                    "frac_of_hbm_roofline": round(ab / (HBM_PEAK_GBS * 1e9) / (sm * 1e-3), 4)}
            if (mm, wt) == (M, wtype):
                ent[PATH_NAME[a.path]] = {"kernel": KERNEL[a.path], "weight_bytes_read": WEIGHT_BYTES[a.path][wt],
                                          "ms_per_step": round(ms_step, 5), "tops": round(value, 2),
                                          "gemm_tops": round(ops / (ms_gemms * 1e-3) / 1e12, 2),
                                          "frac_of_hbm_roofline": extra["step_frac_of_hbm_roofline"],
                                          "note": "the headline measurement"}
            extra[key] = ent
        # the single Q8_0 FC GEMM at M=257 (weight-streaming shape), every path
        extra["cfg1_m257"] = {}
        ab1 = step_alg_bytes(257, wtype, CFG1)
        for pth in (a.path, "h16", "packed", "raw"):
            if PATH_NAME[pth] in extra["cfg1_m257"]:
                continue
            s1, _, _ = measure(ctx, 257, wtype, a.steps, a.warmup, a.rotate_gb, use_graphs=a.graphs,
                               path=pth, layer=CFG1)
            extra["cfg1_m257"][PATH_NAME[pth]] = {
                "us": round(s1 * 1e3, 2), "tops": round(layer_ops(257, CFG1) / (s1 * 1e-3) / 1e12, 2),
                "alg_gbs": round(ab1 / (s1 * 1e-3) / 1e9, 1),
                "frac_of_hbm_roofline": round(ab1 / (HBM_PEAK_GBS * 1e9) / (s1 * 1e-3), 4)}
        extra["cfg1_m257"]["alg_bytes"] = ab1
    if not a.no_fwd:
        import tempfile
        with tempfile.TemporaryDirectory() as d:
            path = os.path.join(d, "cfg4_q8_0.gguf")
            t0 = time.perf_counter()
            write_synthetic_model(path, 24, ema.WTYPE_Q8_0)
            log(f"[bench] cfg4 model written in {time.perf_counter() - t0:.1f} s")
            fwd4 = {}
            for pth in (a.path, "h16", "packed"):
                if PATH_NAME[pth] in fwd4:
                    continue
                fwd, fwd_nr, prof = measure_forward(path, 16, max(3, a.steps // 10), 2, algo=ALGO[pth],
                                                    profile=True)
                fwd4[PATH_NAME[pth]] = {"ms": round(fwd, 3), "ms_no_logits_readback": round(fwd_nr, 3),
                                        "per_op_device_ms": prof}
            extra["transformer_fwd_cfg4"] = {
                "model": "24 layers Q8_0 random-init, hidden 768, 16 heads, MLP 3072, vocab 2025",
                "batch": "16 images x 257 tokens (M=4112)", **fwd4}
            # the same model on one image (M = 257): latency-bound kernels, the single-image call
            f1, f1nr, _ = measure_forward(path, 1, 20, 5, algo=ALGO[a.path])
            extra["transformer_fwd_b1"] = {"path": PATH_NAME[a.path], "batch": "1 image x 257 tokens (M=257)",
                                           "ms": round(f1, 3), "ms_no_logits_readback": round(f1nr, 3)}
            if a.extra:
                path5 = os.path.join(d, "cfg5_q4_k.gguf")
                write_synthetic_model(path5, 24, ema.WTYPE_Q4_K, seed=5)
                f5, f5nr, _ = measure_forward(path5, 64, 3, 1, algo=ALGO[a.path])
                extra["transformer_fwd_q4k_b64"] = {"ms": round(f5, 3), "ms_no_logits_readback": round(f5nr, 3),
                                                    "batch": "64 x 257 tokens (M=16448), one decode step's forward"}
                gen = measure_generate(path5, 64, algo=ALGO[a.path])
                extra["generate_cfg5"] = {
                    "ms_per_generate": round(gen, 2), "ms_per_step": round(gen / 8, 3),
                    "decode_step_device_ms": round(measure_decode_step(ctx, 64), 4),
                    "workload": f"64 images x 257 tokens, 8 steps, Q4_K 24 layers, {PATH_NAME[a.path]}; "
                                "forward + on-device sampling per step, grids read back once"}
    if not a.no_vqgan and not a.only_main:
        import tempfile
        with tempfile.TemporaryDirectory() as d:
            pv = os.path.join(d, "vqgan.gguf")
            t0 = time.perf_counter()
            write_vqgan_model(pv)
            log(f"[bench] VQGAN model written in {time.perf_counter() - t0:.1f} s")
            extra["vqgan_decode"] = measure_vqgan(pv, cpu=not a.no_cpu)
            os.remove(pv)
            pm = os.path.join(d, "maskgit_q4_k.gguf")
            write_maskgit_model(pm, ema.WTYPE_Q4_K)
            e2e = {}
            for B in (1, 8):
                ms = measure_generate_images(pm, B)
                e2e[f"b{B}"] = {"ms_per_call": round(ms, 2), "ms_per_image": round(ms / B, 2)}
            extra["generate_images"] = {
                "workload": "generate() end to end: 24-layer Q4_K transformer (random-init), 8 decode steps "
                            "on the device, then the production VQGAN decoder; images read back",
                "path": "dequantize-fused fp16 FC, fp32 conv", **e2e}
    cpu = None if a.no_cpu else cpu_baseline(host, M, wtype)
    if not a.no_cpu and cpu is not None and cpu.get("kind") == "reference":
        extra["cpu_oracle_int8_omp"] = cpu_oracle_int8(host, M, wtype)   # a multi-core CPU point
    digest = csrc_digest()
    traffic, traffic_src = measured_traffic(
        os.path.join(ROOT, "profiles", f"traffic_{TRAFFIC_FILE[a.path]}_cfg2_q8_m1025.json"), digest)
    line = {
        "metric": "Q8_0/Q4_K GEMM TOPS + % roofline at M=1025/4097; transformer fwd ms",
        "value": round(value, 3),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if a.path in ("h16", "dq") else "int8",
        "data": "synthetic",
        "config": {"workload": "cfg2: one MaskGIT layer's four Q8_0 FC GEMMs (QKV 768->2304, "
                               "out 768->768 +resid, up 768->3072 +GELU, down 3072->768 +resid), "
                               "M=1025, fp32 activations and outputs, " + WORKLOAD_PATH[a.path],
                   "path": PATH_NAME[a.path],
                   "M": M, "weights": "Q8_0", "rotate_gb": a.rotate_gb,
                   "launch": "hip_graph_per_step" if a.graphs else "stream",
                   "csrc_sha256_16": digest},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": KERNEL[a.path], "bytes_per_step": gb, "traffic_source": traffic_src},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
