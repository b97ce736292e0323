"""The VQGAN decoder restated in numpy (TEST INFRASTRUCTURE ONLY: tests and smoke() import it,
the shipped GPU path never does).

Arrays are numpy [N][C][H][W] (the reference's ne = {W, H, C, N}); conv kernels
[OC][IC][KH][KW] (ne = {KW, KH, IC, OC}).

  conv2d       k_conv_2d (src/mg-cpu/mg-cpu.cpp:165-190): zero padding, stride; products
               summed in float64 and rounded once (the reference sums in float32 in
               (ic, kh, kw) order, so the two differ by at most the float32 summation error)
  group_norm   k_group_norm (mg-cpu.cpp:123-147): per (n, group) mean and variance in float64
               (two passes), inv = 1 / sqrt(float32(var) + eps) in float32,
               y = float32(x - mean) * inv; with gamma/beta the fused node's affine + SiLU
               (mg-cpu.cpp:262-276): xn = y * gamma + beta (two roundings), xn / (1 + exp(-xn))
  upscale      k_upscale (mg-cpu.cpp:192-198): nearest neighbour
  decode       build_vqgan_decoder (src/mg-vqgan.cpp:62-110) composed from the above (or with
               the int8 conv of oracle.conv2d_i8, mg-opencl.cpp:598-664)

Parity pins (tests/test_oracle_vqgan.py): each primitive against the reference's own CPU
executor (oracle/_ref/libmgref.so) and against closed forms (a delta kernel shifts the image,
a 1x1 conv is a channel matmul, GroupNorm output has zero mean and unit variance per group,
upscale by 1 is the identity); decode against the reference decoder graph run by libmgref.
"""
from __future__ import annotations

import numpy as np

GROUPS = 32          # mg-vqgan.cpp:14-15
EPS = 1e-5


def conv2d(x, ker, stride=1, pad=0):
    x = np.asarray(x, np.float32)
    ker = np.asarray(ker, np.float32)
    N, IC, IH, IW = x.shape
    OC, KIC, KH, KW = ker.shape
    if KIC != IC:
        raise ValueError("kernel and input channel counts differ")
    OH, OW = (IH + 2 * pad - KH) // stride + 1, (IW + 2 * pad - KW) // stride + 1
    xp = np.zeros((N, IC, IH + 2 * pad, IW + 2 * pad), np.float64)
    xp[:, :, pad:pad + IH, pad:pad + IW] = x
    y = np.zeros((N, OC, OH, OW), np.float64)
    w = ker.astype(np.float64)
    for kh in range(KH):
        for kw in range(KW):
            patch = xp[:, :, kh:kh + stride * (OH - 1) + 1:stride, kw:kw + stride * (OW - 1) + 1:stride]
            y += np.einsum("nchw,oc->nohw", patch, w[:, :, kh, kw], optimize=True)
    return y.astype(np.float32)


def group_norm(x, groups=GROUPS, eps=EPS, gamma=None, beta=None):
    x = np.asarray(x, np.float32)
    N, C, H, W = x.shape
    xg = x.reshape(N, groups, -1).astype(np.float64)
    mean = xg.mean(axis=2, keepdims=True)
    var = ((xg - mean) ** 2).mean(axis=2, keepdims=True)
    inv = np.float32(1.0) / np.sqrt(var.astype(np.float32) + np.float32(eps))
    y = ((xg - mean).astype(np.float32) * inv).reshape(N, C, H, W)
    if gamma is not None:
        g = np.asarray(gamma, np.float32)[None, :, None, None]
        b = np.asarray(beta, np.float32)[None, :, None, None]
        xn = (y * g).astype(np.float32) + b
        y = xn / (np.float32(1.0) + np.exp(-xn))
    return y.astype(np.float32)


def upscale(x, f):
    return np.asarray(x, np.float32).repeat(f, axis=2).repeat(f, axis=3)


def decode(t: dict, grid, E: int, filters: int, mult, R: int, int8: bool = False):
    """t: float tensors by GGUF name (numpy shapes); grid int [B][n_tokens] -> [B][3][side][side].
    int8: every conv is the reference's int8 conv (k_conv2d_i8 on k_quantize_conv_w weights,
    restated by oracle.conv2d_i8), as its runtime runs them on integer-dot devices."""
    grid = np.asarray(grid).reshape(len(grid), -1)
    B, n = grid.shape
    L = int(round(n ** 0.5))
    f = t["vqgan.quantizer.codebook.weight"][grid]                     # [B][n][E]
    x = f.reshape(B, L, L, E).transpose(0, 3, 1, 2).astype(np.float32)   # [B][E][h][w]

    def conv(p, x, pad, bias):
        w = t[p + ".weight"]
        if int8:
            from . import conv2d_i8, conv_quant_w
            qw, dw = conv_quant_w(w)
            y = conv2d_i8(x, qw, dw, w.shape[2], w.shape[3], 1, pad)
        else:
            y = conv2d(x, w, 1, pad)
        return y + t[p + ".bias"][None, :, None, None] if bias else y

    def gn_silu(p, x):
        return group_norm(x, GROUPS, EPS, t[p + ".weight"], t[p + ".bias"])

    def block(p, x, cin, cout):
        h = conv(p + "conv0", gn_silu(p + "norm0", x), 1, False)
        h = conv(p + "conv1", gn_silu(p + "norm1", h), 1, False)
        return h + (x if cin == cout else conv(p + "conv_res", h, 0, False))

    x = conv("vqgan.decoder.conv_in", x, 1, True)
    width = filters * mult[-1]
    for l in range(R):
        x = block(f"vqgan.decoder.res_blocks.0.{l}.", x, width, width)
    for i in range(len(mult) - 1, -1, -1):
        j, out = len(mult) - i, filters * mult[i]
        for l in range(R):
            x = block(f"vqgan.decoder.res_blocks.{j}.{l}.", x, width, out)
            width = out
        if i > 0:
            x = conv(f"vqgan.decoder.res_blocks.{j}.{R + 1}", upscale(x, 2), 1, True)
    return conv("vqgan.decoder.conv_out", gn_silu("vqgan.decoder.norm_out", x), 1, True)
