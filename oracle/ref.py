"""Wrapper for oracle/_ref/libmgref.so — TEST INFRASTRUCTURE ONLY.

libmgref.so is the reference's own F32 CPU executor (mg-tensor.cpp + mg-cpu.cpp +
mg-model.cpp + mg-transformer.cpp, compiled from the reference tree by
``make -C oracle ref`` with oracle/ref_harness.cpp as the C entry layer). It exists only
where that build ran; ``available()`` says whether it did.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_ref", "libmgref.so")
_lib = None


def available() -> bool:
    return os.path.exists(_LIB_PATH)


def lib():
    global _lib
    if _lib is None:
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        L.mgref_last_error.restype = ctypes.c_char_p
        L.mgref_mul_mat.argtypes = [P, I64, I64, P, I64, P, ctypes.c_int, P, P]
        L.mgref_norm_affine.argtypes = [P, I64, I64, P, P, ctypes.c_float, P]
        L.mgref_attention.argtypes = [P, P, P, I64, I64, I64, I64, ctypes.c_float, P]
        L.mgref_transformer_forward.argtypes = [ctypes.c_char_p, P, I64, I64, P, I64]
        L.mgref_generate.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_int,
                                     ctypes.c_float, P, P, P]
        L.mgref_conv2d.argtypes = [P, I64, I64, I64, I64, P, I64, I64, I64, ctypes.c_int, ctypes.c_int, P, I64]
        L.mgref_group_norm.argtypes = [P, I64, I64, I64, I64, ctypes.c_int, ctypes.c_float, P, P, P]
        L.mgref_upscale.argtypes = [P, I64, I64, I64, I64, ctypes.c_int, P]
        L.mgref_vqgan_decode.argtypes = [ctypes.c_char_p, P, I64, P, I64, I64]
        L.mgref_vqgan_graph_sig.argtypes = [ctypes.c_char_p, I64, I64, ctypes.c_char_p, I64]
        L.mgref_vqgan_graph_sig.restype = I64
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _check(rc):
    if rc != 0:
        raise RuntimeError("libmgref: " + lib().mgref_last_error().decode())


def mul_mat(w, x, bias=None, act=0, resid=None):
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    N, K = w.shape
    M = x.shape[0]
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    resid = None if resid is None else np.ascontiguousarray(resid, np.float32)
    y = np.empty((M, N), np.float32)
    _check(lib().mgref_mul_mat(_p(w), N, K, _p(x), M, _p(bias), act, _p(resid), _p(y)))
    return y


def norm_affine(x, gamma, beta, eps):
    x = np.ascontiguousarray(x, np.float32)
    D = x.shape[-1]
    y = np.empty_like(x)
    _check(lib().mgref_norm_affine(_p(x), x.size // D, D, _p(np.ascontiguousarray(gamma, np.float32)),
                                   _p(np.ascontiguousarray(beta, np.float32)), eps, _p(y)))
    return y


def attention(q, k, v, D, S, H, B, scale):
    """q/k/v are [B][S][H*D] linear outputs; returns contiguous {D,S,H,B}."""
    q, k, v = (np.ascontiguousarray(a, np.float32) for a in (q, k, v))
    o = np.empty(D * S * H * B, np.float32)
    _check(lib().mgref_attention(_p(q), _p(k), _p(v), D, S, H, B, scale, _p(o)))
    return o


def transformer_forward(gguf_path: str, tokens, vocab: int):
    tokens = np.ascontiguousarray(tokens, np.int32)
    B, S = tokens.shape
    out = np.empty((B, S, vocab), np.float32)
    _check(lib().mgref_transformer_forward(gguf_path.encode(), _p(tokens), S, B, _p(out), out.size))
    return out


def generate(gguf_path: str, class_id: int, seed: int, steps: int, temperature: float, logits):
    """The reference's generate() loop with the caller's logits per step ([steps][S][vocab]):
    returns (tokens fed to each step's forward [steps][S], final grid [S-1])."""
    logits = np.ascontiguousarray(logits, np.float32)
    S = logits.shape[1]
    toks = np.empty((steps, S), np.int32)
    grid = np.empty(S - 1, np.int32)
    _check(lib().mgref_generate(gguf_path.encode(), class_id, seed, steps, temperature, _p(logits),
                                _p(toks), _p(grid)))
    return toks, grid


# ---- VQGAN decoder ops and graph (layout {W, H, C, N}; numpy arrays [N][C][H][W]) ----
def conv2d(x, ker, stride, pad):
    """x [N][IC][IH][IW], ker [OC][IC][KH][KW] -> [N][OC][OH][OW] (k_conv_2d, mg-cpu.cpp:165-190)"""
    x = np.ascontiguousarray(x, np.float32)
    ker = np.ascontiguousarray(ker, np.float32)
    N, IC, IH, IW = x.shape
    OC, _, KH, KW = ker.shape
    OH, OW = (IH + 2 * pad - KH) // stride + 1, (IW + 2 * pad - KW) // stride + 1
    y = np.empty((N, OC, OH, OW), np.float32)
    _check(lib().mgref_conv2d(_p(x), IW, IH, IC, N, _p(ker), KW, KH, OC, stride, pad, _p(y), y.size))
    return y


def group_norm(x, groups, eps, gamma=None, beta=None):
    """x [N][C][H][W]; with gamma/beta: the fused affine + SiLU node"""
    x = np.ascontiguousarray(x, np.float32)
    N, C, H, W = x.shape
    g = None if gamma is None else np.ascontiguousarray(gamma, np.float32)
    b = None if beta is None else np.ascontiguousarray(beta, np.float32)
    y = np.empty_like(x)
    _check(lib().mgref_group_norm(_p(x), W, H, C, N, groups, eps, _p(g), _p(b), _p(y)))
    return y


def upscale(x, f):
    x = np.ascontiguousarray(x, np.float32)
    N, C, H, W = x.shape
    y = np.empty((N, C, H * f, W * f), np.float32)
    _check(lib().mgref_upscale(_p(x), W, H, C, N, f, _p(y)))
    return y


def vqgan_decode(gguf_path: str, grid, side: int, arena_bytes: int = 1 << 30):
    """the reference's decoder graph on its CPU executor: grid [n_tokens] -> image [3][side][side]"""
    grid = np.ascontiguousarray(grid, np.int32).reshape(-1)
    img = np.empty((3, side, side), np.float32)
    _check(lib().mgref_vqgan_decode(gguf_path.encode(), _p(grid), grid.size, _p(img), img.size, arena_bytes))
    return img


def vqgan_graph_sig(gguf_path: str, n_tokens: int, arena_bytes: int = 1 << 30) -> str:
    n = lib().mgref_vqgan_graph_sig(gguf_path.encode(), n_tokens, arena_bytes, None, 0)
    if n < 0:
        _check(-1)
    buf = ctypes.create_string_buffer(n + 1)
    lib().mgref_vqgan_graph_sig(gguf_path.encode(), n_tokens, arena_bytes, buf, n + 1)
    return buf.value.decode()
