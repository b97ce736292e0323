"""CPU oracle for the edge_maskgit hot path — TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it.
The shipped GPU path (``edge_maskgit_amd``) never imports, loads or falls back to it.

``libmgoracle.so`` (built from ``mg_oracle.c`` by ``oracle/Makefile``) restates the
reference algorithms; each C function cites the reference file:line it follows.
``oracle.ref`` wraps ``_ref/libmgref.so``, the reference's own CPU executor compiled
from its sources, when that build exists.

Parity pins (what checks each function; see tests/test_oracle.py):
  f16 conversion      exhaustive vs numpy float16 (IEEE RNE)
  quantize_q8_0/q4_k  golden bytes written by the reference encoder (tests/golden/)
  dequant             closed forms + round-trip error bounds + golden decode
  quantize_act_q8     closed form, half-away-from-zero ties, zero blocks, brute force
  block_dots          exact integer brute force (numpy int64)
  gemm_q_i8           float64 recomputation from block dots; Q8_0 == Q4_K algebra check
  gemm_f32            reference CPU executor (libmgref) bit-exact
  layernorm_affine    reference CPU executor bit-exact
  attention           reference CPU executor (f32); f16kv = f32 path on rounded inputs
  conv_quant_w,       exact-representation closed form (conv2d_i8 equals the reference CPU
  conv2d_i8           fp32 conv bit for bit when every block quantizes exactly), power-of-two
                      scale equivariance, an independently structured numpy restatement of the
                      block grouping, and the int8 error bound against the fp32 conv
                      (tests/test_oracle_vqgan.py)
  mt64_draws          the C++ standard's known answer (10000th output of seed 5489)
  uniform_draws       generate_canonical closed form over the engine's raw outputs
  decode_step         closed forms on uniform logits (categorical index = ceil(1024 u) - 1,
                      re-masked set = smallest Gumbel draws), argmax limit, temperature-0
                      ordering by probability, cosine-schedule counts, known-token rules
                      (tests/test_oracle_decode.py)
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libmgoracle.so")

WTYPE_F32 = 0
WTYPE_Q8_0 = 8
WTYPE_Q4_K = 12

_lib = None


def build() -> None:
    """Compile the C restatement (and, where the reference tree exists, libmgref)."""
    import subprocess
    subprocess.check_call(["make", "-s", "-B", "-C", _HERE, "all"])
    if os.path.isdir("/root/reference/src"):
        subprocess.check_call(["make", "-s", "-B", "-C", _HERE, "ref"])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        L.mgo_f32_to_f16.restype = ctypes.c_uint16
        L.mgo_f32_to_f16.argtypes = [ctypes.c_float]
        L.mgo_f16_to_f32.restype = ctypes.c_float
        L.mgo_f16_to_f32.argtypes = [ctypes.c_uint16]
        for name in ("mgo_f32_to_f16_array", "mgo_f16_to_f32_array", "mgo_round_f16_array"):
            getattr(L, name).argtypes = [P, P, ctypes.c_size_t]
        L.mgo_quantize_q8_0.argtypes = [P, I64, I64, P]
        L.mgo_quantize_q4_k.argtypes = [P, I64, I64, P]
        L.mgo_q4k_scale_min.argtypes = [P, ctypes.c_int, P, P]
        L.mgo_dequant.argtypes = [ctypes.c_int, P, I64, I64, P]
        L.mgo_quantize_act_q8.argtypes = [P, I64, I64, P, P, P]
        L.mgo_block_dots.argtypes = [ctypes.c_int, P, I64, I64, P, I64, P]
        L.mgo_gemm_q_i8.argtypes = [ctypes.c_int, P, I64, I64, P, P, I64, P, ctypes.c_int, P, P]
        L.mgo_gemm_f32.argtypes = [P, I64, I64, P, I64, P, ctypes.c_int, P, P]
        L.mgo_gemm_q_deq_f32.argtypes = [ctypes.c_int, P, I64, I64, P, I64, P, ctypes.c_int, P, P]
        L.mgo_act.restype = ctypes.c_float
        L.mgo_act.argtypes = [ctypes.c_float, ctypes.c_int]
        L.mgo_layernorm_affine.argtypes = [P, P, P, I64, I64, ctypes.c_float, P]
        L.mgo_attention.argtypes = [P, P, P, P, I64, I64, I64, I64, ctypes.c_float, ctypes.c_int, P]
        L.mgo_get_rows.argtypes = [P, I64, I64, P, I64, P]
        L.mgo_merge_heads.argtypes = [P, I64, I64, I64, I64, P]
        L.mgo_conv_quant_w.argtypes = [P, I64, I64, P, P]
        L.mgo_conv2d_i8.argtypes = [P, I64, I64, I64, I64, P, P, I64, I64, I64, ctypes.c_int, ctypes.c_int, P]
        U64 = ctypes.c_uint64
        L.mgo_mt64_draws.argtypes = [U64, I64, P]
        L.mgo_mt64_draws.restype = None
        L.mgo_uniform_draws.argtypes = [U64, ctypes.c_double, ctypes.c_double, I64, P]
        L.mgo_uniform_draws.restype = None
        L.mgo_decode_step.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_float, P, I64, P, P]
        L.mgo_decode_step.restype = None
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def row_bytes(wtype: int, K: int) -> int:
    if wtype == WTYPE_Q8_0:
        return (K // 32) * 34
    if wtype == WTYPE_Q4_K:
        return (K // 256) * 144
    if wtype == WTYPE_F32:
        return K * 4
    raise ValueError(wtype)


# ---- fp16 -------------------------------------------------------------------
def f32_to_f16_bits(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().mgo_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().mgo_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def round_f16(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().mgo_round_f16_array(_p(x), _p(out), x.size)
    return out


# ---- weight formats -----------------------------------------------------------
def quantize(wtype: int, w) -> np.ndarray:
    """fp32 [N,K] -> raw block bytes [N, row_bytes] (uint8)."""
    w = _f32(w)
    N, K = w.shape
    out = np.zeros((N, row_bytes(wtype, K)), np.uint8)
    if wtype == WTYPE_Q8_0:
        assert K % 32 == 0
        lib().mgo_quantize_q8_0(_p(w), N, K, _p(out))
    elif wtype == WTYPE_Q4_K:
        assert K % 256 == 0
        lib().mgo_quantize_q4_k(_p(w), N, K, _p(out))
    else:
        raise ValueError(wtype)
    return out


def q4k_scale_min(scales12, j: int):
    s = np.ascontiguousarray(scales12, dtype=np.uint8)
    sc = ctypes.c_uint8()
    m = ctypes.c_uint8()
    lib().mgo_q4k_scale_min(_p(s), j, ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def dequant(wtype: int, wq, N: int, K: int) -> np.ndarray:
    wq = np.ascontiguousarray(wq)
    out = np.empty((N, K), np.float32)
    lib().mgo_dequant(wtype, _p(wq), N, K, _p(out))
    return out


# ---- activation quantizer -----------------------------------------------------
def quantize_act_q8(x):
    x = _f32(x)
    M, K = x.shape
    assert K % 32 == 0
    qx = np.empty((M, K), np.int8)
    dx = np.empty((M, K // 32), np.float32)
    sx = np.empty((M, K // 32), np.int32)
    lib().mgo_quantize_act_q8(_p(x), M, K, _p(qx), _p(dx), _p(sx))
    return qx, dx, sx


def block_dots(wtype: int, wq, N: int, K: int, qx) -> np.ndarray:
    qx = np.ascontiguousarray(qx, dtype=np.int8)
    M = qx.shape[0]
    out = np.empty((M, N, K // 32), np.int32)
    lib().mgo_block_dots(wtype, _p(np.ascontiguousarray(wq)), N, K, _p(qx), M, _p(out))
    return out


# ---- VQGAN int8 conv (mg-opencl.cpp:598-664) -------------------------------------
def conv_quant_w(ker):
    """ker [OC][IC][KH][KW] -> (qw int8 [OC][nb*32], dw fp32 [OC][nb]), 32-blocks of the
    kernel's own k = (ic*KH + kh)*KW + kw order"""
    ker = _f32(ker)
    OC = ker.shape[0]
    K = ker.size // OC
    nb = (K + 31) // 32
    qw = np.empty((OC, nb * 32), np.int8)
    dw = np.empty((OC, nb), np.float32)
    lib().mgo_conv_quant_w(_p(ker), OC, K, _p(qw), _p(dw))
    return qw, dw


def conv2d_i8(x, qw, dw, KH, KW, stride=1, pad=0):
    """x [N][IC][IH][IW] with quantized weights from conv_quant_w -> [N][OC][OH][OW]"""
    x = _f32(x)
    N, IC, IH, IW = x.shape
    OC = qw.shape[0]
    OH, OW = (IH + 2 * pad - KH) // stride + 1, (IW + 2 * pad - KW) // stride + 1
    out = np.empty((N, OC, OH, OW), np.float32)
    lib().mgo_conv2d_i8(_p(x), IW, IH, IC, N, _p(np.ascontiguousarray(qw, np.int8)), _p(_f32(dw)),
                        KW, KH, OC, stride, pad, _p(out))
    return out


# ---- GEMMs --------------------------------------------------------------------
def gemm_q_i8(wtype, wq, N, K, qx, dx, bias=None, act=0, resid=None) -> np.ndarray:
    qx = np.ascontiguousarray(qx, dtype=np.int8)
    dx = _f32(dx)
    M = qx.shape[0]
    bias = None if bias is None else _f32(bias)
    resid = None if resid is None else _f32(resid)
    y = np.empty((M, N), np.float32)
    lib().mgo_gemm_q_i8(wtype, _p(np.ascontiguousarray(wq)), N, K, _p(qx), _p(dx), M,
                        _p(bias), act, _p(resid), _p(y))
    return y


def gemm_f32(w, x, bias=None, act=0, resid=None) -> np.ndarray:
    w = _f32(w)
    x = _f32(x)
    N, K = w.shape
    M = x.shape[0]
    bias = None if bias is None else _f32(bias)
    resid = None if resid is None else _f32(resid)
    y = np.empty((M, N), np.float32)
    lib().mgo_gemm_f32(_p(w), N, K, _p(x), M, _p(bias), act, _p(resid), _p(y))
    return y


def gemm_q_deq_f32(wtype, wq, N, K, x, bias=None, act=0, resid=None) -> np.ndarray:
    x = _f32(x)
    M = x.shape[0]
    bias = None if bias is None else _f32(bias)
    resid = None if resid is None else _f32(resid)
    y = np.empty((M, N), np.float32)
    lib().mgo_gemm_q_deq_f32(wtype, _p(np.ascontiguousarray(wq)), N, K, _p(x), M,
                             _p(bias), act, _p(resid), _p(y))
    return y


def act(v: float, a: int) -> float:
    return lib().mgo_act(float(v), int(a))


# ---- norm / attention / glue ----------------------------------------------------
def layernorm_affine(x, gamma, beta, eps: float) -> np.ndarray:
    x = _f32(x)
    D = x.shape[-1]
    rows = x.size // D
    y = np.empty_like(x)
    g = None if gamma is None else _f32(gamma)
    b = None if beta is None else _f32(beta)
    lib().mgo_layernorm_affine(_p(x), _p(g), _p(b), rows, D, eps, _p(y))
    return y


def attention(q, k, v, strides, D, S, H, B, scale: float, f16kv: bool) -> np.ndarray:
    """q/k/v: flat fp32 buffers addressed with element strides {D,S,H,B}."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    st = np.ascontiguousarray(strides, dtype=np.int64)
    o = np.empty(D * S * H * B, np.float32)
    lib().mgo_attention(_p(q), _p(k), _p(v), _p(st), D, S, H, B, scale, int(bool(f16kv)), _p(o))
    return o


def get_rows(a, ids) -> np.ndarray:
    a = _f32(a)
    R, E = a.shape
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    o = np.empty((ids.size, E), np.float32)
    lib().mgo_get_rows(_p(a), E, R, _p(ids), ids.size, _p(o))
    return o


def merge_heads(a, D, S, H, B) -> np.ndarray:
    a = _f32(a)
    o = np.empty(D * S * H * B, np.float32)
    lib().mgo_merge_heads(_p(a), D, S, H, B, _p(o))
    return o


# ---- iterative decoding (src/mg-generate.cpp:82-121) -----------------------------
def mt64_draws(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    lib().mgo_mt64_draws(seed, n, _p(out))
    return out


def uniform_draws(seed: int, a: float, b: float, n: int) -> np.ndarray:
    out = np.empty(n, np.float64)
    lib().mgo_uniform_draws(seed, a, b, n, _p(out))
    return out


def decode_step(logits, tokens, step: int, n_steps: int, seeds, draws_before: int,
                codebook: int = 1024, mask_id: int = 2024, n_tokens: int = 256,
                choice_temp: float = 4.5):
    """One decoding step for B images; returns (new tokens, step samples before re-masking)."""
    logits = _f32(logits)
    B, S, V = logits.shape
    tok = np.ascontiguousarray(tokens, np.int32).copy()
    res = np.empty_like(tok)
    sd = np.ascontiguousarray(seeds, np.uint64)
    lib().mgo_decode_step(_p(logits), B, S, V, codebook, mask_id, n_tokens, step, n_steps,
                          choice_temp, _p(sd), draws_before, _p(tok), _p(res))
    return tok, res
