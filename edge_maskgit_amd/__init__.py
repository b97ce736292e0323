"""edge_maskgit_amd — MI355X (gfx950) backend for the edge_maskgit Q8_0/Q4_K FC hot path.

The product is the native code: ``lib/libmgh.so`` (HIP kernels + the C ABI declared in
``include/mgh.h``) and ``lib/libmg_hip.so`` (the C++ mg tensor/graph API and HipRuntime).
This module is a thin ctypes binding used by tests and bench.py. It never falls back to
a CPU implementation: if the native library is missing or no gfx950 device is present,
calls raise.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG, "lib")
LIBMGH = os.path.join(LIB_DIR, "libmgh.so")

WTYPE_F32 = 0
WTYPE_Q8_0 = 8
WTYPE_Q4_K = 12
ACT_NONE, ACT_GELU, ACT_SILU = 0, 1, 2
EMIT_NONE, EMIT_INT8, EMIT_DEQ_F16 = 0, 1, 2
ALGO_AUTO, ALGO_INT8, ALGO_DEQ_F16 = 0, 1, 2

# every entry point include/mgh.h declares (checked by tests/test_abi.py)
MGH_SYMBOLS = [
    "mgh_create", "mgh_destroy", "mgh_last_error", "mgh_device_name", "mgh_version",
    "mgh_alloc", "mgh_free", "mgh_h2d", "mgh_d2h", "mgh_fill_u32", "mgh_sync",
    "mgh_timer_start", "mgh_timer_stop",
    "mgh_quantize_act_q8", "mgh_gemm_q", "mgh_gemm_q_f32in", "mgh_debug_block_dots",
    "mgh_graph_begin", "mgh_graph_end", "mgh_graph_launch", "mgh_graph_destroy",
    "mgh_quantize_act_q8_codes16",
    "mgh_packed_weight_bytes", "mgh_pack_weights", "mgh_gemm_q_packed", "mgh_debug_block_dots_packed",
    "mgh_gemm_q_packed_f32in",
    "mgh_layernorm_affine", "mgh_flash_attn_f16kv", "mgh_gemm_f32", "mgh_get_rows", "mgh_add",
    "mgh_copy_strided", "mgh_decode_state_bytes", "mgh_decode_work_bytes", "mgh_decode_init",
    "mgh_decode_step", "mgh_packed_weight_bytes_f16", "mgh_pack_weights_f16", "mgh_f32_to_f16",
    "mgh_gemm_h16", "mgh_gemm_h16_f32in", "mgh_gemm_h16_y16", "mgh_gemm_h16_ln", "mgh_flash_attn_f16kv_o16", "mgh_flash_attn_f16in",
    "mgh_softmax", "mgh_binary", "mgh_scale", "mgh_unary", "mgh_gemm_f32_batched",
    "mgh_gemm_h16_f32in_noalloc", "mgh_conv2d", "mgh_group_norm", "mgh_upscale", "mgh_conv2d_ex",
    "mgh_conv2d_packed_bytes", "mgh_conv2d_pack_weights", "mgh_conv2d_i8_weight_bytes",
    "mgh_conv2d_i8_pack_weights", "mgh_conv2d_i8",
    "mgh_packed_weight_bytes_dq", "mgh_pack_weights_dq", "mgh_gemm_dq", "mgh_gemm_dq_f32in",
    "mgh_gemm_dq_y16", "mgh_gemm_dq_ln", "mgh_dequant_weights_f32",
]

_lib = None


class MghError(RuntimeError):
    pass


def build_native(verbose: bool = False) -> None:
    """Compile the native libraries in-tree (see edge_maskgit_amd/build.py)."""
    import importlib
    importlib.import_module(__name__ + ".build").build(verbose=verbose, force=True)


def lib():
    """Load libmgh.so (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBMGH):
            raise MghError(f"native library missing: {LIBMGH} — run __graft_entry__.build()")
        L = ctypes.CDLL(LIBMGH)
        P, I, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        L.mgh_create.argtypes = [I, ctypes.POINTER(P)]
        L.mgh_destroy.argtypes = [P]
        L.mgh_destroy.restype = None
        L.mgh_last_error.argtypes = [P]
        L.mgh_last_error.restype = ctypes.c_char_p
        L.mgh_device_name.argtypes = [P]
        L.mgh_device_name.restype = ctypes.c_char_p
        L.mgh_alloc.argtypes = [P, SZ, ctypes.POINTER(P)]
        L.mgh_free.argtypes = [P, P]
        L.mgh_h2d.argtypes = [P, P, P, SZ]
        L.mgh_d2h.argtypes = [P, P, P, SZ]
        L.mgh_fill_u32.argtypes = [P, P, ctypes.c_uint32, SZ]
        L.mgh_sync.argtypes = [P]
        L.mgh_timer_start.argtypes = [P]
        L.mgh_timer_stop.argtypes = [P, ctypes.POINTER(ctypes.c_float)]
        L.mgh_quantize_act_q8.argtypes = [P, P, I, I, P, P, P]
        L.mgh_gemm_q.argtypes = [P, I, P, I, I, P, P, P, I, P, I, P, P]
        L.mgh_gemm_q_f32in.argtypes = [P, I, I, P, I, I, P, I, P, I, P, P]
        L.mgh_debug_block_dots.argtypes = [P, I, P, I, I, P, I, P]
        L.mgh_quantize_act_q8_codes16.argtypes = [P, P, I, I, P, P, P]
        L.mgh_packed_weight_bytes.argtypes = [I, I, I]
        L.mgh_packed_weight_bytes.restype = SZ
        L.mgh_pack_weights.argtypes = [P, I, P, I, I, P]
        L.mgh_gemm_q_packed.argtypes = [P, I, P, I, I, P, P, P, I, P, I, P, P]
        L.mgh_debug_block_dots_packed.argtypes = [P, I, P, I, I, P, I, P]
        L.mgh_gemm_q_packed_f32in.argtypes = [P, I, I, P, I, I, P, I, P, I, P, P]
        I64 = ctypes.c_int64
        L.mgh_layernorm_affine.argtypes = [P, P, P, P, I, I, ctypes.c_float, P, I, P, P, P]
        L.mgh_flash_attn_f16kv.argtypes = [P, P, P, P, P, I, I, I, I, ctypes.c_float, P, P]
        L.mgh_gemm_f32.argtypes = [P, P, I, I, P, I, P, I, P, P]
        L.mgh_get_rows.argtypes = [P, P, I64, I64, P, I64, P]
        L.mgh_add.argtypes = [P, P, P, I64, P, I64]
        L.mgh_copy_strided.argtypes = [P, P, P, P, P]
        L.mgh_packed_weight_bytes_f16.argtypes = [I, I]
        L.mgh_packed_weight_bytes_f16.restype = SZ
        L.mgh_pack_weights_f16.argtypes = [P, I, P, I, I, P]
        L.mgh_f32_to_f16.argtypes = [P, P, I64, P]
        L.mgh_gemm_h16.argtypes = [P, P, I, I, P, I, P, I, P, P]
        L.mgh_gemm_h16_f32in.argtypes = [P, P, I, I, P, I, P, I, P, P]
        L.mgh_gemm_h16_y16.argtypes = [P, P, I, I, P, I, P, I, P, P]
        L.mgh_gemm_h16_ln.argtypes = [P, P, I, I, P, I, P, I, P, P, P, P, ctypes.c_float, P, I, P, P, P]
        L.mgh_gemm_h16_f32in_noalloc.argtypes = [P, P, I, I, P, I, P, I, P, P]
        L.mgh_packed_weight_bytes_dq.argtypes = [I, I, I]
        L.mgh_packed_weight_bytes_dq.restype = SZ
        L.mgh_pack_weights_dq.argtypes = [P, I, P, I, I, P]
        L.mgh_dequant_weights_f32.argtypes = [P, I, P, I, I, P]
        L.mgh_gemm_dq.argtypes = [P, I, P, I, I, P, I, P, I, P, P]
        L.mgh_gemm_dq_f32in.argtypes = [P, I, P, I, I, P, I, P, I, P, P]
        L.mgh_gemm_dq_y16.argtypes = [P, I, P, I, I, P, I, P, I, P, P]
        L.mgh_gemm_dq_ln.argtypes = [P, I, P, I, I, P, I, P, I, P, P, P, P, ctypes.c_float, P, I, P, P, P]
        L.mgh_flash_attn_f16kv_o16.argtypes = [P, P, P, P, P, I, I, I, I, ctypes.c_float, P, P]
        L.mgh_flash_attn_f16in.argtypes = [P, P, P, P, P, I, I, I, I, ctypes.c_float, P, P, P]
        L.mgh_decode_state_bytes.argtypes = [I]
        L.mgh_decode_state_bytes.restype = SZ
        L.mgh_decode_work_bytes.argtypes = [I, I]
        L.mgh_decode_work_bytes.restype = SZ
        L.mgh_decode_init.argtypes = [P, I, P, P]
        L.mgh_decode_step.argtypes = [P, P, P, P, I, I, I, I, I, I, I, I, ctypes.c_float, P, P]
        L.mgh_softmax.argtypes = [P, P, I64, I, ctypes.c_float, P]
        L.mgh_binary.argtypes = [P, I, P, P, P, P, P, P, P]
        L.mgh_scale.argtypes = [P, P, I64, ctypes.c_float, P]
        L.mgh_unary.argtypes = [P, I, P, I64, P]
        L.mgh_gemm_f32_batched.argtypes = [P, P, P, P, P, P, P, P, I, P, P]
        L.mgh_conv2d.argtypes = [P, P, I, I, I, I, P, I, I, I, I, I, P]
        L.mgh_conv2d_ex.argtypes = [P, P, I, I, I, I, P, P, I, I, I, I, I, P, P, P]
        L.mgh_conv2d_packed_bytes.argtypes = [I, I, I, I]
        L.mgh_conv2d_packed_bytes.restype = ctypes.c_size_t
        L.mgh_conv2d_pack_weights.argtypes = [P, P, I, I, I, I, P]
        L.mgh_conv2d_i8_weight_bytes.argtypes = [I, I, I, I]
        L.mgh_conv2d_i8_weight_bytes.restype = ctypes.c_size_t
        L.mgh_conv2d_i8_pack_weights.argtypes = [P, P, I, I, I, I, P]
        L.mgh_conv2d_i8.argtypes = [P, P, I, I, I, I, P, I, I, I, I, I, P, P, P]
        L.mgh_group_norm.argtypes = [P, P, I, I, I, I, I, ctypes.c_float, P, P, P]
        L.mgh_upscale.argtypes = [P, P, I, I, I, I, I, P]
        L.mgh_graph_begin.argtypes = [P]
        L.mgh_graph_end.argtypes = [P, ctypes.POINTER(P)]
        L.mgh_graph_launch.argtypes = [P, P]
        L.mgh_graph_destroy.argtypes = [P]
        L.mgh_graph_destroy.restype = None
        _lib = L
    return _lib


def packed_weight_bytes_f16(N: int, K: int) -> int:
    return int(lib().mgh_packed_weight_bytes_f16(N, K))


def packed_weight_bytes_dq(wtype: int, N: int, K: int) -> int:
    """bytes of the K-loop-dequant weight layout (GGUF-sized: 1.0625 / 0.5625 bytes per weight
    for N % 16 == 0)"""
    return int(lib().mgh_packed_weight_bytes_dq(wtype, N, K))


def decode_state_bytes(B: int) -> int:
    return int(lib().mgh_decode_state_bytes(B))


def decode_work_bytes(B: int, S: int) -> int:
    return int(lib().mgh_decode_work_bytes(B, S))


def packed_weight_bytes(wtype: int, N: int, K: int) -> int:
    """Size of mgh_pack_weights' output (0 for an invalid type/shape)."""
    return int(lib().mgh_packed_weight_bytes(wtype, N, K))


class DeviceBuffer:
    """Owned device allocation (freed with the context)."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        ctx._check(lib().mgh_alloc(ctx.h, self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    def free(self):
        if self.ptr:
            lib().mgh_free(self.ctx.h, ctypes.c_void_p(self.ptr))
            self.ptr = None

    @property
    def p(self):
        return ctypes.c_void_p(self.ptr)


class Context:
    """One mgh_ctx (device + stream). Not thread-safe, like the reference runtime."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        rc = lib().mgh_create(device, ctypes.byref(h))
        if rc != 0:
            raise MghError(f"mgh_create({device}) failed with {rc} (no gfx950 device?)")
        self.h = h
        self._bufs: list[DeviceBuffer] = []

    def close(self):
        if self.h:
            for b in self._bufs:
                b.free()
            self._bufs.clear()
            lib().mgh_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc):
        if rc != 0:
            raise MghError(f"mgh error {rc}: {lib().mgh_last_error(self.h).decode()}")

    @property
    def device_name(self) -> str:
        return lib().mgh_device_name(self.h).decode()

    # ---- memory ----
    def alloc(self, nbytes: int) -> DeviceBuffer:
        b = DeviceBuffer(self, nbytes)
        self._bufs.append(b)
        return b

    def upload(self, arr: np.ndarray) -> DeviceBuffer:
        arr = np.ascontiguousarray(arr)
        b = self.alloc(max(arr.nbytes, 1))
        self._check(lib().mgh_h2d(self.h, b.p, arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes))
        return b

    def write(self, buf: DeviceBuffer, arr: np.ndarray):
        """Copy a host array into the start of an existing device buffer."""
        arr = np.ascontiguousarray(arr)
        if arr.nbytes > buf.nbytes:
            raise ValueError("write: array larger than the buffer")
        self._check(lib().mgh_h2d(self.h, buf.p, arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes))

    def download(self, buf: DeviceBuffer, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        self._check(lib().mgh_d2h(self.h, out.ctypes.data_as(ctypes.c_void_p), buf.p, out.nbytes))
        return out

    def free(self, buf: DeviceBuffer):
        buf.free()
        if buf in self._bufs:
            self._bufs.remove(buf)

    def sync(self):
        self._check(lib().mgh_sync(self.h))

    def timer_start(self):
        self._check(lib().mgh_timer_start(self.h))

    def timer_stop(self) -> float:
        ms = ctypes.c_float()
        self._check(lib().mgh_timer_stop(self.h, ctypes.byref(ms)))
        return ms.value

    # ---- kernels (device pointers in, device pointers out; stream-ordered) ----
    @staticmethod
    def _ptr(b):
        if b is None:
            return None
        return b.p if isinstance(b, DeviceBuffer) else ctypes.c_void_p(int(b))

    def fill_u32(self, buf, value, n_words):
        self._check(lib().mgh_fill_u32(self.h, self._ptr(buf), value, n_words))

    def quantize_act_q8(self, x, M, K, qx, dx, sx=None):
        P = self._ptr
        self._check(lib().mgh_quantize_act_q8(self.h, P(x), M, K, P(qx), P(dx), P(sx)))

    def gemm_q(self, wtype, w, N, K, qx, dx, sx, M, bias, act, resid, y):
        P = self._ptr
        self._check(lib().mgh_gemm_q(self.h, wtype, P(w), N, K, P(qx), P(dx), P(sx), M,
                                     P(bias), act, P(resid), P(y)))

    def quantize_act_q8_codes16(self, x, M, K, qx16, dx, sx=None):
        P = self._ptr
        self._check(lib().mgh_quantize_act_q8_codes16(self.h, P(x), M, K, P(qx16), P(dx), P(sx)))

    def pack_weights(self, wtype, w, N, K, wp):
        P = self._ptr
        self._check(lib().mgh_pack_weights(self.h, wtype, P(w), N, K, P(wp)))

    def gemm_q_packed(self, wtype, wp, N, K, qx16, dx, sx, M, bias, act, resid, y):
        P = self._ptr
        self._check(lib().mgh_gemm_q_packed(self.h, wtype, P(wp), N, K, P(qx16), P(dx), P(sx), M,
                                            P(bias), act, P(resid), P(y)))

    def layernorm_affine(self, x, gamma, beta, rows, D, eps, y, emit=0, codes=None, dx=None, s4=None):
        P = self._ptr
        self._check(lib().mgh_layernorm_affine(self.h, P(x), P(gamma), P(beta), rows, D, eps, P(y),
                                               emit, P(codes), P(dx), P(s4)))

    def flash_attn_f16kv(self, q, k, v, strides, D, S, H, B, scale, o, o_strides=None):
        P = self._ptr
        st = (ctypes.c_int64 * 4)(*strides)
        ost = (ctypes.c_int64 * 4)(*o_strides) if o_strides is not None else None
        self._check(lib().mgh_flash_attn_f16kv(self.h, P(q), P(k), P(v), st, D, S, H, B, scale,
                                               P(o), ost))

    def gemm_f32(self, w, N, K, x, M, bias, act, resid, y):
        P = self._ptr
        self._check(lib().mgh_gemm_f32(self.h, P(w), N, K, P(x), M, P(bias), act, P(resid), P(y)))

    def get_rows(self, a, E, R, ids, n, out):
        P = self._ptr
        self._check(lib().mgh_get_rows(self.h, P(a), E, R, P(ids), n, P(out)))

    def add(self, a, b, nb, out, n):
        P = self._ptr
        self._check(lib().mgh_add(self.h, P(a), P(b), nb, P(out), n))

    def copy_strided(self, a, ne, strides, out):
        P = self._ptr
        self._check(lib().mgh_copy_strided(self.h, P(a), (ctypes.c_int64 * 4)(*ne),
                                           (ctypes.c_int64 * 4)(*strides), P(out)))

    def pack_weights_f16(self, wtype, w, N, K, wp16):
        self._check(lib().mgh_pack_weights_f16(self.h, wtype, self._ptr(w), N, K, self._ptr(wp16)))

    def f32_to_f16(self, x, n, x16):
        self._check(lib().mgh_f32_to_f16(self.h, self._ptr(x), n, self._ptr(x16)))

    def gemm_h16(self, wp16, N, K, x16, M, bias, act, resid, y):
        P = self._ptr
        self._check(lib().mgh_gemm_h16(self.h, P(wp16), N, K, P(x16), M, P(bias), act, P(resid), P(y)))

    def gemm_h16_ln(self, wp16, N, K, x16, M, bias, act, resid, y, gamma, beta, eps, y_ln, emit=0, codes=None,
                    dx=None, s4=None):
        """gemm_h16 into y, then the LayerNorm-affine of y's rows into y_ln (and the emitted
        operand), as gemm_h16 followed by layernorm_affine(y)."""
        P = self._ptr
        self._check(lib().mgh_gemm_h16_ln(self.h, P(wp16), N, K, P(x16), M, P(bias), act, P(resid), P(y), P(gamma),
                                          P(beta), eps, P(y_ln), emit, P(codes), P(dx), P(s4)))

    def gemm_h16_y16(self, wp16, N, K, x16, M, bias, act, resid, y16):
        P = self._ptr
        self._check(lib().mgh_gemm_h16_y16(self.h, P(wp16), N, K, P(x16), M, P(bias), act, P(resid), P(y16)))

    def flash_attn_f16kv_o16(self, q, k, v, strides, D, S, H, B, scale, o16, o_strides=None):
        P = self._ptr
        st = (ctypes.c_int64 * 4)(*strides)
        ost = None if o_strides is None else (ctypes.c_int64 * 4)(*o_strides)
        self._check(lib().mgh_flash_attn_f16kv_o16(self.h, P(q), P(k), P(v), st, D, S, H, B, scale, P(o16), ost))

    def flash_attn_f16in(self, q16, k16, v16, strides, D, S, H, B, scale, o=None, o16=None, o_strides=None):
        """Attention on fp16 q/k/v (element strides as for flash_attn_f16kv); exactly one of
        o (fp32) and o16 (fp16) is given."""
        P = self._ptr
        st = (ctypes.c_int64 * 4)(*strides)
        ost = None if o_strides is None else (ctypes.c_int64 * 4)(*o_strides)
        self._check(lib().mgh_flash_attn_f16in(self.h, P(q16), P(k16), P(v16), st, D, S, H, B, scale,
                                               P(o), P(o16), ost))

    def gemm_h16_f32in(self, wp16, N, K, x, M, bias, act, resid, y):
        P = self._ptr
        self._check(lib().mgh_gemm_h16_f32in(self.h, P(wp16), N, K, P(x), M, P(bias), act, P(resid), P(y)))

    def dequant_weights_f32(self, wtype, w, N, K, out):
        self._check(lib().mgh_dequant_weights_f32(self.h, wtype, self._ptr(w), N, K, self._ptr(out)))

    def pack_weights_dq(self, wtype, w, N, K, wdq):
        self._check(lib().mgh_pack_weights_dq(self.h, wtype, self._ptr(w), N, K, self._ptr(wdq)))

    def gemm_dq(self, wtype, wdq, N, K, x16, M, bias, act, resid, y):
        P = self._ptr
        self._check(lib().mgh_gemm_dq(self.h, wtype, P(wdq), N, K, P(x16), M, P(bias), act, P(resid), P(y)))

    def gemm_dq_f32in(self, wtype, wdq, N, K, x, M, bias, act, resid, y):
        P = self._ptr
        self._check(lib().mgh_gemm_dq_f32in(self.h, wtype, P(wdq), N, K, P(x), M, P(bias), act, P(resid), P(y)))

    def gemm_dq_y16(self, wtype, wdq, N, K, x16, M, bias, act, resid, y16):
        P = self._ptr
        self._check(lib().mgh_gemm_dq_y16(self.h, wtype, P(wdq), N, K, P(x16), M, P(bias), act, P(resid), P(y16)))

    def gemm_dq_ln(self, wtype, wdq, N, K, x16, M, bias, act, resid, y, gamma, beta, eps, y_ln, emit=0,
                   codes=None, dx=None, s4=None):
        P = self._ptr
        self._check(lib().mgh_gemm_dq_ln(self.h, wtype, P(wdq), N, K, P(x16), M, P(bias), act, P(resid), P(y),
                                         P(gamma), P(beta), eps, P(y_ln), emit, P(codes), P(dx), P(s4)))

    def gemm_h16_f32in_noalloc(self, wp16, N, K, x, M, bias, act, resid, y):
        """mgh_gemm_h16_f32in with its scratch in the library's fixed per-GPU array."""
        P = self._ptr
        self._check(lib().mgh_gemm_h16_f32in_noalloc(self.h, P(wp16), N, K, P(x), M, P(bias), act, P(resid),
                                                     P(y)))

    def decode_init(self, seeds, state):
        """seeds: host sequence of B uint64 seeds; state: mgh_decode_state_bytes(B) bytes."""
        sd = (ctypes.c_uint64 * len(seeds))(*[int(v) for v in seeds])
        self._check(lib().mgh_decode_init(self.h, len(seeds), sd, self._ptr(state)))

    def decode_step(self, state, work, logits, B, S, V, codebook, mask_id, n_tokens, step, n_steps,
                    choice_temp, tokens, result):
        P = self._ptr
        self._check(lib().mgh_decode_step(self.h, P(state), P(work), P(logits), B, S, V, codebook,
                                          mask_id, n_tokens, step, n_steps, choice_temp, P(tokens),
                                          P(result)))

    def gemm_q_packed_f32in(self, algo, wtype, wp, N, K, x, M, bias, act, resid, y):
        P = self._ptr
        self._check(lib().mgh_gemm_q_packed_f32in(self.h, algo, wtype, P(wp), N, K, P(x), M,
                                                  P(bias), act, P(resid), P(y)))

    def debug_block_dots_packed(self, wtype, wp, N, K, qx16, M, out):
        P = self._ptr
        self._check(lib().mgh_debug_block_dots_packed(self.h, wtype, P(wp), N, K, P(qx16), M, P(out)))

    def gemm_q_f32in(self, algo, wtype, w, N, K, x, M, bias, act, resid, y):
        P = self._ptr
        self._check(lib().mgh_gemm_q_f32in(self.h, algo, wtype, P(w), N, K, P(x), M,
                                           P(bias), act, P(resid), P(y)))

    def softmax(self, x, rows, D, scale, y):
        self._check(lib().mgh_softmax(self.h, self._ptr(x), rows, D, scale, self._ptr(y)))

    def binary(self, op, a, a_strides, b, b_ne, b_strides, ne, out):
        P, A = self._ptr, (lambda v: (ctypes.c_int64 * 4)(*v))
        self._check(lib().mgh_binary(self.h, op, P(a), A(a_strides), P(b), A(b_ne), A(b_strides), A(ne), P(out)))

    def scale(self, x, n, s, y):
        self._check(lib().mgh_scale(self.h, self._ptr(x), n, s, self._ptr(y)))

    def unary(self, act, x, n, y):
        self._check(lib().mgh_unary(self.h, act, self._ptr(x), n, self._ptr(y)))

    def gemm_f32_batched(self, w, w_ne, w_strides, x, x_ne, x_strides, bias, act, resid, y):
        P, A = self._ptr, (lambda v: (ctypes.c_int64 * 4)(*v))
        self._check(lib().mgh_gemm_f32_batched(self.h, P(w), A(w_ne), A(w_strides), P(x), A(x_ne), A(x_strides),
                                               P(bias), act, P(resid), P(y)))

    # ---- VQGAN decoder ops, layout {W, H, C, N} ----
    def conv2d(self, x, IW, IH, IC, N, ker, KW, KH, OC, stride, pad, y):
        P = self._ptr
        self._check(lib().mgh_conv2d(self.h, P(x), IW, IH, IC, N, P(ker), KW, KH, OC, stride, pad, P(y)))

    def conv2d_ex(self, x, IW, IH, IC, N, ker, packed, KW, KH, OC, stride, pad, bias, resid, y):
        P = self._ptr
        self._check(lib().mgh_conv2d_ex(self.h, P(x), IW, IH, IC, N, P(ker), P(packed), KW, KH, OC, stride, pad,
                                        P(bias), P(resid), P(y)))

    @staticmethod
    def conv2d_packed_bytes(KW, KH, IC, OC) -> int:
        return lib().mgh_conv2d_packed_bytes(KW, KH, IC, OC)

    def conv2d_pack_weights(self, ker, KW, KH, IC, OC, packed):
        P = self._ptr
        self._check(lib().mgh_conv2d_pack_weights(self.h, P(ker), KW, KH, IC, OC, P(packed)))

    @staticmethod
    def conv2d_i8_weight_bytes(KW, KH, IC, OC) -> int:
        return lib().mgh_conv2d_i8_weight_bytes(KW, KH, IC, OC)

    def conv2d_i8_pack_weights(self, ker, KW, KH, IC, OC, wq):
        P = self._ptr
        self._check(lib().mgh_conv2d_i8_pack_weights(self.h, P(ker), KW, KH, IC, OC, P(wq)))

    def conv2d_i8(self, x, IW, IH, IC, N, wq, KW, KH, OC, stride, pad, bias, resid, y):
        P = self._ptr
        self._check(lib().mgh_conv2d_i8(self.h, P(x), IW, IH, IC, N, P(wq), KW, KH, OC, stride, pad, P(bias),
                                        P(resid), P(y)))

    def group_norm(self, x, W, H, C, N, groups, eps, gamma, beta, y):
        P = self._ptr
        self._check(lib().mgh_group_norm(self.h, P(x), W, H, C, N, groups, eps, P(gamma), P(beta), P(y)))

    def upscale(self, x, W, H, C, N, factor, y):
        self._check(lib().mgh_upscale(self.h, self._ptr(x), W, H, C, N, factor, self._ptr(y)))

    # ---- graphs ----
    def graph_begin(self):
        self._check(lib().mgh_graph_begin(self.h))

    def graph_end(self) -> "Graph":
        g = ctypes.c_void_p()
        self._check(lib().mgh_graph_end(self.h, ctypes.byref(g)))
        return Graph(self, g)

    def debug_block_dots(self, wtype, w, N, K, qx, M, out):
        P = self._ptr
        self._check(lib().mgh_debug_block_dots(self.h, wtype, P(w), N, K, P(qx), M, P(out)))


class Graph:
    """A captured, instantiated sequence of calls (mgh_graph)."""

    def __init__(self, ctx: Context, h):
        self.ctx = ctx
        self.h = h

    def launch(self):
        self.ctx._check(lib().mgh_graph_launch(self.ctx.h, self.h))

    def destroy(self):
        if self.h:
            lib().mgh_graph_destroy(self.h)
            self.h = None


def gpu_available() -> bool:
    """True if libmgh.so loads and a gfx950 device can be opened."""
    try:
        with Context(0):
            return True
    except Exception:
        return False
