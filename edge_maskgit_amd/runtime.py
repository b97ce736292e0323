"""ctypes binding of lib/libmg_hip.so (include/mgr.h): the C++ transformer runtime.

TransformerRuntime loads a GGUF model, builds the reference's transformer graph
(mg::build_transformer) and runs it on the GPU through HipRuntime — the role of the
reference's TransformerFwd hook (include/mg-generate.hpp:15). No CPU fallback: loading raises
when the native library or the device is missing.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import LIB_DIR, MghError

MGR_SYMBOLS = ["mgr_load", "mgr_free", "mgr_last_error", "mgr_hparams", "mgr_device_name",
               "mgr_forward", "mgr_profile_enable", "mgr_profile_report", "mgr_gguf_info",
               "mgr_graph_stats", "mgr_decode_params", "mgr_generate", "mgr_named", "mgr_decode_images",
               "mgr_image_side", "mgr_generate_images"]

_lib = None


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(LIB_DIR, "libmg_hip.so")
        if not os.path.exists(path):
            raise MghError(f"{path} is missing: run edge_maskgit_amd.build_native() first")
        L = ctypes.CDLL(path)
        P, I = ctypes.c_void_p, ctypes.c_int
        L.mgr_load.argtypes = [ctypes.c_char_p, I, I, ctypes.POINTER(P)]
        L.mgr_free.argtypes = [P]
        L.mgr_free.restype = None
        L.mgr_last_error.restype = ctypes.c_char_p
        L.mgr_hparams.argtypes = [P, P]
        L.mgr_device_name.argtypes = [P]
        L.mgr_device_name.restype = ctypes.c_char_p
        L.mgr_forward.argtypes = [P, P, I, I, P]
        L.mgr_profile_enable.argtypes = [P, I]
        L.mgr_profile_report.argtypes = [P, ctypes.c_char_p, ctypes.c_size_t]
        L.mgr_gguf_info.argtypes = [ctypes.c_char_p, P, ctypes.POINTER(ctypes.c_int64)]
        L.mgr_graph_stats.argtypes = [ctypes.c_char_p, I, I, P]
        L.mgr_decode_params.argtypes = [P, P, P, P]
        L.mgr_generate.argtypes = [P, P, P, I, I, ctypes.c_float, P]
        L.mgr_named.argtypes = [P, ctypes.c_char_p, P, ctypes.c_int64]
        L.mgr_decode_images.argtypes = [P, P, I, P]
        L.mgr_image_side.argtypes = [P]
        L.mgr_generate_images.argtypes = [P, P, P, I, I, ctypes.c_float, P, P]
        _lib = L
    return _lib


def _check(rc):
    if rc < 0:
        raise MghError("mgr: " + lib().mgr_last_error().decode())
    return rc


HPARAM_NAMES = ("n_layer", "n_head", "n_embd", "head_dim", "vocab_size", "n_positions",
                "mask_token_id")


def gguf_info(path: str) -> dict:
    """Host-only parse of a GGUF file (the C++ loader)."""
    hp = np.zeros(7, np.int32)
    nt = ctypes.c_int64()
    _check(lib().mgr_gguf_info(path.encode(), hp.ctypes.data_as(ctypes.c_void_p), ctypes.byref(nt)))
    d = dict(zip(HPARAM_NAMES, (int(v) for v in hp)))
    d["n_tensors"] = int(nt.value)
    return d


def graph_stats(path: str, S: int, B: int) -> tuple:
    """Host-only: node count of the forward graph and the count per mg::Op code."""
    counts = np.zeros(32, np.int32)
    n = _check(lib().mgr_graph_stats(path.encode(), S, B, counts.ctypes.data_as(ctypes.c_void_p)))
    return n, counts


class TransformerRuntime:
    """A GGUF model on one GPU. algo: 2 = dequant-fp16 FC layers (default, the reference's
    choice on a device without cl_arm_integer_dot_product), 1 = int8-dot."""

    def __init__(self, path: str, device: int = 0, algo: int = 2):
        h = ctypes.c_void_p()
        _check(lib().mgr_load(path.encode(), device, algo, ctypes.byref(h)))
        self.h = h
        hp = np.zeros(7, np.int32)
        _check(lib().mgr_hparams(self.h, hp.ctypes.data_as(ctypes.c_void_p)))
        self.hparams = dict(zip(HPARAM_NAMES, (int(v) for v in hp)))
        nt, cb, ct = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_float()
        _check(lib().mgr_decode_params(self.h, ctypes.byref(nt), ctypes.byref(cb), ctypes.byref(ct)))
        self.hparams.update(n_tokens=nt.value, codebook_size=cb.value, choice_temperature=ct.value)

    def close(self):
        if self.h:
            lib().mgr_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def device_name(self) -> str:
        return lib().mgr_device_name(self.h).decode()

    def forward(self, tokens: np.ndarray, readback: bool = True):
        """tokens int32 [B][S] -> logits float32 [B][S][vocab] (None without readback)."""
        tok = np.ascontiguousarray(tokens, dtype=np.int32)
        if tok.ndim == 1:
            tok = tok[None]
        B, S = tok.shape
        out = np.empty((B, S, self.hparams["vocab_size"]), np.float32) if readback else None
        _check(lib().mgr_forward(self.h, tok.ctypes.data_as(ctypes.c_void_p), S, B,
                                 None if out is None else out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def generate(self, class_ids, seeds, steps: int = 8, temperature: float = -1.0) -> np.ndarray:
        """Iterative decoding on the device (mgr_generate): one image per class id / seed;
        returns the final token grids int32 [B][n_tokens]."""
        cls = np.ascontiguousarray(class_ids, dtype=np.int32).reshape(-1)
        sd = np.ascontiguousarray(seeds, dtype=np.uint64).reshape(-1)
        if cls.shape != sd.shape:
            raise ValueError("one seed per class id")
        out = np.empty((cls.size, self.hparams["n_tokens"]), np.int32)
        _check(lib().mgr_generate(self.h, cls.ctypes.data_as(ctypes.c_void_p),
                                  sd.ctypes.data_as(ctypes.c_void_p), cls.size, steps, temperature,
                                  out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def decode_images(self, grids, readback: bool = True):
        """VQGAN decode (mgr_decode_images): token grids int32 [B][n_tokens] -> images float32
        [B][3][side][side] (None without readback)."""
        g = np.ascontiguousarray(grids, dtype=np.int32)
        if g.ndim == 1:
            g = g[None]
        if g.ndim != 2 or g.shape[1] != self.hparams["n_tokens"]:
            raise ValueError(f"grids must be [B][{self.hparams['n_tokens']}]")
        side = _check(lib().mgr_image_side(self.h))
        out = np.empty((g.shape[0], 3, side, side), np.float32) if readback else None
        _check(lib().mgr_decode_images(self.h, g.ctypes.data_as(ctypes.c_void_p), g.shape[0],
                                       None if out is None else out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def generate_images(self, class_ids, seeds, steps: int = 8, temperature: float = -1.0):
        """generate() end to end (mgr_generate_images): token grids int32 [B][n_tokens] and
        images float32 [B][3][side][side]."""
        cls = np.ascontiguousarray(class_ids, dtype=np.int32).reshape(-1)
        sd = np.ascontiguousarray(seeds, dtype=np.uint64).reshape(-1)
        if cls.shape != sd.shape:
            raise ValueError("one seed per class id")
        side = _check(lib().mgr_image_side(self.h))
        if side <= 0:
            raise MghError("mgr: the model has no VQGAN decoder")
        grids = np.empty((cls.size, self.hparams["n_tokens"]), np.int32)
        imgs = np.empty((cls.size, 3, side, side), np.float32)
        _check(lib().mgr_generate_images(self.h, cls.ctypes.data_as(ctypes.c_void_p),
                                         sd.ctypes.data_as(ctypes.c_void_p), cls.size, steps, temperature,
                                         grids.ctypes.data_as(ctypes.c_void_p),
                                         imgs.ctypes.data_as(ctypes.c_void_p)))
        return grids, imgs

    def named(self, name: str) -> np.ndarray:
        """A named node of the last forward (its values are current only if that forward ran
        with MG_DUMP_NAMED set in the environment), flat float32."""
        n = _check(lib().mgr_named(self.h, name.encode(), None, 0))
        out = np.empty(n, np.float32)
        _check(lib().mgr_named(self.h, name.encode(), out.ctypes.data_as(ctypes.c_void_p), n))
        return out

    def profile(self, on: bool = True):
        _check(lib().mgr_profile_enable(self.h, int(on)))

    def profile_report(self) -> list:
        buf = ctypes.create_string_buffer(8192)
        _check(lib().mgr_profile_report(self.h, buf, len(buf)))
        rows = []
        for line in buf.value.decode().splitlines():
            name, cnt, ms = line.rsplit(" ", 2)
            rows.append((name, int(cnt), float(ms)))
        return rows
