"""Transformer forward composed from the oracle's pinned primitives (TEST INFRASTRUCTURE ONLY).

Restates the reference graph of src/mg-transformer.cpp:32-111 node by node:
  x = LN(get_rows(token_embd, ids) + pos_embd[:S])                     (:41-48)
  per layer: q, k, v FC; flash attention on {D,S,H,B} views; merge heads (:59-85)
             x = LN(FC_o(a) + x); x = LN(FC_down(GELU(FC_up(x))) + x)   (:87-99)
  logits = LN(GELU(FC_proj(x))) token_embd^T + output.bias             (:102-110)
Each FC node uses the semantics of the reference kernel that runs it:
  * "f32"  — F32 weights: mg-cpu.cpp:48-72 (oracle.gemm_f32);
  * "int8" — Q8_0/Q4_K weights, int8-dot path: k_quantize_q8 + k_mul_mat_*_i8
             (mg-opencl.cpp:424-590; oracle.quantize_act_q8 + oracle.gemm_q_i8);
  * "deq"  — Q8_0/Q4_K weights, dequantize-then-F32 (mg-opencl.cpp:320-411;
             oracle.gemm_q_deq_f32).
Attention is the fp16-K/V variant (mg-opencl.cpp:859-937) when f16kv, else the F32 CPU one.
`Layers` exposes the pieces separately, so each can be applied to given input activations.
"""
from __future__ import annotations

import numpy as np

from . import (WTYPE_Q4_K, WTYPE_Q8_0, attention, gemm_f32, gemm_q_deq_f32, gemm_q_i8,
               get_rows, layernorm_affine, merge_heads, quantize, quantize_act_q8)

FC = ("attn_q", "attn_k", "attn_v", "attn_o", "ffn_up", "ffn_down")


class Layers:
    """The forward's pieces, each a function of its input activations (so a test can feed each
    piece the GPU's own input): embed, attention sublayer, MLP sublayer, head (LN output and
    logits). t: float tensors by GGUF name (FC weights before quantization)."""

    def __init__(self, t: dict, n_head: int, B: int, S: int, quant: str = "f32", algo: str = "int8",
                 f16kv: bool = True, eps: float = 1e-12):
        self.t, self.H, self.B, self.S = t, n_head, B, S
        self.E = t["token_embd.weight"].shape[1]
        self.D = self.E // n_head
        self.wt = {"q8_0": WTYPE_Q8_0, "q4_k": WTYPE_Q4_K}.get(quant)
        self.algo, self.f16kv, self.eps = algo, f16kv, eps
        self._wq = {}

    def fc(self, name, x, act=0, resid=None):
        t = self.t
        w, b = t[name + ".weight"], t[name + ".bias"]
        N, K = w.shape
        if self.wt is None:
            return gemm_f32(w, x, bias=b, act=act, resid=resid)
        if name not in self._wq:
            self._wq[name] = quantize(self.wt, w)
        wq = self._wq[name]
        if self.algo == "int8":
            qx, dx, _ = quantize_act_q8(x)
            return gemm_q_i8(self.wt, wq, N, K, qx, dx, bias=b, act=act, resid=resid)
        return gemm_q_deq_f32(self.wt, wq, N, K, x, bias=b, act=act, resid=resid)

    def ln(self, name, x):
        return layernorm_affine(x, self.t[name + ".weight"], self.t[name + ".bias"], self.eps)

    def embed(self, tokens):                                  # :41-48
        B, S, E = self.B, self.S, self.E
        x = get_rows(self.t["token_embd.weight"], tokens.reshape(-1))
        x = (x.reshape(B, S, E) + self.t["pos_embd.weight"][:S][None]).reshape(B * S, E).astype(np.float32)
        return self.ln("token_embd_norm", x)

    def attn(self, l, x):                                     # :59-92
        p = f"blk.{l}."
        B, S, E, D, H = self.B, self.S, self.E, self.D, self.H
        q, k, v = (self.fc(p + n, x) for n in ("attn_q", "attn_k", "attn_v"))
        scale = np.float32(1.0) / np.sqrt(np.float32(D))
        a = attention(q, k, v, (1, E, D, E * S), D, S, H, B, float(scale), self.f16kv)
        a = merge_heads(a, D, S, H, B).reshape(B * S, E)
        return self.ln(p + "attn_norm", self.fc(p + "attn_o", a, resid=x))

    def mlp(self, l, x):                                      # :94-99
        p = f"blk.{l}."
        f = self.fc(p + "ffn_up", x, act=1)
        return self.ln(p + "ffn_norm", self.fc(p + "ffn_down", f, resid=x))

    def head_norm(self, x):                                   # :102-106
        return self.ln("output_norm", self.fc("output_proj", x, act=1))

    def logits(self, h):                                      # :107-109
        return gemm_f32(self.t["token_embd.weight"], h, bias=self.t["output.bias"])


def transformer_forward(t: dict, n_layer: int, n_head: int, tokens: np.ndarray, quant: str = "f32",
                        algo: str = "int8", f16kv: bool = True, eps: float = 1e-12) -> np.ndarray:
    """t: float tensors by GGUF name (FC weights before quantization); tokens [B][S]."""
    B, S = tokens.shape
    L = Layers(t, n_head, B, S, quant, algo, f16kv, eps)
    x = L.embed(tokens)
    for l in range(n_layer):
        x = L.mlp(l, L.attn(l, x))
    return L.logits(L.head_norm(x)).reshape(B, S, -1)
