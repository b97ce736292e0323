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
"""
from __future__ import annotations

import numpy as np

from . import (WTYPE_Q4_K, WTYPE_Q8_0, attention, gemm_f32, gemm_q_deq_f32, gemm_q_i8,
               get_rows, layernorm_affine, merge_heads, quantize, quantize_act_q8)

FC = ("attn_q", "attn_k", "attn_v", "attn_o", "ffn_up", "ffn_down")


def transformer_forward(t: dict, n_layer: int, n_head: int, tokens: np.ndarray, quant: str = "f32",
                        algo: str = "int8", f16kv: bool = True, eps: float = 1e-12) -> np.ndarray:
    """t: float tensors by GGUF name (FC weights before quantization); tokens [B][S]."""
    B, S = tokens.shape
    E = t["token_embd.weight"].shape[1]
    D = E // n_head
    wt = {"q8_0": WTYPE_Q8_0, "q4_k": WTYPE_Q4_K}.get(quant)

    def fc(name, x, act=0, resid=None):
        w, b = t[name + ".weight"], t[name + ".bias"]
        N, K = w.shape
        if wt is None:
            return gemm_f32(w, x, bias=b, act=act, resid=resid)
        wq = quantize(wt, w)
        if algo == "int8":
            qx, dx, _ = quantize_act_q8(x)
            return gemm_q_i8(wt, wq, N, K, qx, dx, bias=b, act=act, resid=resid)
        return gemm_q_deq_f32(wt, wq, N, K, x, bias=b, act=act, resid=resid)

    def ln(name, x):
        return layernorm_affine(x, t[name + ".weight"], t[name + ".bias"], eps)

    x = get_rows(t["token_embd.weight"], tokens.reshape(-1))
    x = (x.reshape(B, S, E) + t["pos_embd.weight"][:S][None]).reshape(B * S, E).astype(np.float32)
    x = ln("token_embd_norm", x)
    scale = np.float32(1.0) / np.sqrt(np.float32(D))
    st = (1, E, D, E * S)
    for l in range(n_layer):
        p = f"blk.{l}."
        q, k, v = (fc(p + n, x) for n in ("attn_q", "attn_k", "attn_v"))
        a = attention(q, k, v, st, D, S, n_head, B, float(scale), f16kv)
        a = merge_heads(a, D, S, n_head, B).reshape(B * S, E)
        x = ln(p + "attn_norm", fc(p + "attn_o", a, resid=x))
        f = fc(p + "ffn_up", x, act=1)
        x = ln(p + "ffn_norm", fc(p + "ffn_down", f, resid=x))
    h = ln("output_norm", fc("output_proj", x, act=1))
    logits = gemm_f32(t["token_embd.weight"], h, bias=t["output.bias"])
    return logits.reshape(B, S, -1)
