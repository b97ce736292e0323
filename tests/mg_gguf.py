"""GGUF v3 writer and synthetic MaskGIT transformer models (TEST INFRASTRUCTURE).

Writes the layout the reference's converter produces (tools/convert_to_gguf.py:158-266):
`maskgit.*` metadata, tensor dims innermost-first (reversed numpy shape), FC weights as
F32 / Q8_0 / Q4_K blocks (quantized by the oracle's encoders, which are pinned to the
reference encoder's bytes), everything else F32, 32-byte aligned data.

Synthetic weights follow the benchmark's random-init recipe: FC weights ~N(0, 0.02), biases
~N(0, 0.01), embeddings ~N(0, 0.02), LayerNorm gamma ~ 1 + N(0, 0.02), beta ~N(0, 0.01).
"""
from __future__ import annotations

import numpy as np

import oracle

from edge_maskgit_amd.gguf import ALIGN, GGML_F32, GGML_Q4_K, GGML_Q8_0, write_gguf  # noqa: F401

FC_NAMES = ("attn_q", "attn_k", "attn_v", "attn_o", "ffn_up", "ffn_down")


def synthetic_model(n_layer: int = 2, quant: str = "f32", seed: int = 0, n_embd: int = 768,
                    n_head: int = 16, n_ffn: int = 3072, vocab: int = 2025, n_pos: int = 257):
    """Random-init MaskGIT transformer: returns (meta, float tensors dict, quant)."""
    rng = np.random.default_rng(seed)
    t = {}

    def nrm(shape, s):
        return (rng.standard_normal(shape) * s).astype(np.float32)

    t["token_embd.weight"] = nrm((vocab, n_embd), 0.02)
    t["pos_embd.weight"] = nrm((n_pos, n_embd), 0.02)
    t["token_embd_norm.weight"] = 1 + nrm(n_embd, 0.02)
    t["token_embd_norm.bias"] = nrm(n_embd, 0.01)
    for l in range(n_layer):
        p = f"blk.{l}."
        for nm in FC_NAMES:
            n_out = n_ffn if nm == "ffn_up" else n_embd
            n_in = n_ffn if nm == "ffn_down" else n_embd
            t[p + nm + ".weight"] = nrm((n_out, n_in), 0.02)
            t[p + nm + ".bias"] = nrm(n_out, 0.01)
        for nm in ("attn_norm", "ffn_norm"):
            t[p + nm + ".weight"] = 1 + nrm(n_embd, 0.02)
            t[p + nm + ".bias"] = nrm(n_embd, 0.01)
    t["output_proj.weight"] = nrm((n_embd, n_embd), 0.02)
    t["output_proj.bias"] = nrm(n_embd, 0.01)
    t["output_norm.weight"] = 1 + nrm(n_embd, 0.02)
    t["output_norm.bias"] = nrm(n_embd, 0.01)
    t["output.bias"] = nrm(vocab, 0.01)
    meta = [("general.architecture", "str", "maskgit"), ("general.name", "str", "synthetic"),
            ("general.alignment", "u32", ALIGN), ("maskgit.n_layer", "u32", n_layer),
            ("maskgit.n_head", "u32", n_head), ("maskgit.n_embd", "u32", n_embd),
            ("maskgit.n_ffn", "u32", n_ffn), ("maskgit.head_dim", "u32", n_embd // n_head),
            ("maskgit.vocab_size", "u32", vocab), ("maskgit.n_tokens", "u32", n_pos - 1),
            ("maskgit.n_positions", "u32", n_pos), ("maskgit.mask_token_id", "i32", vocab - 1),
            ("maskgit.layernorm_eps", "f32", 1e-12), ("maskgit.quant", "str", quant),
            ("maskgit.vqgan.codebook_size", "u32", 1024),
            ("maskgit.sampling.choice_temperature", "f32", 4.5)]
    return meta, t


def is_fc(name: str) -> bool:
    return name.endswith(tuple(n + ".weight" for n in FC_NAMES)) or name == "output_proj.weight"


def encode(tensors: dict, quant: str) -> list:
    """[(name, shape, ggml type, bytes)] with FC weights in the given format."""
    out = []
    for name, a in tensors.items():
        if quant in ("q8_0", "q4_k") and is_fc(name):
            wt = oracle.WTYPE_Q8_0 if quant == "q8_0" else oracle.WTYPE_Q4_K
            out.append((name, a.shape, GGML_Q8_0 if quant == "q8_0" else GGML_Q4_K,
                        oracle.quantize(wt, a).tobytes()))
        else:
            out.append((name, a.shape, GGML_F32, np.ascontiguousarray(a, np.float32).tobytes()))
    return out


def write_model(path: str, n_layer: int = 2, quant: str = "f32", seed: int = 0, n_pos: int = 257) -> dict:
    """Write a synthetic model; returns the float tensors (pre-quantization)."""
    meta, t = synthetic_model(n_layer, quant, seed, n_pos=n_pos)
    write_gguf(path, meta, encode(t, quant))
    return t


def tokens(rng, S: int, B: int, vocab: int = 2025, n_codes: int = 1024, mask_id: int = 2024) -> np.ndarray:
    """Token ids as MaskGIT feeds them: position 0 = class token 1024 + class, positions
    1..S-1 codebook ids with half replaced by the mask id (mg-generate.cpp:48-59)."""
    t = rng.integers(0, n_codes, (B, S)).astype(np.int32)
    t[:, 0] = 1024 + rng.integers(0, 1000, B)
    m = rng.random((B, S - 1)) < 0.5
    t[:, 1:][m] = mask_id
    return t


def vqgan_tensors(rng, E: int = 32, codebook: int = 64, filters: int = 32, mult=(1, 2), R: int = 1) -> dict:
    """Random decoder weights under the converter's names (tools/convert_to_gguf.py:216-226),
    numpy shapes (conv [OC][IC][KH][KW]); conv weights ~N(0, 1/fan_in) keep activations O(1)."""
    t = {}

    def conv(name, oc, ic, k, bias):
        t[name + ".weight"] = (rng.standard_normal((oc, ic, k, k)) / np.sqrt(ic * k * k)).astype(np.float32)
        if bias:
            t[name + ".bias"] = (0.05 * rng.standard_normal(oc)).astype(np.float32)

    def gn(name, c):
        t[name + ".weight"] = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
        t[name + ".bias"] = (0.1 * rng.standard_normal(c)).astype(np.float32)

    def block(p, cin, cout):
        gn(p + "norm0", cin)
        conv(p + "conv0", cout, cin, 3, False)
        gn(p + "norm1", cout)
        conv(p + "conv1", cout, cout, 3, False)
        if cin != cout:
            conv(p + "conv_res", cout, cout, 1, False)

    t["vqgan.quantizer.codebook.weight"] = rng.standard_normal((codebook, E)).astype(np.float32)
    width = filters * mult[-1]
    conv("vqgan.decoder.conv_in", width, E, 3, True)
    for l in range(R):
        block(f"vqgan.decoder.res_blocks.0.{l}.", width, width)
    for i in range(len(mult) - 1, -1, -1):
        j, out = len(mult) - i, filters * mult[i]
        for l in range(R):
            block(f"vqgan.decoder.res_blocks.{j}.{l}.", width, out)
            width = out
        if i > 0:
            conv(f"vqgan.decoder.res_blocks.{j}.{R + 1}", width, width, 3, True)
    gn("vqgan.decoder.norm_out", width)
    conv("vqgan.decoder.conv_out", 3, width, 3, True)
    return t


def write_vqgan_model(path: str, n_tokens: int = 16, E: int = 32, codebook: int = 64, filters: int = 32,
                      mult=(1, 2), R: int = 1, seed: int = 0) -> int:
    """A GGUF holding only a VQGAN decoder and its metadata; returns the image side."""
    rng = np.random.default_rng(seed)
    t = vqgan_tensors(rng, E, codebook, filters, mult, R)
    L = int(round(n_tokens ** 0.5))
    side = L * 2 ** (len(mult) - 1)
    meta = [("general.architecture", "str", "maskgit"), ("general.name", "str", "synthetic-vqgan"),
            ("general.alignment", "u32", ALIGN), ("maskgit.n_tokens", "u32", n_tokens),
            ("maskgit.resolution", "u32", side),
            ("maskgit.vqgan.codebook_size", "u32", codebook), ("maskgit.vqgan.embedding_dim", "u32", E),
            ("maskgit.vqgan.filters", "u32", filters), ("maskgit.vqgan.num_res_blocks", "u32", R),
            ("maskgit.vqgan.group_norm_groups", "u32", 32),
            ("maskgit.vqgan.channel_multipliers", "i32_array", list(mult))]
    write_gguf(path, meta, [(n, a.shape, GGML_F32, a.tobytes()) for n, a in t.items()])
    return side


def write_maskgit_model(path: str, n_layer: int = 2, quant: str = "q8_0", seed: int = 0, n_pos: int = 17,
                        E: int = 32, filters: int = 32, mult=(1, 2), R: int = 1) -> tuple:
    """transformer and VQGAN decoder in one GGUF, as the reference's converter writes a model
    (tools/convert_to_gguf.py:158-266); returns (transformer tensors, decoder tensors)."""
    meta, t = synthetic_model(n_layer, quant, seed, n_pos=n_pos)
    v = vqgan_tensors(np.random.default_rng(seed + 1), E, 1024, filters, mult, R)
    L = int(round((n_pos - 1) ** 0.5))
    meta = meta + [("maskgit.resolution", "u32", L * 2 ** (len(mult) - 1)),
                   ("maskgit.vqgan.embedding_dim", "u32", E), ("maskgit.vqgan.filters", "u32", filters),
                   ("maskgit.vqgan.num_res_blocks", "u32", R), ("maskgit.vqgan.group_norm_groups", "u32", 32),
                   ("maskgit.vqgan.channel_multipliers", "i32_array", list(mult))]
    write_gguf(path, meta, encode(t, quant) + [(n, a.shape, GGML_F32, a.tobytes()) for n, a in v.items()])
    return t, v
