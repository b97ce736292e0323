"""Host side of the transformer runtime, no GPU needed: the GGUF writer/reader pair, the
forward graph's structure, and the oracle forward pinned against the reference's own CPU
executor (oracle/_ref, built from the reference sources)."""
import os

import numpy as np
import pytest

import oracle
from oracle import forward as ofwd
from oracle import ref
from tests import mg_gguf
from edge_maskgit_amd import runtime as rt


@pytest.fixture(scope="module")
def f32_model(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("gguf") / "tiny_f32.gguf")
    t = mg_gguf.write_model(p, n_layer=2, quant="f32", seed=1)
    return p, t


def test_gguf_info(f32_model):
    path, t = f32_model
    info = rt.gguf_info(path)
    assert info["n_layer"] == 2 and info["n_head"] == 16 and info["n_embd"] == 768
    assert info["head_dim"] == 48 and info["vocab_size"] == 2025 and info["n_positions"] == 257
    assert info["mask_token_id"] == 2024
    assert info["n_tensors"] == len(t) == 4 + 2 * 16 + 5


@pytest.mark.parametrize("quant", ["q8_0", "q4_k"])
def test_gguf_info_quantized(tmp_path, quant):
    p = str(tmp_path / f"tiny_{quant}.gguf")
    mg_gguf.write_model(p, n_layer=1, quant=quant, seed=2)
    assert rt.gguf_info(p)["n_layer"] == 1
    # the quantized FC blocks occupy exactly the block-format bytes
    size = os.path.getsize(p)
    assert size < 40e6


def test_forward_graph_structure(f32_model):
    """build_transformer's node set for 2 layers (mg-transformer.cpp:32-111), by op code:
    MulMat = 6 per layer + head proj + logits; Norm = embedding + 2 per layer + head;
    FlashAttention / Cont = 1 per layer; Reshape = 3 head splits + 1 merge per layer;
    Permute = 3 + 1 per layer; GetRows = Add = 1."""
    path, _ = f32_model
    n, c = rt.graph_stats(path, 257, 2)
    OP = dict(Add=1, MulMat=4, GetRows=5, Norm=7, FlashAttention=13, Reshape=14, Permute=16, Cont=17)
    L = 2
    assert c[OP["MulMat"]] == 6 * L + 2
    assert c[OP["Norm"]] == 1 + 2 * L + 1
    assert c[OP["FlashAttention"]] == L and c[OP["Cont"]] == L
    assert c[OP["Reshape"]] == 4 * L and c[OP["Permute"]] == 4 * L
    assert c[OP["GetRows"]] == 1 and c[OP["Add"]] == 1
    assert n == int(c.sum())


def test_forward_graph_structure_unfused_attention(f32_model, monkeypatch):
    """MG_NO_FLASH_ATTN (mg-transformer.cpp:55, 75-81): per layer the attention is
    mul_mat(k, q) -> soft_max -> mul_mat(permute(v), scores), no FlashAttention node."""
    path, _ = f32_model
    monkeypatch.setenv("MG_NO_FLASH_ATTN", "1")
    n, c = rt.graph_stats(path, 257, 1)
    OP = dict(MulMat=4, SoftMax=6, FlashAttention=13, Permute=16, Cont=17)
    L = 2
    assert c[OP["MulMat"]] == 8 * L + 2
    assert c[OP["SoftMax"]] == L and c[OP["FlashAttention"]] == 0
    assert c[OP["Permute"]] == 5 * L and c[OP["Cont"]] == L
    assert n == int(c.sum())


def test_sequence_longer_than_position_table_rejected(f32_model):
    """the position table is viewed as its first S rows: S beyond its 257 rows is an error, not
    a read past the tensor"""
    path, _ = f32_model
    rt.graph_stats(path, 257, 1)
    with pytest.raises(Exception, match="position table"):
        rt.graph_stats(path, 258, 1)


def test_gguf_rejects_malformed_files(f32_model, tmp_path):
    """truncated data, an impossible tensor count and a zero dimension are reported, never
    mapped past the end of the file"""
    import struct
    from edge_maskgit_amd import MghError
    path, _ = f32_model
    raw = open(path, "rb").read()
    cut = tmp_path / "cut.gguf"
    cut.write_bytes(raw[: len(raw) - 4096])
    with pytest.raises(MghError, match="past EOF"):
        rt.gguf_info(str(cut))
    many = tmp_path / "many.gguf"
    many.write_bytes(raw[:8] + struct.pack("<Q", 1 << 60) + raw[16:])
    with pytest.raises(MghError, match="tensor count"):
        rt.gguf_info(str(many))


def test_graph_api_semantics():
    """build_forward restarts the node list, contiguity is strict on size-1 dimensions, as the
    reference's graph core (checks in tests/graph_harness.cpp, host only)"""
    import ctypes
    lib = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_build", "libgraph_harness.so")
    if not os.path.exists(lib):
        pytest.fail(f"{lib} missing: run __graft_entry__.build()")
    assert ctypes.CDLL(lib).gh_api_checks() == 0


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref/libmgref.so not built (needs /root/reference)")
def test_oracle_forward_matches_reference_cpu(f32_model):
    """The oracle forward (F32 weights, F32 attention) against the reference's own CPU
    executor on the same GGUF file: the reference loader reads our writer's file, and the
    composition of pinned primitives reproduces its logits."""
    path, t = f32_model
    rng = np.random.default_rng(5)
    tok = mg_gguf.tokens(rng, 17, 1)
    want = ref.transformer_forward(path, tok, 2025)
    got = ofwd.transformer_forward(t, 2, 16, tok, quant="f32", f16kv=False)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err <= 1e-5, err
