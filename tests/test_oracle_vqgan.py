"""The VQGAN oracle (oracle/vqgan.py) pinned, and this project's decoder graph checked against
the reference builder's (host only, no GPU).

  * closed forms: a delta kernel copies (or, with stride 2, subsamples) the image; a 1x1 conv is
    a channel matmul; GroupNorm gives zero mean and unit variance per group, and its fused node
    with gamma = 1, beta = 0 is SiLU of the plain node; upscale by 1 is the identity;
  * the reference's own CPU executor (oracle/_ref/libmgref.so): conv within the float32
    summation error, GroupNorm bit-exact in >= 99% of the values and within 2 ulp (float64 sums
    in another order), the fused node within 1e-6 * max, upscale exact, and the whole decoder on
    small synthetic models;
  * build_vqgan_decoder (include/mg-vqgan.hpp) emits the reference builder's graph node for node
    (op, shape, strides, parameters, sources), on small models and at the production size;
  * the int8 conv oracle (oracle.conv_quant_w / conv2d_i8): where every block quantizes exactly it
    equals the reference CPU fp32 conv bit for bit; a vectorized restatement of the 32-block
    grouping gives the same bits; power-of-two input scaling is exact; and it stays within the
    quantization error of the fp32 conv.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle
from oracle import ref
from oracle import vqgan as ov
from tests import mg_gguf

needs_ref = pytest.mark.skipif(not ref.available(), reason="oracle/_ref/libmgref.so not built (needs /root/reference)")
HARNESS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_build", "libgraph_harness.so")

SMALL = [dict(n_tokens=16, E=32, codebook=64, filters=32, mult=(1, 2), R=1),
         dict(n_tokens=64, E=32, codebook=48, filters=32, mult=(1, 1, 2), R=2)]
FULL = dict(n_tokens=256, E=256, codebook=1024, filters=128, mult=(1, 1, 2, 2, 4), R=2)


def test_conv2d_closed_forms():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 5, 9, 7)).astype(np.float32)
    delta = np.zeros((5, 5, 3, 3), np.float32)
    for c in range(5):
        delta[c, c, 1, 1] = 1
    assert np.array_equal(ov.conv2d(x, delta, 1, 1), x)
    assert np.array_equal(ov.conv2d(x, delta, 2, 1), x[:, :, ::2, ::2])
    w = rng.standard_normal((6, 5, 1, 1)).astype(np.float32)
    want = np.einsum("oc,nchw->nohw", w[:, :, 0, 0].astype(np.float64), x.astype(np.float64)).astype(np.float32)
    assert np.array_equal(ov.conv2d(x, w, 1, 0), want)
    # a kernel that reads only its top-left tap shifts the padded image by one pixel
    tl = np.zeros((5, 5, 3, 3), np.float32)
    for c in range(5):
        tl[c, c, 0, 0] = 1
    y = ov.conv2d(x, tl, 1, 1)
    assert np.array_equal(y[:, :, 1:, 1:], x[:, :, :-1, :-1]) and not y[:, :, 0, :].any() and not y[:, :, :, 0].any()


def test_group_norm_closed_forms():
    rng = np.random.default_rng(1)
    x = (3 * rng.standard_normal((2, 64, 6, 5)) + 2).astype(np.float32)
    y = ov.group_norm(x, 32, 1e-5).astype(np.float64).reshape(2, 32, -1)
    assert np.abs(y.mean(axis=2)).max() < 1e-5
    assert np.abs(y.var(axis=2) - 1).max() < 1e-4
    one, zero = np.ones(64, np.float32), np.zeros(64, np.float32)
    plain = ov.group_norm(x, 32, 1e-5)
    fused = ov.group_norm(x, 32, 1e-5, one, zero)
    assert np.array_equal(fused, plain / (np.float32(1) + np.exp(-plain)))
    assert np.array_equal(ov.upscale(x, 1), x)


@needs_ref
@pytest.mark.parametrize("shape,k,stride,pad", [((1, 3, 8, 8), 3, 1, 1), ((2, 16, 9, 7), 3, 2, 1),
                                                 ((1, 64, 12, 12), 1, 1, 0), ((1, 4, 6, 6), 5, 1, 2)])
def test_conv2d_vs_reference_cpu(shape, k, stride, pad):
    rng = np.random.default_rng(sum(shape) + k)
    x = rng.standard_normal(shape).astype(np.float32)
    ker = (rng.standard_normal((11, shape[1], k, k)) / np.sqrt(shape[1] * k * k)).astype(np.float32)
    want = ref.conv2d(x, ker, stride, pad)
    got = ov.conv2d(x, ker, stride, pad)
    assert got.shape == want.shape
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


@needs_ref
@pytest.mark.parametrize("shape,G", [((1, 64, 8, 8), 32), ((3, 6, 5, 3), 3), ((1, 128, 32, 32), 32)])
def test_group_norm_vs_reference_cpu(shape, G):
    rng = np.random.default_rng(shape[1] + G)
    x = (2 * rng.standard_normal(shape) + 0.5).astype(np.float32)
    want = ref.group_norm(x, G, 1e-5)
    got = ov.group_norm(x, G, 1e-5)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulp.max() <= 2 and (ulp == 0).mean() >= 0.99
    C = shape[1]
    gm = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    bt = (0.1 * rng.standard_normal(C)).astype(np.float32)
    want = ref.group_norm(x, G, 1e-5, gm, bt)
    got = ov.group_norm(x, G, 1e-5, gm, bt)
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


@needs_ref
def test_upscale_vs_reference_cpu():
    x = np.random.default_rng(2).standard_normal((2, 3, 5, 4)).astype(np.float32)
    for f in (1, 2, 3):
        assert np.array_equal(ov.upscale(x, f), ref.upscale(x, f))


@needs_ref
@pytest.mark.parametrize("cfg", SMALL, ids=["L4-two-levels", "L8-three-levels-R2"])
def test_decode_vs_reference_cpu(tmp_path, cfg):
    """the oracle's decoder composition against the reference decoder graph on its CPU executor"""
    path = str(tmp_path / "vq.gguf")
    side = mg_gguf.write_vqgan_model(path, seed=3, **cfg)
    rng = np.random.default_rng(4)
    t = mg_gguf.vqgan_tensors(np.random.default_rng(3), cfg["E"], cfg["codebook"], cfg["filters"], cfg["mult"], cfg["R"])
    for _ in range(2):
        grid = rng.integers(0, cfg["codebook"], cfg["n_tokens"]).astype(np.int32)
        want = ref.vqgan_decode(path, grid, side)
        got = ov.decode(t, grid[None], cfg["E"], cfg["filters"], cfg["mult"], cfg["R"])[0]
        assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def _our_sig(path, n_tokens, B=1):
    if not os.path.exists(HARNESS):
        pytest.fail(f"{HARNESS} missing: run __graft_entry__.build()")
    L = ctypes.CDLL(HARNESS)
    L.gh_vqgan_graph_sig.argtypes = [ctypes.c_char_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                     ctypes.c_char_p, ctypes.c_int64]
    L.gh_vqgan_graph_sig.restype = ctypes.c_int64
    L.gh_last_error.restype = ctypes.c_char_p
    n = L.gh_vqgan_graph_sig(path.encode(), n_tokens, B, 3 << 30, None, 0)
    if n < 0:
        raise RuntimeError(L.gh_last_error().decode())
    buf = ctypes.create_string_buffer(n + 1)
    L.gh_vqgan_graph_sig(path.encode(), n_tokens, B, 3 << 30, buf, n + 1)
    return buf.value.decode()


@needs_ref
@pytest.mark.parametrize("cfg", SMALL + [FULL], ids=["L4", "L8-R2", "production"])
def test_decoder_graph_matches_reference_builder(tmp_path, cfg):
    path = str(tmp_path / "vq.gguf")
    mg_gguf.write_vqgan_model(path, seed=0, **cfg)
    ours = _our_sig(path, cfg["n_tokens"])
    theirs = ref.vqgan_graph_sig(path, cfg["n_tokens"], 3 << 30)
    assert ours.count("\n") > 10
    assert ours == theirs
    # B grids: the same nodes, each carrying the batch in its outermost dimension
    batched = _our_sig(path, cfg["n_tokens"], B=3)
    assert batched.count("\n") == ours.count("\n")


def test_decoder_rejects_non_square_grid(tmp_path):
    path = str(tmp_path / "vq.gguf")
    mg_gguf.write_vqgan_model(path, seed=0, **SMALL[0])
    with pytest.raises(RuntimeError, match="square"):
        _our_sig(path, 15)


# ---- the int8 conv of the reference's integer-dot devices (mg-opencl.cpp:598-664) ----

def _exact_i8_case(rng, N, IC, IH, IW, OC, k):
    """inputs +-127/128 and weights q * 2^-7 with a +-127 in every (channel, 32-block): every
    block of both operands quantizes exactly (d = 1/128 resp. 2^-7), and every partial sum is a
    multiple of 2^-14 below 2^10, so the int8 conv must equal the fp32 conv bit for bit"""
    x = (rng.choice([-1.0, 1.0], (N, IC, IH, IW)) * (127 / 128)).astype(np.float32)
    K = IC * k * k
    q = rng.integers(-127, 128, (OC, K))
    for b in range(0, K, 32):
        q[:, b] = rng.choice([-127, 127], OC)
    return x, (q * 2.0 ** -7).astype(np.float32).reshape(OC, IC, k, k), q


@pytest.mark.parametrize("N,IC,IH,IW,OC,k,stride,pad", [(2, 8, 7, 9, 5, 3, 1, 1), (1, 32, 6, 6, 4, 3, 2, 1),
                                                      (1, 64, 5, 4, 3, 1, 1, 0), (1, 5, 6, 5, 2, 3, 1, 2)])
def test_conv_i8_exact_quantization_closed_form(N, IC, IH, IW, OC, k, stride, pad):
    rng = np.random.default_rng(IC * 7 + OC)
    x, ker, q = _exact_i8_case(rng, N, IC, IH, IW, OC, k)
    qw, dw = oracle.conv_quant_w(ker)
    K = IC * k * k
    assert np.array_equal(qw[:, :K], q) and not qw[:, K:].any() and np.all(dw == np.float32(2.0 ** -7))
    got = oracle.conv2d_i8(x, qw, dw, k, k, stride, pad)
    assert np.array_equal(got, ov.conv2d(x, ker, stride, pad))
    if ref.available():
        assert np.array_equal(got, ref.conv2d(x, ker, stride, pad))


def _round_away(v):
    v = v.astype(np.float64)
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def _i8_numpy(x, ker, stride, pad):
    """the int8 conv vectorized: im2col in the kernel's k order, [pixel][block][32] groups"""
    N, IC, IH, IW = x.shape
    OC, _, KH, KW = ker.shape
    OH, OW = (IH + 2 * pad - KH) // stride + 1, (IW + 2 * pad - KW) // stride + 1
    K = IC * KH * KW
    nb = (K + 31) // 32
    xp = np.zeros((N, IC, IH + 2 * pad, IW + 2 * pad), np.float32)
    xp[:, :, pad:pad + IH, pad:pad + IW] = x
    cols = np.zeros((N, OH * OW, nb * 32), np.float32)
    for ic in range(IC):
        for kh in range(KH):
            for kw in range(KW):
                patch = xp[:, ic, kh:kh + stride * (OH - 1) + 1:stride, kw:kw + stride * (OW - 1) + 1:stride]
                cols[:, :, (ic * KH + kh) * KW + kw] = patch.reshape(N, -1)
    w = np.zeros((OC, nb * 32), np.float32)
    w[:, :K] = ker.reshape(OC, K)

    def quant(a):
        blk = a.reshape(a.shape[:-1] + (nb, 32))
        d = np.abs(blk).max(-1) / np.float32(127)
        inv = np.where(d > 0, np.float32(1) / np.where(d > 0, d, 1), 0).astype(np.float32)
        return _round_away(blk * inv[..., None]).astype(np.int64), d.astype(np.float32)

    qx, dx = quant(cols)
    qw, dw = quant(w)
    idot = np.einsum("nmbi,obi->nmob", qx, qw).astype(np.float32)
    acc = np.zeros((N, OH * OW, OC), np.float32)
    for b in range(nb):
        acc = acc + (dx[:, :, None, b] * dw[None, None, :, b]) * idot[..., b]
    return acc.transpose(0, 2, 1).reshape(N, OC, OH, OW)


@pytest.mark.parametrize("N,IC,IH,IW,OC,k,stride,pad", [(2, 8, 7, 9, 5, 3, 1, 1), (1, 20, 6, 5, 7, 3, 2, 1),
                                                      (1, 48, 4, 4, 9, 1, 1, 0)])
def test_conv_i8_block_grouping_and_scaling(N, IC, IH, IW, OC, k, stride, pad):
    """wide per-channel magnitude differences make the 32-block grouping matter: the loop oracle
    equals the vectorized restatement bit for bit; inputs scaled by 4 give outputs scaled by 4
    exactly; the int8 result stays within the quantization error of the fp32 conv"""
    rng = np.random.default_rng(IC + OC + k)
    x = (rng.standard_normal((N, IC, IH, IW)) * (2.0 ** rng.integers(-4, 5, (1, IC, 1, 1)))).astype(np.float32)
    ker = (rng.standard_normal((OC, IC, k, k)) * (2.0 ** rng.integers(-3, 4, (OC, IC, 1, 1)))).astype(np.float32)
    qw, dw = oracle.conv_quant_w(ker)
    got = oracle.conv2d_i8(x, qw, dw, k, k, stride, pad)
    assert np.array_equal(got, _i8_numpy(x, ker, stride, pad))
    assert np.array_equal(oracle.conv2d_i8(4 * x, qw, dw, k, k, stride, pad), 4 * got)
    f32 = ov.conv2d(x, ker, stride, pad)
    assert np.abs(got - f32).max() <= 3e-2 * np.abs(f32).max()
