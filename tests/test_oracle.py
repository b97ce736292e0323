"""Pins for the CPU oracle (runs without a GPU).

Each check is chosen so that a plausible mistake in the oracle — a dropped term, a
wrong sign or index, a transposed operand, a wrong rounding mode — fails it:
golden bytes from the reference encoder, the reference's own CPU executor
(oracle/_ref/libmgref.so) where it was built, exhaustive/brute-force comparisons,
closed forms and error bounds.
"""
import os

import numpy as np
import pytest

import oracle
from oracle import ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz")
needs_ref = pytest.mark.skipif(not ref.available(), reason="oracle/_ref/libmgref.so not built")


# ---- binary16 -----------------------------------------------------------------------
def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    # dense coverage of the half range, ties and the subnormal/overflow edges
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 6.1035156e-05, 5.9604645e-08,
                     2.9802322e-08, 2.9802326e-08, 1.0 + 2**-11, 1.0 + 3 * 2**-11, -2.5e-8,
                     np.inf, -np.inf], np.float32)
    mid = (np.arange(-70000, 70000, 0.37)).astype(np.float32)
    tiny = (rng.standard_normal(200000) * 1e-5).astype(np.float32)
    x = np.concatenate([x, edge, mid, tiny])
    x = x[~np.isnan(x)]
    got = oracle.f32_to_f16_bits(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---- encoders: golden bytes from the reference encoder ------------------------------
def test_q8_0_encoder_matches_reference_bytes():
    g = np.load(GOLDEN)
    assert np.array_equal(oracle.quantize(oracle.WTYPE_Q8_0, g["q8_in"]), g["q8_out"])


def test_q4_k_encoder_matches_reference_bytes():
    g = np.load(GOLDEN)
    assert np.array_equal(oracle.quantize(oracle.WTYPE_Q4_K, g["q4_in"]), g["q4_out"])


# ---- decoders -------------------------------------------------------------------------
def test_q8_0_dequant_closed_form_and_bound():
    g = np.load(GOLDEN)
    w, wq = g["q8_in"], g["q8_out"]
    N, K = w.shape
    deq = oracle.dequant(oracle.WTYPE_Q8_0, wq, N, K)
    blk = wq.reshape(N, K // 32, 34)
    d16 = blk[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    q = blk[:, :, 2:].view(np.int8).astype(np.float32)
    assert np.array_equal(deq, (d16[..., None] * q).reshape(N, K))
    # round trip: |w - deq| <= d/2 + 127*|d - fp16(d)| per block (d = amax/127 in fp32)
    amax = np.abs(w.reshape(N, K // 32, 32)).max(-1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    bound = d / 2 * 1.0001 + 127 * np.abs(d - d16) + 1e-12
    err = np.abs(w - deq).reshape(N, K // 32, 32).max(-1)
    assert (err <= bound).all()


def test_q4_k_scale_min_unpack_exhaustive():
    # Pack every (sc, m) pair into the ggml 12-byte layout (high 2 bits of sub-blocks 4..7 in
    # bits 6-7 of bytes 0..7) and check the unpack returns it for every sub-block slot.
    for sc in range(64):
        for m in range(64):
            for j in range(8):
                s = np.zeros(12, np.uint8)
                if j < 4:
                    s[j] = sc
                    s[j + 4] = m
                else:
                    s[j + 4] = (sc & 0xF) | ((m & 0xF) << 4)
                    s[j - 4] = (sc >> 4) << 6
                    s[j] = (m >> 4) << 6
                assert oracle.q4k_scale_min(s, j) == (sc, m)


def test_q4_k_dequant_error_bound():
    g = np.load(GOLDEN)
    w, wq = g["q4_in"], g["q4_out"]
    N, K = w.shape
    deq = oracle.dequant(oracle.WTYPE_Q4_K, wq, N, K)
    # per sub-block error of the min/max quantizer: step/2 plus fp16 rounding of d/dmin and
    # 6-bit rounding of the scale and min (each bounded by d/2 and dmin/2 per unit of q)
    sub = w.reshape(N, K // 32, 32)
    rng_ = sub.max(-1) - np.minimum(sub.min(-1), 0)
    step = rng_ / 15.0
    err = np.abs(w - deq).reshape(N, K // 32, 32).max(-1)
    assert (err <= step * 1.6 + 0.02 * np.abs(sub).max(-1) + 1e-6).all()
    # random weights: relative RMS error small
    rel = np.sqrt(((w - deq) ** 2).mean()) / np.sqrt((w ** 2).mean())
    assert rel < 0.12


# ---- activation quantizer ---------------------------------------------------------------
def test_act_quant_ties_half_away_from_zero():
    x = np.zeros((2, 64), np.float32)
    x[0, 0] = 127.0                        # d = 1, id = 1
    x[0, 1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]
    qx, dx, sx = oracle.quantize_act_q8(x)
    assert dx[0, 0] == 1.0
    assert list(qx[0, 0:9]) == [127, 1, 2, 3, -1, -2, -3, 127, -127]
    assert dx[0, 1] == 0.0 and (qx[0, 32:] == 0).all()   # all-zero block
    assert dx[1].tolist() == [0.0, 0.0] and (qx[1] == 0).all()
    assert np.array_equal(sx, qx.reshape(2, 2, 32).astype(np.int32).sum(-1))


def test_act_quant_closed_form(rng):
    x = rng.standard_normal((33, 768)).astype(np.float32) * 3
    qx, dx, sx = oracle.quantize_act_q8(x)
    xb = x.reshape(33, 24, 32)
    amax = np.abs(xb).max(-1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    assert np.array_equal(dx, d)
    idv = (np.float32(1.0) / d).astype(np.float32)
    prod = (xb * idv[..., None]).astype(np.float32)
    want = np.where(prod >= 0, np.floor(prod + 0.5), -np.floor(-prod + 0.5))   # round half away
    assert np.array_equal(qx.reshape(33, 24, 32).astype(np.float32), want)
    assert np.abs(qx).max() <= 127


# ---- int32 block dots: exact brute force --------------------------------------------------
def _q8_ints(wq, N, K):
    return wq.reshape(N, K // 32, 34)[:, :, 2:].view(np.int8).astype(np.int64).reshape(N, K)


def _q4_nibbles(wq, N, K):
    sb = wq.reshape(N, K // 256, 144)[:, :, 16:].astype(np.int64)    # [N, nsb, 128]
    out = np.zeros((N, K // 256, 8, 32), np.int64)
    for j in range(8):
        byte = sb[:, :, (j // 2) * 32:(j // 2) * 32 + 32]
        out[:, :, j, :] = (byte >> 4) if j % 2 else (byte & 0xF)
    return out.reshape(N, K)


@pytest.mark.parametrize("wtype", [oracle.WTYPE_Q8_0, oracle.WTYPE_Q4_K])
def test_block_dots_brute_force(rng, wtype):
    M, N, K = 7, 9, 512
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq = oracle.quantize(wtype, w)
    qx = rng.integers(-127, 128, (M, K)).astype(np.int8)
    got = oracle.block_dots(wtype, wq, N, K, qx)
    wi = _q8_ints(wq, N, K) if wtype == oracle.WTYPE_Q8_0 else _q4_nibbles(wq, N, K)
    want = np.einsum("mtk,ntk->mnt", qx.astype(np.int64).reshape(M, K // 32, 32),
                     wi.reshape(N, K // 32, 32))
    assert np.array_equal(got, want)


# ---- int8-dot GEMMs ---------------------------------------------------------------------
def _block_scales(wtype, wq, N, K):
    """Per-(n, t) weight scale and min, decoded from the block bytes."""
    if wtype == oracle.WTYPE_Q8_0:
        d = wq.reshape(N, K // 32, 34)[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
        return d, np.zeros_like(d)
    sb = wq.reshape(N, K // 256, 144)
    d = sb[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dm = sb[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    sc = np.zeros((N, K // 256, 8))
    mn = np.zeros((N, K // 256, 8))
    for n in range(N):
        for s in range(K // 256):
            for j in range(8):
                a, b = oracle.q4k_scale_min(sb[n, s, 4:16], j)
                sc[n, s, j] = a * d[n, s]
                mn[n, s, j] = b * dm[n, s]
    return sc.reshape(N, K // 32), mn.reshape(N, K // 32)


@pytest.mark.parametrize("wtype", [oracle.WTYPE_Q8_0, oracle.WTYPE_Q4_K])
@pytest.mark.parametrize("act", [0, 1, 2])
def test_gemm_i8_float64_recompute(rng, wtype, act):
    M, N, K = 13, 24, 512
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    resid = rng.standard_normal((M, N)).astype(np.float32)
    wq = oracle.quantize(wtype, w)
    qx, dx, sx = oracle.quantize_act_q8(x)
    y = oracle.gemm_q_i8(wtype, wq, N, K, qx, dx, bias=bias, act=act, resid=resid)
    dots = oracle.block_dots(wtype, wq, N, K, qx).astype(np.float64)
    sc, mn = _block_scales(wtype, wq, N, K)
    acc = (dots * sc[None] * dx[:, None, :]).sum(-1) - (sx[:, None, :] * mn[None] * dx[:, None, :]).sum(-1)
    v = acc + bias[None]
    if act == 1:
        from scipy.special import erf
        v = 0.5 * v * (1 + erf(v / np.sqrt(2.0)))
    elif act == 2:
        v = v / (1 + np.exp(-v))
    v = v + resid
    assert np.abs(y - v).max() <= 1e-5 * np.abs(v).max()


@pytest.mark.parametrize("wtype", [oracle.WTYPE_Q8_0, oracle.WTYPE_Q4_K])
def test_gemm_i8_vs_dequant_f32_deviation(rng, wtype):
    """The int8-activation path deviates from dequantize-then-F32 by the per-32 activation
    quantization error only (documented ~6e-3 of max|y| for Q8_0 at these statistics)."""
    M, N, K = 64, 96, 768
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq = oracle.quantize(wtype, w) if wtype == oracle.WTYPE_Q8_0 else oracle.quantize(wtype, w)
    qx, dx, _ = oracle.quantize_act_q8(x)
    y8 = oracle.gemm_q_i8(wtype, wq, N, K, qx, dx)
    yf = oracle.gemm_q_deq_f32(wtype, wq, N, K, x)
    rel = np.abs(y8 - yf).max() / np.abs(yf).max()
    assert rel < 2e-2


# ---- F32 paths vs the reference CPU executor ---------------------------------------------
@needs_ref
@pytest.mark.parametrize("act", [0, 1, 2])
def test_gemm_f32_bitexact_vs_reference_cpu(rng, act):
    M, N, K = 17, 40, 96
    w = rng.standard_normal((N, K)).astype(np.float32) * 0.1
    x = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    r = rng.standard_normal((M, N)).astype(np.float32)
    for bias, resid in ((None, None), (b, None), (b, r), (None, r)):
        got = oracle.gemm_f32(w, x, bias=bias, act=act, resid=resid)
        want = ref.mul_mat(w, x, bias=bias, act=act, resid=resid)
        assert np.array_equal(got, want)


@needs_ref
def test_layernorm_bitexact_vs_reference_cpu(rng):
    x = (rng.standard_normal((37, 768)) * 2 + 0.5).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(768)).astype(np.float32)
    b = (0.1 * rng.standard_normal(768)).astype(np.float32)
    assert np.array_equal(oracle.layernorm_affine(x, g, b, 1e-12), ref.norm_affine(x, g, b, 1e-12))


@needs_ref
def test_attention_bitexact_vs_reference_cpu(rng):
    D, S, H, B = 48, 37, 4, 2
    q, k, v = (rng.standard_normal((B, S, H * D)).astype(np.float32) for _ in range(3))
    strides = [1, H * D, D, H * D * S]            # mg-opencl.cpp:1493-1496 for [B][S][H*D]
    got = oracle.attention(q, k, v, strides, D, S, H, B, 1 / np.sqrt(D), f16kv=False)
    want = ref.attention(q, k, v, D, S, H, B, np.float32(1 / np.sqrt(np.float32(D))))
    assert np.array_equal(got, want)


def test_attention_f16kv_is_f32_on_rounded_inputs(rng):
    D, S, H, B = 48, 33, 2, 1
    q, k, v = (rng.standard_normal((B, S, H * D)).astype(np.float32) for _ in range(3))
    st = [1, H * D, D, H * D * S]
    a = oracle.attention(q, k, v, st, D, S, H, B, 0.125, f16kv=True)
    r = [oracle.round_f16(t) for t in (q, k, v)]
    b = oracle.attention(*r, st, D, S, H, B, 0.125, f16kv=False)
    assert np.array_equal(a, b)
    # and it is a softmax-weighted average: textbook float64 attention agrees closely
    qq, kk, vv = (t.reshape(S, H, D).transpose(1, 0, 2).astype(np.float64) for t in r)
    s = qq @ kk.transpose(0, 2, 1) * 0.125
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    o = (p @ vv).reshape(-1)
    assert np.abs(a - o).max() < 1e-5


def test_get_rows_and_merge(rng):
    a = rng.standard_normal((10, 6)).astype(np.float32)
    ids = np.array([3, -1, 0, 9, -10], np.int32)
    got = oracle.get_rows(a, ids)
    assert np.array_equal(got, a[[3, 9, 0, 9, 0]])
    D, S, H, B = 4, 3, 5, 2
    t = rng.standard_normal(D * S * H * B).astype(np.float32)
    m = oracle.merge_heads(t, D, S, H, B)
    assert np.array_equal(m, t.reshape(B, H, S, D).transpose(0, 2, 1, 3).reshape(-1))
