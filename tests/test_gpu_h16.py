"""GPU parity of the dequantize-fused fp16 FC path: mgh_pack_weights_f16, mgh_f32_to_f16,
mgh_gemm_h16 / mgh_gemm_h16_f32in (k_gemm_fc.hip: the tiled kernel and, for a few activation
rows, the skinny-M kernel).

Bars:
  * packed weights: the oracle's dequantization (pinned to the reference decoder) rounded to
    fp16, bit for bit; the activation rounding: numpy's IEEE round-to-nearest-even, bit for bit;
  * the GEMM itself: against a float64 product of the same fp16 operands (+ bias, activation,
    residual in float64), max|y - ref| <= 1e-5 * max|ref| — only the fp32 accumulation order
    differs, so a wrong index, a dropped K stage or a mis-summed split shows as O(1);
  * the path as a whole: within 1e-3 * max|y| of the reference's dequantize-then-F32 product on
    the fp32 activations (oracle.gemm_q_deq_f32 = mg-cpu.cpp:48-72 semantics);
  * repeated calls are bit-identical (split-K partials are summed in a fixed order).
"""
import numpy as np
import pytest
from scipy.special import erf

import edge_maskgit_amd as ema
import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = ema.Context(0)
    yield c
    c.close()


def _rel(y, ref):
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def _act64(v, act):
    if act == 1:
        return 0.5 * v * (1.0 + erf(v / np.sqrt(2.0)))
    if act == 2:
        return v / (1.0 + np.exp(-v))
    return v


def _pack16(ctx, wtype, wq, N, K):
    dW = ctx.upload(wq)
    dP = ctx.alloc(ema.packed_weight_bytes_f16(N, K))
    ctx.pack_weights_f16(wtype, dW, N, K, dP)
    ctx.free(dW)
    return dP


@pytest.mark.parametrize("wtype", [ema.WTYPE_Q8_0, ema.WTYPE_Q4_K])
@pytest.mark.parametrize("N,K", [(1, 256), (96, 512), (2304, 768), (768, 3072)])
def test_pack_f16_matches_oracle(ctx, wtype, N, K):
    print(f"pack_f16 wtype={wtype} N={N} K={K}", flush=True)
    rng = np.random.default_rng(N + K + wtype)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[0, :32] = 0.0
    wq = oracle.quantize(wtype, w)
    assert ema.packed_weight_bytes_f16(N, K) == 2 * N * K
    dP = _pack16(ctx, wtype, wq, N, K)
    got = ctx.download(dP, (N, K), np.float16)
    ctx.free(dP)
    want = oracle.dequant(wtype, wq, N, K).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_f32_to_f16_rounding(ctx):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(4096 * 8) * np.exp(rng.uniform(-20, 12, 4096 * 8))).astype(np.float32)
    x[:8] = [0.0, -0.0, 65504.0, 65520.0, 1e-8, -6.1e-5, np.float32(2049.0), np.float32(2051.0)]
    dX, dH = ctx.upload(x), ctx.alloc(x.size * 2)
    ctx.f32_to_f16(dX, x.size, dH)
    got = ctx.download(dH, x.shape, np.float16)
    ctx.free(dX)
    ctx.free(dH)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


# the first eight run the skinny-M kernel (k_gemv_fc: M <= 16, or M <= 32 with K <= 1024),
# the rest the tiled plans; the pairs (16 | 17, 32 | 33) sit on both sides of the switch and N = 132
# ends in a partial 16-row weight group
SHAPES = [(1, 4, 64), (7, 132, 256), (1, 2304, 768), (16, 3072, 768), (17, 2304, 768),
          (32, 768, 768), (16, 768, 3072), (24, 132, 768), (33, 768, 768), (17, 768, 3072),
          (65, 128, 768), (257, 3072, 768), (1025, 2304, 768),
          (1025, 768, 768), (1025, 768, 3072), (300, 256, 3072), (4097, 768, 3072),
          (4112, 3072, 768), (4500, 2304, 768), (6150, 2048, 2048), (2731, 1024, 2048)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("act,res", [(0, False), (1, False), (0, True), (2, True)])
def test_gemm_h16_vs_float64(ctx, M, N, K, act, res):
    print(f"gemm_h16 M={M} N={N} K={K} act={act} resid={res}", flush=True)
    rng = np.random.default_rng(M * 7 + N * 3 + K + act)
    w16 = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    x16 = rng.standard_normal((M, K)).astype(np.float16)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    resid = rng.standard_normal((M, N)).astype(np.float32) if res else None
    dW, dX, dB = ctx.upload(w16), ctx.upload(x16), ctx.upload(bias)
    dR = ctx.upload(resid) if res else None
    dY = ctx.alloc(M * N * 4)
    ctx.gemm_h16(dW, N, K, dX, M, dB, act, dR, dY)
    y = ctx.download(dY, (M, N), np.float32)
    ctx.gemm_h16(dW, N, K, dX, M, dB, act, dR, dY)
    y2 = ctx.download(dY, (M, N), np.float32)
    for t in (dW, dX, dB, dR, dY):
        if t is not None:
            ctx.free(t)
    ref = _act64(x16.astype(np.float64) @ w16.astype(np.float64).T + bias, act)
    if res:
        ref = ref + resid
    err = _rel(y, ref)
    print(f"  rel err vs float64 {err:.2e}")
    assert err <= 1e-5
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


def test_gemm_h16_split_k_sequence(ctx):
    """Split-K launches of different shapes back to back (4 splits, 2 splits, 4 again) share
    the context's workspace: the repeated shape gives the same bits, and each result meets the
    float64 bar."""
    rng = np.random.default_rng(11)
    shapes = [(257, 768, 3072, 1), (1025, 768, 3072, 0), (257, 768, 3072, 1)]
    bufs, outs = {}, []
    for M, N, K, act in shapes:
        print(f"split-K sequence M={M} N={N} K={K} act={act}", flush=True)
        if (M, N, K) not in bufs:
            w16 = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
            x16 = rng.standard_normal((M, K)).astype(np.float16)
            bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
            bufs[(M, N, K)] = (w16, x16, bias, ctx.upload(w16), ctx.upload(x16), ctx.upload(bias),
                               ctx.alloc(M * N * 4))
        w16, x16, bias, dW, dX, dB, dY = bufs[(M, N, K)]
        ctx.gemm_h16(dW, N, K, dX, M, dB, act, None, dY)
        y = ctx.download(dY, (M, N), np.float32)
        ref = _act64(x16.astype(np.float64) @ w16.astype(np.float64).T + bias, act)
        assert _rel(y, ref) <= 1e-5
        outs.append(y)
    for v in bufs.values():
        for t in v[3:]:
            ctx.free(t)
    assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))


@pytest.mark.parametrize("wtype", [ema.WTYPE_Q8_0, ema.WTYPE_Q4_K])
@pytest.mark.parametrize("M,N,K,act,res", [(257, 768, 768, 0, True), (1025, 3072, 768, 1, False),
                                           (1025, 768, 3072, 0, True), (64, 2304, 768, 0, False),
                                           (257, 768, 3072, 0, True), (3, 3072, 768, 1, False),
                                           (9, 768, 3072, 0, True)])
def test_gemm_h16_f32in_vs_dequant_f32(ctx, wtype, M, N, K, act, res):
    print(f"gemm_h16_f32in wtype={wtype} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + N + K + wtype)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq = oracle.quantize(wtype, w)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    resid = rng.standard_normal((M, N)).astype(np.float32) if res else None
    dP = _pack16(ctx, wtype, wq, N, K)
    dX, dB, dY = ctx.upload(x), ctx.upload(bias), ctx.alloc(M * N * 4)
    dR = ctx.upload(resid) if res else None
    ctx.gemm_h16_f32in(dP, N, K, dX, M, dB, act, dR, dY)
    y = ctx.download(dY, (M, N), np.float32)
    for t in (dP, dX, dB, dR, dY):
        if t is not None:
            ctx.free(t)
    ref = oracle.gemm_q_deq_f32(wtype, wq, N, K, x, bias=bias, act=act, resid=resid)
    err = _rel(y, ref)
    print(f"  rel err vs dequantize-then-F32 {err:.2e}")
    assert err <= 1e-3


@pytest.mark.parametrize("M,N,K,act,exact", [(5, 768, 3072, 1, True), (20, 2304, 768, 0, True),
                                             (65, 128, 768, 0, True), (1025, 3072, 768, 1, True),
                                             (1025, 768, 3072, 0, True), (4097, 3072, 768, 2, True),
                                             (1025, 2304, 768, 1, False)])
def test_gemm_h16_f32in_equals_rounded_operand(ctx, M, N, K, act, exact):
    """The in-kernel fp32 -> fp16 rounding (XF32 variant) gives the same bits as rounding with
    mgh_f32_to_f16 first and running the fp16-operand kernel, where the tile plan is the same
    for both operand forms. At (1025, 2304, 768) the fp16 operand fits all its 64 x 64 tiles on
    the GPU at once and takes them, the fp32 one keeps 64 x 128 tiles: the same products summed
    in another order, so the bar there is fp32 summation-order agreement."""
    print(f"gemm_h16 f32in == f32_to_f16 + gemm_h16: M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + 3 * N + K)
    w16 = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    x = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    dW, dX, dB = ctx.upload(w16), ctx.upload(x), ctx.upload(bias)
    dH, dY1, dY2 = ctx.alloc(M * K * 2), ctx.alloc(M * N * 4), ctx.alloc(M * N * 4)
    ctx.gemm_h16_f32in(dW, N, K, dX, M, dB, act, None, dY1)
    ctx.f32_to_f16(dX, M * K, dH)
    ctx.gemm_h16(dW, N, K, dH, M, dB, act, None, dY2)
    y1, y2 = ctx.download(dY1, (M, N), np.float32), ctx.download(dY2, (M, N), np.float32)
    for t in (dW, dX, dB, dH, dY1, dY2):
        ctx.free(t)
    if exact:
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    else:
        assert np.abs(y1 - y2).max() <= 2e-6 * np.abs(y2).max()


@pytest.mark.parametrize("M,N,K,act", [(9, 3072, 768, 1), (257, 3072, 768, 1), (1025, 768, 3072, 0)])
def test_gemm_h16_y16_is_rounded_output(ctx, M, N, K, act):
    """The fp16-output variant stores exactly the fp32 result rounded to nearest fp16."""
    print(f"gemm_h16_y16 M={M} N={N} K={K} act={act}", flush=True)
    rng = np.random.default_rng(M + N + 7 * K)
    w16 = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    x16 = rng.standard_normal((M, K)).astype(np.float16)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    dW, dX, dB = ctx.upload(w16), ctx.upload(x16), ctx.upload(bias)
    dY, dH = ctx.alloc(M * N * 4), ctx.alloc(M * N * 2)
    ctx.gemm_h16(dW, N, K, dX, M, dB, act, None, dY)
    ctx.gemm_h16_y16(dW, N, K, dX, M, dB, act, None, dH)
    y, h = ctx.download(dY, (M, N), np.float32), ctx.download(dH, (M, N), np.float16)
    for t in (dW, dX, dB, dY, dH):
        ctx.free(t)
    assert np.array_equal(h.view(np.uint16), y.astype(np.float16).view(np.uint16))


def test_gemm_h16_rejects_bad_args(ctx):
    buf = ctx.alloc(1 << 20)
    for (N, K) in [(6, 64), (8, 96), (0, 64)]:
        with pytest.raises(ema.MghError):
            ctx.gemm_h16(buf, N, K, buf, 4, None, 0, None, buf)
    with pytest.raises(ema.MghError):
        ctx.gemm_h16(buf, 8, 64, buf, 4, None, 3, None, buf)
    with pytest.raises(ema.MghError):
        ctx.f32_to_f16(buf, 12, buf)
    ctx.free(buf)


# mgh_gemm_h16_ln: the first five split K (the reduce normalizes the rows: panel heights 1 and 8,
# a partial last panel, LayerNorm widths 256..2048), the rest run the LayerNorm kernel after the
# GEMM (no split, the skinny-M kernel, the long-K plan)
LN_SHAPES = [(257, 768, 3072), (1025, 768, 3072), (700, 2048, 3072), (300, 256, 3072), (200, 512, 2048),
             (257, 768, 768), (16, 768, 3072), (513, 2048, 1024), (4112, 768, 3072)]


@pytest.mark.parametrize("M,N,K", LN_SHAPES)
@pytest.mark.parametrize("emit", [0, 1, 2])
@pytest.mark.parametrize("act", [0, 1])
def test_gemm_h16_ln_equals_gemm_then_layernorm(ctx, M, N, K, emit, act):
    """mgh_gemm_h16_ln gives the bits of mgh_gemm_h16 followed by mgh_layernorm_affine on its
    output: y, the normalized rows and every emitted operand (with an activation the fused
    reduce is not used and the pair runs as two launches)."""
    res = M % 2 == 1
    print(f"gemm_h16_ln M={M} N={N} K={K} emit={emit} act={act} resid={res}", flush=True)
    rng = np.random.default_rng(M + N + K + 3 * emit + act)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    dP = _pack16(ctx, ema.WTYPE_Q8_0, oracle.quantize(ema.WTYPE_Q8_0, w), N, K)
    x16 = rng.standard_normal((M, K)).astype(np.float16)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.standard_normal(N)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(N)).astype(np.float32)
    dX, dB, dG, dBe = ctx.upload(x16), ctx.upload(bias), ctx.upload(gamma), ctx.upload(beta)
    dR = ctx.upload(rng.standard_normal((M, N)).astype(np.float32)) if res else None
    T = N // 32
    outs = []
    for mode in ("apart", "fused", "fused_no_y"):
        y, yl = ctx.alloc(M * N * 4), ctx.alloc(M * N * 4)
        c, dx, s4 = (ctx.alloc(M * N * 2), ctx.alloc(M * T * 4), ctx.alloc(M * T * 4)) if emit else (None, None, None)
        if mode == "fused":
            ctx.gemm_h16_ln(dP, N, K, dX, M, dB, act, dR, y, dG, dBe, 1e-5, yl, emit, c, dx, s4)
        elif mode == "fused_no_y":                # only the LayerNorm's outputs wanted (y NULL)
            ctx.fill_u32(y, 0x7FC00000, M * N)
            ctx.gemm_h16_ln(dP, N, K, dX, M, dB, act, dR, None, dG, dBe, 1e-5, yl, emit, c, dx, s4)
        else:
            ctx.gemm_h16(dP, N, K, dX, M, dB, act, dR, y)
            ctx.layernorm_affine(y, dG, dBe, M, N, 1e-5, yl, emit, c, dx, s4)
        o = [ctx.download(y, (M, N), np.float32).view(np.uint32), ctx.download(yl, (M, N), np.float32).view(np.uint32)]
        if mode == "fused_no_y":
            assert (o[0] == 0x7FC00000).all()     # y untouched
            o[0] = outs[0][0]
        if emit:
            o += [ctx.download(c, (M, N), np.float16).view(np.uint16), ctx.download(dx, (M, T), np.float32).view(np.uint32),
                  ctx.download(s4, (M, T), np.uint32)]
        outs.append(o)
        for t in (y, yl, c, dx, s4):
            if t is not None:
                ctx.free(t)
    for t in (dP, dX, dB, dG, dBe, dR):
        if t is not None:
            ctx.free(t)
    for o in outs[1:]:
        for a, b in zip(outs[0], o):
            assert np.array_equal(a, b)
    assert np.isfinite(outs[1][1].view(np.float32)).all()


def test_gemm_h16_ln_rejects_bad_arguments(ctx):
    """mgh_gemm_h16_ln: LayerNorm widths other than multiples of 256 up to 2048 are
    unsupported, emit modes are 0..2 and an emitted operand needs its buffers."""
    N, K, M = 768, 768, 4
    w, x, y = ctx.alloc(2048 * K * 2), ctx.alloc(M * K * 2), ctx.alloc(M * 2048 * 4)
    g, b, yl = ctx.alloc(2048 * 4), ctx.alloc(2048 * 4), ctx.alloc(M * 2048 * 4)
    for bad_n in (384, 2304):
        with pytest.raises(ema.MghError):
            ctx.gemm_h16_ln(w, bad_n, K, x, M, None, 0, None, y, g, b, 1e-5, yl)
    with pytest.raises(ema.MghError):
        ctx.gemm_h16_ln(w, N, K, x, M, None, 0, None, y, g, b, 1e-5, yl, emit=3)
    with pytest.raises(ema.MghError):
        ctx.gemm_h16_ln(w, N, K, x, M, None, 0, None, y, g, b, 1e-5, yl, emit=2)      # no codes buffer
    with pytest.raises(ema.MghError):
        ctx.gemm_h16_ln(w, N, K, x, M, None, 0, None, y, None, b, 1e-5, yl)            # no gamma
    for t in (w, x, y, g, b, yl):
        ctx.free(t)
