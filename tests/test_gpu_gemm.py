"""GPU parity: activation quantizer, MFMA block dots and quantized FC GEMMs vs the oracle.

Bars (the path's acceptance bars):
  * qx / dx / sx of the quantizer: bit-exact.
  * int32 block dot products of the production GEMM's MFMA path: bit-exact.
  * fp32 GEMM outputs: max|y - y_oracle| <= 1e-3 * max|y_oracle| against the int8-dot oracle
    with identical activation quantization (observed error is ~1e-6 relative).
The deviation of the int8 path from dequantize-then-F32 is reported, not gated by 1e-3
(it is the activation-quantization error of the reference's own int8 path).
"""
import numpy as np
import pytest

import edge_maskgit_amd as ema
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-3


@pytest.fixture(scope="module")
def ctx():
    c = ema.Context(0)
    yield c
    c.close()


def _rel_err(y, ref):
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def _weights(rng, wtype, N, K, scale=0.02):
    w = (rng.standard_normal((N, K)) * scale).astype(np.float32)
    return w, oracle.quantize(wtype, w)


# ---- activation quantizer -------------------------------------------------------------
@pytest.mark.parametrize("M,K", [(1, 32), (3, 64), (257, 768), (1025, 3072)])
def test_quantize_act_bitexact(ctx, M, K):
    rng = np.random.default_rng(M * 7 + K)
    x = rng.standard_normal((M, K)).astype(np.float32) * 2
    x[0, :32] = 0.0                         # zero block
    if K >= 64:
        x[0, 32] = 127.0                    # d = 1: exact .5 ties must round away from zero
        x[0, 33:39] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5]
    print(f"quantize_act M={M} K={K}", flush=True)
    qx_r, dx_r, sx_r = oracle.quantize_act_q8(x)
    dX = ctx.upload(x)
    dq, dd, ds = ctx.alloc(M * K), ctx.alloc(M * K // 32 * 4), ctx.alloc(M * K // 32 * 4)
    ctx.quantize_act_q8(dX, M, K, dq, dd, ds)
    qx = ctx.download(dq, (M, K), np.int8)
    dx = ctx.download(dd, (M, K // 32), np.float32)
    sx = ctx.download(ds, (M, K // 32), np.int32)
    assert np.array_equal(dx.view(np.uint32), dx_r.view(np.uint32))
    assert np.array_equal(qx, qx_r)
    assert np.array_equal(sx, sx_r)
    for b in (dX, dq, dd, ds):
        ctx.free(b)


# ---- MFMA block dots -----------------------------------------------------------------
DOT_SHAPES = [(1, 32, 256), (33, 70, 512), (130, 200, 768), (257, 3072, 768)]


@pytest.mark.parametrize("wtype", [ema.WTYPE_Q8_0, ema.WTYPE_Q4_K])
@pytest.mark.parametrize("M,N,K", DOT_SHAPES)
def test_block_dots_bitexact(ctx, wtype, M, N, K):
    rng = np.random.default_rng(M + N + K + wtype)
    print(f"block_dots wtype={wtype} M={M} N={N} K={K}", flush=True)
    _, wq = _weights(rng, wtype, N, K)
    qx = rng.integers(-127, 128, (M, K)).astype(np.int8)
    qx[0, :32] = 127
    qx[-1, -32:] = -127
    ref = oracle.block_dots(wtype, wq, N, K, qx)
    dW, dQ = ctx.upload(wq), ctx.upload(qx)
    dO = ctx.alloc(M * N * (K // 32) * 4)
    ctx.debug_block_dots(wtype, dW, N, K, dQ, M, dO)
    got = ctx.download(dO, (M, N, K // 32), np.int32)
    assert np.array_equal(got, ref)
    for b in (dW, dQ, dO):
        ctx.free(b)


# ---- GEMMs ----------------------------------------------------------------------------
GEMM_SHAPES = [(1, 64, 256), (5, 96, 512), (70, 130, 768), (257, 3072, 768), (129, 768, 3072)]


def _run_gemm(ctx, wtype, M, N, K, act, use_bias, use_resid, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w, wq = _weights(rng, wtype, N, K)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32) if use_bias else None
    resid = rng.standard_normal((M, N)).astype(np.float32) if use_resid else None
    dW, dX = ctx.upload(wq), ctx.upload(x)
    dB = ctx.upload(bias) if use_bias else None
    dR = ctx.upload(resid) if use_resid else None
    dY = ctx.alloc(M * N * 4)
    ctx.gemm_q_f32in(ema.ALGO_INT8, wtype, dW, N, K, dX, M, dB, act, dR, dY)
    y = ctx.download(dY, (M, N), np.float32)
    for b in (dW, dX, dB, dR, dY):
        if b is not None:
            ctx.free(b)
    qx, dx, _ = oracle.quantize_act_q8(x)
    ref = oracle.gemm_q_i8(wtype, wq, N, K, qx, dx, bias=bias, act=act, resid=resid)
    return x, wq, bias, resid, y, ref


@pytest.mark.parametrize("wtype", [ema.WTYPE_Q8_0, ema.WTYPE_Q4_K])
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_gemm_int8_vs_oracle(ctx, wtype, M, N, K):
    print(f"gemm_int8 wtype={wtype} M={M} N={N} K={K}", flush=True)
    _, _, _, _, y, ref = _run_gemm(ctx, wtype, M, N, K, 0, True, False, seed=M * N + K)
    err = _rel_err(y, ref)
    print(f"  rel err vs int8 oracle {err:.2e}")
    assert err <= TOL


@pytest.mark.parametrize("wtype", [ema.WTYPE_Q8_0, ema.WTYPE_Q4_K])
@pytest.mark.parametrize("act,use_bias,use_resid", [(0, False, False), (0, True, True),
                                                    (1, True, False), (2, True, True),
                                                    (1, False, True)])
def test_gemm_int8_epilogues(ctx, wtype, act, use_bias, use_resid):
    M, N, K = 77, 200, 512
    print(f"gemm_epilogue wtype={wtype} act={act} bias={use_bias} resid={use_resid}", flush=True)
    _, _, _, _, y, ref = _run_gemm(ctx, wtype, M, N, K, act, use_bias, use_resid, seed=act + 10)
    assert _rel_err(y, ref) <= TOL


@pytest.mark.parametrize("wtype", [ema.WTYPE_Q8_0, ema.WTYPE_Q4_K])
def test_gemm_int8_deviation_from_dequant_f32(ctx, wtype):
    """Report (and loosely bound) the int8 path's distance from dequantize-then-F32."""
    M, N, K = 257, 3072, 768
    x, wq, bias, _, y, _ = _run_gemm(ctx, wtype, M, N, K, 0, True, False, seed=99)
    yf = oracle.gemm_q_deq_f32(wtype, wq, N, K, x, bias=bias)
    err = _rel_err(y, yf)
    print(f"  int8 path vs dequant-F32: {err:.2e} of max|y| (wtype {wtype})")
    assert err < 2e-2


@pytest.mark.parametrize("wtype,M,N,K", [(ema.WTYPE_Q8_0, 4097, 3072, 768),
                                         (ema.WTYPE_Q8_0, 4097, 768, 3072),
                                         (ema.WTYPE_Q4_K, 4097, 2304, 768),
                                         (ema.WTYPE_Q4_K, 4112, 768, 3072)])
def test_gemm_full_size_row_sample(ctx, wtype, M, N, K):
    """Full-size GEMMs (M = 4097): rows are independent, so check a random row sample of the full
    GPU result against the oracle evaluated on those rows only."""
    print(f"gemm_full wtype={wtype} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    _, wq = _weights(rng, wtype, N, K)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    resid = rng.standard_normal((M, N)).astype(np.float32)
    dW, dX, dB, dR = ctx.upload(wq), ctx.upload(x), ctx.upload(bias), ctx.upload(resid)
    dY = ctx.alloc(M * N * 4)
    ctx.gemm_q_f32in(ema.ALGO_INT8, wtype, dW, N, K, dX, M, dB, 1, dR, dY)
    y = ctx.download(dY, (M, N), np.float32)
    for b in (dW, dX, dB, dR, dY):
        ctx.free(b)
    rows = np.unique(np.concatenate([rng.choice(M, 48, replace=False), [0, M - 1]]))
    qx, dx, _ = oracle.quantize_act_q8(x[rows])
    ref = oracle.gemm_q_i8(wtype, wq, N, K, qx, dx, bias=bias, act=1, resid=resid[rows])
    assert np.isfinite(y).all()
    assert _rel_err(y[rows], ref) <= TOL


def test_gemm_rejects_bad_shapes(ctx):
    with pytest.raises(ema.MghError):
        ctx.gemm_q_f32in(ema.ALGO_INT8, ema.WTYPE_Q4_K, 1, 8, 128, 1, 4, None, 0, None, 1)
    with pytest.raises(ema.MghError):
        ctx.gemm_q_f32in(ema.ALGO_INT8, 3, 1, 8, 128, 1, 4, None, 0, None, 1)
    with pytest.raises(ema.MghError):
        ctx.gemm_q_f32in(ema.ALGO_INT8, ema.WTYPE_Q8_0, 1, 8, 96, 1, 4, None, 0, None, 1)
    # M == 0 is a no-op
    ctx.gemm_q_f32in(ema.ALGO_INT8, ema.WTYPE_Q8_0, 1, 8, 128, 1, 0, None, 0, None, 1)


def test_graph_replay_matches_eager(ctx):
    """A captured quantize+GEMM graph replayed several times, with eager work and syncs
    between replays, reproduces the eager result every time."""
    rng = np.random.default_rng(5)
    M, N, K = 300, 768, 768
    for wtype in (ema.WTYPE_Q8_0, ema.WTYPE_Q4_K):
        x = rng.standard_normal((M, K)).astype(np.float32)
        _, wq = _weights(rng, wtype, N, K)
        dW, dX, dY = ctx.upload(wq), ctx.upload(x), ctx.alloc(M * N * 4)
        dq, dd, ds = ctx.alloc(M * K), ctx.alloc(M * K // 32 * 4), ctx.alloc(M * K // 32 * 4)
        def step():
            ctx.quantize_act_q8(dX, M, K, dq, dd, ds)
            ctx.gemm_q(wtype, dW, N, K, dq, dd, ds, M, None, ema.ACT_GELU, None, dY)
        step()
        eager = ctx.download(dY, (M, N), np.float32)
        ctx.graph_begin()
        step()
        g = ctx.graph_end()
        junk = ctx.upload(np.zeros((M, N), np.float32))
        for rep in range(4):
            ctx.gemm_q(wtype, dW, N, K, dq, dd, ds, M, None, 0, None, junk)   # eager work between
            ctx.sync()
            g.launch()
            got = ctx.download(dY, (M, N), np.float32)
            assert np.array_equal(got, eager), f"replay {rep} differs"
        g.destroy()
        for b in (dW, dX, dY, dq, dd, ds, junk):
            ctx.free(b)


@pytest.mark.parametrize("wtype", [ema.WTYPE_Q8_0, ema.WTYPE_Q4_K])
@pytest.mark.parametrize("M,N,K", [(5, 96, 512), (257, 768, 768), (70, 130, 768), (33, 64, 3072)])
def test_gemm_q_int8_input_vs_oracle(ctx, wtype, M, N, K):
    """mgh_gemm_q on int8 codes given by the caller (the reference's qx/dx/sx layout)."""
    print(f"gemm_q int8-input wtype={wtype} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + 3 * N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    _, wq = _weights(rng, wtype, N, K)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    qx, dx, sx = oracle.quantize_act_q8(x)
    dW, dQ, dD, dS, dB = (ctx.upload(a) for a in (wq, qx, dx, sx, bias))
    dY = ctx.alloc(M * N * 4)
    ctx.gemm_q(wtype, dW, N, K, dQ, dD, dS, M, dB, ema.ACT_SILU, None, dY)
    y = ctx.download(dY, (M, N), np.float32)
    ref = oracle.gemm_q_i8(wtype, wq, N, K, qx, dx, bias=bias, act=ema.ACT_SILU)
    for b in (dW, dQ, dD, dS, dB, dY):
        ctx.free(b)
    assert _rel_err(y, ref) <= TOL


@pytest.mark.parametrize("M,K", [(3, 256), (1025, 768)])
def test_quantize_codes16_bitexact(ctx, M, K):
    rng = np.random.default_rng(K + M)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0, 0] = 127.0
    x[0, 1:4] = [2.5, -2.5, 0.5]
    qx_r, dx_r, sx_r = oracle.quantize_act_q8(x)
    dX = ctx.upload(x)
    dq, dd, ds = ctx.alloc(M * K * 2), ctx.alloc(M * K // 32 * 4), ctx.alloc(M * K // 32 * 4)
    ctx.quantize_act_q8_codes16(dX, M, K, dq, dd, ds)
    codes = ctx.download(dq, (M, K), np.float16)
    assert np.array_equal(codes.astype(np.int32), qx_r.astype(np.int32))
    assert np.array_equal(ctx.download(dd, (M, K // 32), np.float32), dx_r)
    assert np.array_equal(ctx.download(ds, (M, K // 32), np.int32), sx_r)
    for b in (dX, dq, dd, ds):
        ctx.free(b)
