"""GPU parity of the VQGAN decoder's ops (k_vqgan.hip) through the C ABI.

Bars:
  * Conv2D: against a float64 im2col product of the same fp32 operands, max|y - ref| <= 1e-5 *
    max|ref| (only the fp32 summation order differs from the reference's k_conv_2d,
    src/mg-cpu/mg-cpu.cpp:165-190), over 3x3 / 1x1 / 5x5 kernels, stride 1 and 2, padding,
    output tiles that do not fill 64 pixels or 64 channels, and batches of images;
  * GroupNorm: the CPU executor's formula (mg-cpu.cpp:123-147) evaluated in numpy — mean and
    variance in float64, inv = 1 / sqrt(float32(var) + eps) in float32, y = float32(x - mean) *
    inv — within 2 ulp, and at least 99% of the values bit-exact (the double sums run in another
    order); the fused affine + SiLU (mg-cpu.cpp:262-276) within 1e-6 * max|y|; groups spread over
    several statistics chunks included (the largest decoder resolution, 256 x 256 x 128);
  * Upscale: exact.
"""
import numpy as np
import pytest

import edge_maskgit_amd as ema

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = ema.Context(0)
    yield c
    c.close()


def conv_ref(x, ker, stride, pad):
    """x [N][IC][IH][IW], ker [OC][IC][KH][KW] -> [N][OC][OH][OW] in float64"""
    N, IC, IH, IW = x.shape
    OC, _, KH, KW = ker.shape
    OH, OW = (IH + 2 * pad - KH) // stride + 1, (IW + 2 * pad - KW) // stride + 1
    xp = np.zeros((N, IC, IH + 2 * pad, IW + 2 * pad), np.float64)
    xp[:, :, pad:pad + IH, pad:pad + IW] = x
    cols = np.empty((N, OH, OW, IC, KH, KW), np.float64)
    for kh in range(KH):
        for kw in range(KW):
            cols[:, :, :, :, kh, kw] = xp[:, :, kh:kh + stride * OH:stride, kw:kw + stride * OW:stride].transpose(0, 2, 3, 1)
    y = cols.reshape(N * OH * OW, -1) @ ker.reshape(OC, -1).astype(np.float64).T
    return y.reshape(N, OH, OW, OC).transpose(0, 3, 1, 2)


CONV = [  # IW, IH, IC, N, KW, KH, OC, stride, pad
    (9, 7, 5, 2, 3, 3, 7, 1, 1), (10, 10, 3, 1, 3, 3, 8, 2, 1), (8, 8, 33, 2, 1, 1, 65, 1, 0),
    (5, 5, 2, 1, 5, 5, 3, 1, 2), (65, 33, 20, 1, 3, 3, 130, 1, 1), (16, 16, 256, 1, 3, 3, 512, 1, 1),
    (32, 32, 128, 2, 3, 3, 64, 1, 1), (64, 64, 64, 1, 1, 1, 32, 1, 0), (7, 7, 4, 1, 3, 3, 3, 1, 0),
]


@pytest.mark.parametrize("IW,IH,IC,N,KW,KH,OC,stride,pad", CONV)
def test_conv2d_vs_float64(ctx, IW, IH, IC, N, KW, KH, OC, stride, pad):
    print(f"conv2d IW={IW} IH={IH} IC={IC} N={N} K={KW}x{KH} OC={OC} s={stride} p={pad}", flush=True)
    rng = np.random.default_rng(IW * 31 + IC * 7 + OC + KW)
    x = rng.standard_normal((N, IC, IH, IW)).astype(np.float32)
    ker = (rng.standard_normal((OC, IC, KH, KW)) / np.sqrt(IC * KH * KW)).astype(np.float32)
    OH, OW = (IH + 2 * pad - KH) // stride + 1, (IW + 2 * pad - KW) // stride + 1
    dX, dK, dY = ctx.upload(x), ctx.upload(ker), ctx.alloc(N * OC * OH * OW * 4)
    ctx.conv2d(dX, IW, IH, IC, N, dK, KW, KH, OC, stride, pad, dY)
    y = ctx.download(dY, (N, OC, OH, OW), np.float32)
    ctx.conv2d(dX, IW, IH, IC, N, dK, KW, KH, OC, stride, pad, dY)
    y2 = ctx.download(dY, (N, OC, OH, OW), np.float32)
    for b in (dX, dK, dY):
        ctx.free(b)
    ref = conv_ref(x, ker, stride, pad)
    err = np.abs(y - ref).max() / np.abs(ref).max()
    print(f"  rel err vs float64 {err:.2e}")
    assert err <= 1e-5
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


def gn_ref(x, G, eps, gamma=None, beta=None):
    """the CPU executor's GroupNorm (+ affine + SiLU) on x [N][C][H][W], numpy"""
    N, C, H, W = x.shape
    xg = x.reshape(N, G, -1).astype(np.float64)
    mean = xg.mean(axis=2, keepdims=True)
    var = ((xg - mean) ** 2).mean(axis=2, keepdims=True)
    inv = np.float32(1.0) / np.sqrt(var.astype(np.float32) + np.float32(eps))
    y = ((xg - mean).astype(np.float32) * inv).reshape(N, C, H, W)
    if gamma is not None:
        xn = y * gamma[None, :, None, None] + beta[None, :, None, None]
        y = xn / (np.float32(1.0) + np.exp(-xn))
    return y.astype(np.float32)


GN = [(16, 16, 512, 1, 32), (9, 7, 64, 2, 32), (64, 64, 128, 1, 32), (256, 256, 128, 1, 32),
      (5, 3, 6, 3, 3), (32, 32, 256, 2, 32)]


@pytest.mark.parametrize("W,H,C,N,G", GN)
@pytest.mark.parametrize("affine", [False, True])
def test_group_norm(ctx, W, H, C, N, G, affine):
    print(f"group_norm W={W} H={H} C={C} N={N} G={G} affine={affine}", flush=True)
    rng = np.random.default_rng(W * 3 + C + N + affine)
    x = (rng.standard_normal((N, C, H, W)) * 2.0 + 0.5).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32) if affine else None
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32) if affine else None
    dX, dY = ctx.upload(x), ctx.alloc(x.nbytes)
    dG = ctx.upload(gamma) if affine else None
    dB = ctx.upload(beta) if affine else None
    ctx.group_norm(dX, W, H, C, N, G, 1e-5, dG, dB, dY)
    y = ctx.download(dY, x.shape, np.float32)
    for b in (dX, dY, dG, dB):
        if b is not None:
            ctx.free(b)
    ref = gn_ref(x, G, 1e-5, gamma, beta)
    if affine:
        assert np.abs(y - ref).max() <= 1e-6 * np.abs(ref).max()
    else:
        ulp = np.abs(y.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
        same = float((ulp == 0).mean())
        print(f"  bit-exact {same:.4f}, max {int(ulp.max())} ulp")
        assert ulp.max() <= 2 and same >= 0.99


@pytest.mark.parametrize("W,H,C,N,f", [(16, 16, 512, 1, 2), (7, 5, 3, 2, 3), (128, 128, 128, 1, 2)])
def test_upscale(ctx, W, H, C, N, f):
    rng = np.random.default_rng(W + C)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    dX, dY = ctx.upload(x), ctx.alloc(x.nbytes * f * f)
    ctx.upscale(dX, W, H, C, N, f, dY)
    y = ctx.download(dY, (N, C, H * f, W * f), np.float32)
    ctx.free(dX)
    ctx.free(dY)
    assert np.array_equal(y, x.repeat(f, axis=2).repeat(f, axis=3))


def test_vqgan_ops_reject_bad_args(ctx):
    d = ctx.alloc(1 << 12)
    with pytest.raises(ema.MghError):
        ctx.conv2d(d, 2, 2, 1, 1, d, 3, 3, 1, 1, 0, d)          # kernel larger than the input
    with pytest.raises(ema.MghError):
        ctx.conv2d(d, 4, 4, 1, 1, d, 3, 3, 1, 0, 1, d)          # stride 0
    with pytest.raises(ema.MghError):
        ctx.group_norm(d, 4, 4, 6, 1, 4, 1e-5, None, None, d)   # C % groups != 0
    with pytest.raises(ema.MghError):
        ctx.group_norm(d, 4, 4, 8, 1, 4, 1e-5, d, None, d)      # gamma without beta
    with pytest.raises(ema.MghError):
        ctx.upscale(d, 4, 4, 1, 1, 0, d)
    ctx.free(d)
