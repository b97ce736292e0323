"""GPU parity of the VQGAN decoder's ops (k_vqgan.hip) through the C ABI.

Reference values come from the pinned numpy oracle (oracle/vqgan.py), and for whole decoder
graphs also from the reference's own CPU executor (oracle/_ref/libmgref.so). Bars:
  * Conv2D: against the float64 sum of the same fp32 products rounded once, max|y - ref| <= 1e-5 *
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
import oracle
from edge_maskgit_amd import runtime as rt
from oracle import ref
from oracle import vqgan as ov
from tests import mg_gguf

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = ema.Context(0)
    yield c
    c.close()


# kernels: IC % 16 == 0 packed tap-major MFMA ("pk": 128 x 128 tiles, "pkn": 256 x 16 for
# OC <= 16; split over K when one image's output gives too few workgroups); else OC <= 8 one
# thread per pixel ("few"), or the reference-layout MFMA ("gen")
CONV = [  # IW, IH, IC, N, KW, KH, OC, stride, pad
    (9, 7, 5, 2, 3, 3, 7, 1, 1), (10, 10, 3, 1, 3, 3, 8, 2, 1), (5, 5, 2, 1, 5, 5, 3, 1, 2),
    (7, 7, 4, 1, 3, 3, 3, 1, 0), (32, 32, 128, 1, 3, 3, 3, 1, 1),                     # few, pkn
    (256, 256, 128, 1, 3, 3, 3, 1, 1), (20, 9, 32, 2, 3, 3, 16, 2, 1),                # pkn
    (8, 8, 33, 2, 1, 1, 65, 1, 0), (65, 33, 20, 1, 3, 3, 130, 1, 1),                  # gen
    (16, 16, 256, 1, 3, 3, 512, 1, 1), (16, 16, 512, 2, 3, 3, 512, 1, 1),             # pk, split
    (32, 32, 128, 2, 3, 3, 64, 1, 1), (64, 64, 64, 1, 1, 1, 32, 1, 0),                # pk
    (9, 7, 32, 1, 3, 3, 130, 2, 1), (13, 11, 48, 3, 3, 3, 200, 1, 1),                 # pk, tails
    (128, 128, 128, 1, 3, 3, 128, 1, 1), (32, 32, 256, 1, 1, 1, 256, 1, 0),           # pk
    (11, 6, 16, 1, 5, 5, 24, 1, 2),                                                   # pk, 5x5
    (256, 192, 16, 1, 3, 3, 16, 1, 1),                                                # pk, no split
    (4, 4, 4096, 260, 3, 3, 16, 1, 1),            # pk, 256 splits: images launched in groups of 255 + 5
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
    want = ov.conv2d(x, ker, stride, pad)
    err = np.abs(y - want).max() / np.abs(want).max()
    print(f"  rel err vs float64 {err:.2e}")
    assert err <= 1e-5
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    if OC <= 8 and IC % 16 and ref.available():
        # the one-thread-per-pixel kernel performs the CPU executor's float operations in its order
        assert np.array_equal(y, ref.conv2d(x, ker, stride, pad))


@pytest.mark.parametrize("IW,IH,IC,KW,KH,OC", [(16, 16, 512, 3, 3, 512), (128, 128, 128, 3, 3, 128),
                                                (32, 32, 128, 3, 3, 3), (65, 33, 20, 3, 3, 130)])
def test_conv2d_batch_invariant(ctx, IW, IH, IC, KW, KH, OC):
    """an image's output does not depend on the batch it is in (the split plan is per image)"""
    print(f"conv2d batch IW={IW} IH={IH} IC={IC} OC={OC}", flush=True)
    rng = np.random.default_rng(IC + OC)
    x = rng.standard_normal((3, IC, IH, IW)).astype(np.float32)
    ker = (rng.standard_normal((OC, IC, KH, KW)) / np.sqrt(IC * KH * KW)).astype(np.float32)
    dX, dK, dY = ctx.upload(x), ctx.upload(ker), ctx.alloc(3 * OC * IH * IW * 4)
    ctx.conv2d(dX, IW, IH, IC, 3, dK, KW, KH, OC, 1, 1, dY)
    y3 = ctx.download(dY, (3, OC, IH, IW), np.float32)
    for b in range(3):
        d1 = ctx.upload(np.ascontiguousarray(x[b:b + 1]))
        ctx.conv2d(d1, IW, IH, IC, 1, dK, KW, KH, OC, 1, 1, dY)
        assert np.array_equal(ctx.download(dY, (1, OC, IH, IW), np.float32)[0], y3[b])
        ctx.free(d1)
    for d in (dX, dK, dY):
        ctx.free(d)


@pytest.mark.parametrize("IW,IH,IC,N,KW,KH,OC,stride,pad", [
    (16, 16, 256, 1, 3, 3, 512, 1, 1), (32, 32, 128, 2, 3, 3, 64, 1, 1), (9, 7, 32, 1, 3, 3, 130, 2, 1),
    (32, 32, 128, 1, 3, 3, 3, 1, 1), (65, 33, 20, 1, 3, 3, 130, 1, 1), (64, 64, 128, 1, 1, 1, 128, 1, 0),
    (256, 192, 16, 1, 3, 3, 16, 1, 1)])
def test_conv2d_ex_bias_residual_packed(ctx, IW, IH, IC, N, KW, KH, OC, stride, pad):
    """the fused Add nodes: out = (conv + bias) + resid, each rounded as its own node, equal bit for
    bit to the plain conv followed by the two additions in float32; the packed weights from
    mgh_conv2d_pack_weights give the same bits as the per-call packing"""
    print(f"conv2d_ex IW={IW} IH={IH} IC={IC} N={N} K={KW}x{KH} OC={OC} s={stride} p={pad}", flush=True)
    rng = np.random.default_rng(IW + IC + OC)
    x = rng.standard_normal((N, IC, IH, IW)).astype(np.float32)
    ker = (rng.standard_normal((OC, IC, KH, KW)) / np.sqrt(IC * KH * KW)).astype(np.float32)
    bias = rng.standard_normal(OC).astype(np.float32)
    OH, OW = (IH + 2 * pad - KH) // stride + 1, (IW + 2 * pad - KW) // stride + 1
    res = rng.standard_normal((N, OC, OH, OW)).astype(np.float32)
    dX, dK, dB, dR = ctx.upload(x), ctx.upload(ker), ctx.upload(bias), ctx.upload(res)
    dY = ctx.alloc(res.nbytes)
    ctx.conv2d(dX, IW, IH, IC, N, dK, KW, KH, OC, stride, pad, dY)
    plain = ctx.download(dY, res.shape, np.float32)
    ctx.conv2d_ex(dX, IW, IH, IC, N, dK, None, KW, KH, OC, stride, pad, dB, dR, dY)
    fused = ctx.download(dY, res.shape, np.float32)
    assert np.array_equal(fused, (plain + bias[None, :, None, None]) + res)
    nbytes = ctx.conv2d_packed_bytes(KW, KH, IC, OC)
    assert (nbytes > 0) == (IC % 16 == 0)
    if nbytes:
        dP = ctx.alloc(nbytes)
        ctx.conv2d_pack_weights(dK, KW, KH, IC, OC, dP)
        ctx.conv2d_ex(dX, IW, IH, IC, N, None, dP, KW, KH, OC, stride, pad, dB, dR, dY)
        assert np.array_equal(ctx.download(dY, res.shape, np.float32), fused)
        ctx.free(dP)
    for b in (dX, dK, dB, dR, dY):
        ctx.free(b)


# planes of 4k elements take the 16-byte path (9 x 7, 5 x 3: single elements); a group spans
# 1 .. 520 statistics chunks of 4096 (1040 x 1024 x 2 channels, one group: more chunks than threads)
GN = [(16, 16, 512, 1, 32), (9, 7, 64, 2, 32), (64, 64, 128, 1, 32), (256, 256, 128, 1, 32),
      (5, 3, 6, 3, 3), (32, 32, 256, 2, 32), (1040, 1024, 2, 1, 1)]


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
    want = ov.group_norm(x, G, 1e-5, gamma, beta)
    if affine:
        assert np.abs(y - want).max() <= 1e-6 * np.abs(want).max()
    else:
        ulp = np.abs(y.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
        same = float((ulp == 0).mean())
        print(f"  bit-exact {same:.4f}, max {int(ulp.max())} ulp")
        assert ulp.max() <= 2 and same >= 0.99


@pytest.mark.parametrize("W,H,C,N,f", [(16, 16, 512, 1, 2), (7, 5, 3, 2, 3), (128, 128, 128, 1, 2),
                                        (7, 3, 5, 2, 2), (2, 9, 3, 3, 2), (6, 4, 2, 1, 1)])
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
    with pytest.raises(ema.MghError):      # the generic kernel needs the reference-layout weights
        ctx.conv2d_ex(d, 4, 4, 3, 1, None, d, 3, 3, 16, 1, 1, None, None, d)
    with pytest.raises(ema.MghError):      # no packed kernel for IC % 16 != 0
        ctx.conv2d_pack_weights(d, 3, 3, 3, 16, d)
    ctx.free(d)


# ---- whole decoder graphs through mgr_decode_images (mg::HipRuntime) ----
SMALL = [dict(n_tokens=16, E=32, codebook=64, filters=32, mult=(1, 2), R=1),
         dict(n_tokens=64, E=32, codebook=48, filters=32, mult=(1, 1, 2), R=2)]


@pytest.mark.parametrize("cfg", SMALL, ids=["L4-two-levels", "L8-three-levels-R2"])
def test_decode_graph_vs_reference(tmp_path, cfg):
    """the decoder graph on the GPU against the oracle composition and, where it is built, the
    reference decoder on its CPU executor: max|img - ref| <= 1e-4 * max|ref| (float32 sums in
    another order through every conv); B grids in one graph equal B single decodes bit for bit"""
    print(f"decode graph {cfg}", flush=True)
    path = str(tmp_path / "vq.gguf")
    side = mg_gguf.write_vqgan_model(path, seed=5, **cfg)
    t = mg_gguf.vqgan_tensors(np.random.default_rng(5), cfg["E"], cfg["codebook"], cfg["filters"], cfg["mult"], cfg["R"])
    rng = np.random.default_rng(6)
    grids = rng.integers(0, cfg["codebook"], (3, cfg["n_tokens"])).astype(np.int32)
    with rt.TransformerRuntime(path) as m:
        imgs = m.decode_images(grids)
        singles = [m.decode_images(g[None])[0] for g in grids]
    assert imgs.shape == (3, 3, side, side)
    for b in range(3):
        assert np.array_equal(imgs[b], singles[b])
        want = ov.decode(t, grids[b:b + 1], cfg["E"], cfg["filters"], cfg["mult"], cfg["R"])[0]
        err = np.abs(imgs[b] - want).max() / np.abs(want).max()
        print(f"  image {b}: rel err vs oracle {err:.2e}")
        assert err <= 1e-4
        if ref.available():
            want = ref.vqgan_decode(path, grids[b], side)
            assert np.abs(imgs[b] - want).max() <= 1e-4 * np.abs(want).max()


def test_decode_graph_production_size(tmp_path):
    """the production decoder (256 tokens, 128 filters, multipliers 1,1,2,2,4, two res blocks:
    a 256 x 256 image) on random weights: finite, repeatable bit for bit, and two grids in one
    graph equal their single decodes; its convolutions, GroupNorms and up-samplings at these
    shapes are checked against the oracle by the op tests above"""
    path = str(tmp_path / "vq.gguf")
    side = mg_gguf.write_vqgan_model(path, seed=7, n_tokens=256, E=256, codebook=1024, filters=128,
                                     mult=(1, 1, 2, 2, 4), R=2)
    grids = np.random.default_rng(8).integers(0, 1024, (2, 256)).astype(np.int32)
    with rt.TransformerRuntime(path) as m:
        a = m.decode_images(grids)
        b = m.decode_images(grids)
        one = m.decode_images(grids[1:])
    assert a.shape == (2, 3, side, side) and side == 256
    assert np.isfinite(a).all() and np.abs(a).max() > 0
    assert np.array_equal(a, b)
    assert np.array_equal(a[1], one[0])


def test_decode_images_in_groups(tmp_path):
    """11 grids decode as groups of 8 + 3: each image equals its single decode bit for bit"""
    cfg = SMALL[0]
    path = str(tmp_path / "vq.gguf")
    mg_gguf.write_vqgan_model(path, seed=12, **cfg)
    grids = np.random.default_rng(13).integers(0, cfg["codebook"], (11, cfg["n_tokens"])).astype(np.int32)
    with rt.TransformerRuntime(path) as m:
        imgs = m.decode_images(grids)
        for b in (0, 7, 8, 10):
            assert np.array_equal(imgs[b], m.decode_images(grids[b:b + 1])[0])


def test_decode_rejects_bad_grids(tmp_path):
    path = str(tmp_path / "vq.gguf")
    mg_gguf.write_vqgan_model(path, seed=0, **SMALL[0])
    with rt.TransformerRuntime(path) as m:
        with pytest.raises(ValueError):
            m.decode_images(np.zeros((1, 15), np.int32))
        with pytest.raises(ema.MghError, match="codebook"):
            m.decode_images(np.full((1, 16), 64, np.int32))


# ---- the int8 conv (mgh_conv2d_i8): bit-exact against the oracle's restatement of the
# reference's k_quantize_conv_w + k_conv2d_i8 ----
I8 = [  # IW, IH, IC, N, KW, KH, OC, stride, pad
    (9, 7, 8, 2, 3, 3, 5, 1, 1), (10, 10, 5, 1, 3, 3, 70, 2, 1), (16, 16, 256, 1, 3, 3, 512, 1, 1),
    (32, 32, 128, 2, 3, 3, 64, 1, 1), (64, 64, 128, 1, 1, 1, 128, 1, 0), (65, 33, 20, 1, 3, 3, 130, 1, 1),
    (32, 32, 128, 1, 3, 3, 3, 1, 1), (11, 6, 16, 1, 5, 5, 24, 1, 2), (64, 64, 64, 1, 3, 3, 128, 1, 1),
    # rows of 4 / 8 / 16 pixels (a ragged last 16-pixel tile, a partial last block at K = 180)
    (8, 5, 32, 2, 3, 3, 20, 1, 1), (16, 8, 20, 1, 3, 3, 24, 1, 1), (4, 9, 64, 3, 3, 3, 40, 1, 1),
    (12, 12, 32, 1, 3, 3, 16, 1, 1),
]


@pytest.mark.parametrize("IW,IH,IC,N,KW,KH,OC,stride,pad", I8)
def test_conv2d_i8_vs_oracle(ctx, IW, IH, IC, N, KW, KH, OC, stride, pad):
    print(f"conv2d_i8 IW={IW} IH={IH} IC={IC} N={N} K={KW}x{KH} OC={OC} s={stride} p={pad}", flush=True)
    rng = np.random.default_rng(IW + 3 * IC + OC)
    x = (rng.standard_normal((N, IC, IH, IW)) * (2.0 ** rng.integers(-3, 4, (1, IC, 1, 1)))).astype(np.float32)
    ker = (rng.standard_normal((OC, IC, KH, KW)) / np.sqrt(IC * KH * KW)).astype(np.float32)
    bias = rng.standard_normal(OC).astype(np.float32)
    OH, OW = (IH + 2 * pad - KH) // stride + 1, (IW + 2 * pad - KW) // stride + 1
    res = rng.standard_normal((N, OC, OH, OW)).astype(np.float32)
    K = IC * KH * KW
    nb = (K + 31) // 32
    OT = (OC + 15) // 16                  # channel tiles: codes [OT][nb][16][32], scales [OT][nb][16]
    nbytes = ctx.conv2d_i8_weight_bytes(KW, KH, IC, OC)
    codes_bytes = (OT * nb * 512 + 255) // 256 * 256
    assert nbytes == codes_bytes + OT * nb * 16 * 4
    dX, dK, dB, dR, dQ = ctx.upload(x), ctx.upload(ker), ctx.upload(bias), ctx.upload(res), ctx.alloc(nbytes)
    dY = ctx.alloc(res.nbytes)
    ctx.conv2d_i8_pack_weights(dK, KW, KH, IC, OC, dQ)
    raw = ctx.download(dQ, (nbytes,), np.uint8)
    qw_all = raw[:OT * nb * 512].view(np.int8).reshape(OT, nb, 16, 32).transpose(0, 2, 1, 3).reshape(OT * 16, nb * 32)
    dw_all = raw[codes_bytes:].view(np.float32).reshape(OT, nb, 16).transpose(0, 2, 1).reshape(OT * 16, nb)
    qw, dw = oracle.conv_quant_w(ker)
    assert np.array_equal(qw_all[:OC].astype(np.int32), qw.astype(np.int32)) and np.array_equal(dw_all[:OC], dw)
    assert not qw_all[OC:].any() and not dw_all[OC:].any()      # padding channels: zero codes and scales
    ctx.conv2d_i8(dX, IW, IH, IC, N, dQ, KW, KH, OC, stride, pad, None, None, dY)
    y = ctx.download(dY, res.shape, np.float32)
    want = oracle.conv2d_i8(x, qw, dw, KH, KW, stride, pad)
    mism = int((y != want).sum())
    print(f"  {mism} of {y.size} outputs differ from the oracle")
    assert mism == 0
    ctx.conv2d_i8(dX, IW, IH, IC, N, dQ, KW, KH, OC, stride, pad, dB, dR, dY)
    assert np.array_equal(ctx.download(dY, res.shape, np.float32), (want + bias[None, :, None, None]) + res)
    for b in (dX, dK, dB, dR, dQ, dY):
        ctx.free(b)


def _conv_i8_setup(ctx, rng, N, IC, IH, IW, OC, k):
    x = (rng.standard_normal((N, IC, IH, IW)) * (2.0 ** rng.integers(-3, 4, (1, IC, 1, 1)))).astype(np.float32)
    ker = (rng.standard_normal((OC, IC, k, k)) / np.sqrt(IC * k * k)).astype(np.float32)
    dX, dK = ctx.upload(x), ctx.upload(ker)
    dQ = ctx.alloc(ctx.conv2d_i8_weight_bytes(k, k, IC, OC))
    ctx.conv2d_i8_pack_weights(dK, k, k, IC, OC, dQ)
    return x, ker, dX, dK, dQ


def test_conv2d_i8_large_tiles_vs_oracle(ctx):
    """32 images of 64 x 64 with 64 output channels give the GEMM pass its 4 x 4 wave tiles
    (2048 waves, 4-deep ring); K = 144 leaves a partial last block. Bit-exact."""
    N, IC, IH, IW, OC = 32, 16, 64, 64, 64
    print(f"conv2d_i8 large tiles N={N} IC={IC} {IH}x{IW} OC={OC}", flush=True)
    rng = np.random.default_rng(77)
    x, ker, dX, dK, dQ = _conv_i8_setup(ctx, rng, N, IC, IH, IW, OC, 3)
    dY = ctx.alloc(N * OC * IH * IW * 4)
    ctx.conv2d_i8(dX, IW, IH, IC, N, dQ, 3, 3, OC, 1, 1, None, None, dY)
    y = ctx.download(dY, (N, OC, IH, IW), np.float32)
    qw, dw = oracle.conv_quant_w(ker)
    want = oracle.conv2d_i8(x, qw, dw, 3, 3, 1, 1)
    mism = int((y != want).sum())
    print(f"  {mism} of {y.size} outputs differ from the oracle")
    assert mism == 0
    for b in (dX, dK, dQ, dY):
        ctx.free(b)


@pytest.mark.parametrize("N,IC,IH,IW,OC,stride,pad", [(32, 16, 64, 64, 136, 1, 1), (16, 16, 64, 64, 1024, 2, 0)])
def test_conv2d_i8_one_pass_vs_oracle(ctx, N, IC, IH, IW, OC, stride, pad):
    """Shapes that take the one-pass kernel (quantizer inside the GEMM, >= 2048 waves): 32 images
    of 64 x 64 with 136 output channels (the second 128-channel tile is partial), and stride 2
    without padding (31 x 31 outputs, a ragged last pixel group); K = 144 leaves a partial last
    block. Bit-exact, with bias and residual."""
    print(f"conv2d_i8 one pass N={N} IC={IC} {IH}x{IW} OC={OC} stride={stride} pad={pad}", flush=True)
    rng = np.random.default_rng(78 + stride)
    x, ker, dX, dK, dQ = _conv_i8_setup(ctx, rng, N, IC, IH, IW, OC, 3)
    OH, OW = (IH + 2 * pad - 3) // stride + 1, (IW + 2 * pad - 3) // stride + 1
    bias = rng.standard_normal(OC).astype(np.float32)
    res = rng.standard_normal((N, OC, OH, OW)).astype(np.float32)
    dB, dR, dY = ctx.upload(bias), ctx.upload(res), ctx.alloc(res.nbytes)
    qw, dw = oracle.conv_quant_w(ker)
    want = oracle.conv2d_i8(x, qw, dw, 3, 3, stride, pad)
    ctx.conv2d_i8(dX, IW, IH, IC, N, dQ, 3, 3, OC, stride, pad, None, None, dY)
    y = ctx.download(dY, res.shape, np.float32)
    mism = int((y != want).sum())
    print(f"  {mism} of {y.size} outputs differ from the oracle")
    assert mism == 0
    ctx.conv2d_i8(dX, IW, IH, IC, N, dQ, 3, 3, OC, stride, pad, dB, dR, dY)
    assert np.array_equal(ctx.download(dY, res.shape, np.float32), (want + bias[None, :, None, None]) + res)
    for b in (dX, dK, dQ, dB, dR, dY):
        ctx.free(b)


# (IW, IH, IC, OC, N, sub-batch): the whole batch and its sub-batches take different GEMM wave
# tiles and ring depths (4 x 4 with rings of 2 and 4, 4 x 2, 2 x 2 with rings of 4 and 8, 4 x 1
# with rings of 3 and 6, 2 x 1, 1 x 1) or the one-pass kernel (3 x 3 and 1 x 1; 5 x 5 stays on
# two passes); every image's result must be bit-identical
I8_BATCH = [(64, 64, 256, 256, 8, 1, 3), (64, 64, 256, 256, 8, 4, 3), (128, 128, 128, 128, 16, 1, 3),
            (128, 128, 128, 3, 16, 4, 3), (96, 64, 64, 256, 2, 1, 3), (32, 32, 512, 512, 4, 1, 3),
            (128, 128, 256, 128, 16, 4, 1), (128, 128, 256, 64, 16, 1, 1), (128, 128, 16, 128, 16, 4, 5)]


@pytest.mark.parametrize("IW,IH,IC,OC,N,sub,k", I8_BATCH)
def test_conv2d_i8_batch_invariant(ctx, IW, IH, IC, OC, N, sub, k):
    print(f"conv2d_i8 batch invariance {IW}x{IH} IC={IC} OC={OC} k={k} N={N} in groups of {sub}", flush=True)
    rng = np.random.default_rng(IW + IC + OC + N + k)
    x, ker, dX, dK, dQ = _conv_i8_setup(ctx, rng, N, IC, IH, IW, OC, k)
    M = IW * IH
    pad = k // 2
    dY = ctx.alloc(N * OC * M * 4)
    ctx.conv2d_i8(dX, IW, IH, IC, N, dQ, k, k, OC, 1, pad, None, None, dY)
    whole = ctx.download(dY, (N, OC, IH, IW), np.float32)
    for g in range(0, N, sub):
        dXg = ctx.upload(np.ascontiguousarray(x[g:g + sub]))
        dYg = ctx.alloc(sub * OC * M * 4)
        ctx.conv2d_i8(dXg, IW, IH, IC, sub, dQ, k, k, OC, 1, pad, None, None, dYg)
        part = ctx.download(dYg, (sub, OC, IH, IW), np.float32)
        assert np.array_equal(part, whole[g:g + sub]), f"images {g}..{g + sub - 1} differ"
        ctx.free(dXg)
        ctx.free(dYg)
    for b in (dX, dK, dQ, dY):
        ctx.free(b)


def _check_decoder_nodes(m, t, grid, cfg, int8):
    """every node of one decode, recomputed from the GPU's own input to it (MG_DUMP_NAMED):
    conv chains (conv + bias / + residual) bit-exact for the int8 conv, <= 1e-5 * max against
    the float64 conv for the fp32 one; GroupNorm + SiLU <= 1e-6 * max; gather and up-sampling
    exact. Returns the number of nodes checked."""
    E, F, mult, R = cfg["E"], cfg["filters"], cfg["mult"], cfg["R"]
    L = int(round(cfg["n_tokens"] ** 0.5))
    n_checked = 0

    def get(name, C, side):
        return m.named(name).reshape(1, C, side, side)

    def conv_ref(p, x, pad, bias=False, resid=None):
        w = t[p + ".weight"]
        if int8:
            qw, dw = oracle.conv_quant_w(w)
            y = oracle.conv2d_i8(x, qw, dw, w.shape[2], w.shape[3], 1, pad)
        else:
            y = ov.conv2d(x, w, 1, pad)
        if bias:
            y = y + t[p + ".bias"][None, :, None, None]
        return y if resid is None else y + resid

    def same(name, got, want, exact):
        nonlocal n_checked
        n_checked += 1
        if exact:
            assert np.array_equal(got, want), f"{name}: {int((got != want).sum())} values differ"
        else:
            err = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
            assert err <= (1e-5 if "norm" not in name else 1e-6), f"{name}: rel err {err:.2e}"

    x_in = get("vqgan.decoder.conv_in.in", E, L)
    same("conv_in.in", x_in, t["vqgan.quantizer.codebook.weight"][grid].reshape(1, L, L, E).transpose(0, 3, 1, 2), True)
    width, side = F * mult[-1], L
    x = get("vqgan.decoder.conv_in", width, side)
    same("conv_in", x, conv_ref("vqgan.decoder.conv_in", x_in, 1, bias=True), int8)

    def block(p, x, cin, cout):
        n0 = get(p + "norm0", cin, side)
        same(p + "norm0", n0, ov.group_norm(x, 32, 1e-5, t[p + "norm0.weight"], t[p + "norm0.bias"]), False)
        c0 = get(p + "conv0", cout, side)
        same(p + "conv0", c0, conv_ref(p + "conv0", n0, 1), int8)
        n1 = get(p + "norm1", cout, side)
        same(p + "norm1", n1, ov.group_norm(c0, 32, 1e-5, t[p + "norm1.weight"], t[p + "norm1.bias"]), False)
        out = get(p + "out", cout, side)
        if cin == cout:           # conv1 + x: the residual Add runs in conv1's epilogue
            same(p + "out", out, conv_ref(p + "conv1", n1, 1, resid=x), int8)
        else:                     # h + conv_res(h), the upstream shortcut quirk
            h = get(p + "conv1", cout, side)
            same(p + "conv1", h, conv_ref(p + "conv1", n1, 1), int8)
            same(p + "out", out, conv_ref(p + "conv_res", h, 0, resid=h), int8)
        return out

    for l in range(R):
        x = block(f"vqgan.decoder.res_blocks.0.{l}.", x, width, width)
    for i in range(len(mult) - 1, -1, -1):
        j, o = len(mult) - i, F * mult[i]
        for l in range(R):
            x = block(f"vqgan.decoder.res_blocks.{j}.{l}.", x, width, o)
            width = o
        if i > 0:
            pu = f"vqgan.decoder.res_blocks.{j}.{R + 1}"
            side *= 2
            up = get(pu + ".in", width, side)
            same(pu + ".in", up, ov.upscale(x, 2), True)
            x = get(pu, width, side)
            same(pu, x, conv_ref(pu, up, 1, bias=True), int8)
    n = get("vqgan.decoder.norm_out", width, side)
    same("norm_out", n, ov.group_norm(x, 32, 1e-5, t["vqgan.decoder.norm_out.weight"], t["vqgan.decoder.norm_out.bias"]), False)
    img = get("vqgan.decoder.conv_out", 3, side)
    same("conv_out", img, conv_ref("vqgan.decoder.conv_out", n, 1, bias=True), int8)
    return n_checked, img


@pytest.mark.parametrize("algo", [1, 2], ids=["int8-conv", "fp32-conv"])
def test_decode_graph_per_node(tmp_path, monkeypatch, algo):
    """the decoder graph node by node from the GPU's own inputs (a fixed bar at every depth: an
    int8 conv requantizes its input, so a last-ulp difference in a GroupNorm output can move a
    code of the next conv, and end to end only compounded noise could be bounded); the
    runtime's int8 algorithm runs every conv as the reference's int8 conv, as its runtime does
    on integer-dot devices, and MG_NO_ARM_CONV=1 keeps the fp32 conv there"""
    cfg = SMALL[1]
    path = str(tmp_path / "vq.gguf")
    mg_gguf.write_vqgan_model(path, seed=9, **cfg)
    t = mg_gguf.vqgan_tensors(np.random.default_rng(9), cfg["E"], cfg["codebook"], cfg["filters"], cfg["mult"], cfg["R"])
    grid = np.random.default_rng(10).integers(0, cfg["codebook"], cfg["n_tokens"]).astype(np.int32)
    monkeypatch.setenv("MG_DUMP_NAMED", "1")
    with rt.TransformerRuntime(path, algo=algo) as m:
        img = m.decode_images(grid[None])[0]
        n, last = _check_decoder_nodes(m, t, grid, cfg, int8=algo == 1)
    print(f"algo {algo}: {n} nodes checked")
    assert n >= 20 and np.array_equal(img, last[0])
    if algo == 1:
        monkeypatch.setenv("MG_NO_ARM_CONV", "1")
        with rt.TransformerRuntime(path, algo=1) as m:
            m.decode_images(grid[None])
            _check_decoder_nodes(m, t, grid, cfg, int8=False)


def test_generate_images_end_to_end(tmp_path):
    """the reference's whole generate() on one model file (transformer + decoder): the grids of
    mgr_generate_images equal mgr_generate's, its images equal mgr_decode_images of those grids
    bit for bit and the oracle decoder's within 1e-4 * max"""
    path = str(tmp_path / "maskgit.gguf")
    _, v = mg_gguf.write_maskgit_model(path, n_layer=2, quant="q8_0", n_pos=17, E=32, filters=32, mult=(1, 2), R=1)
    cls, seeds = np.array([3, 207, 999], np.int32), np.array([1, 42, 7], np.uint64)
    with rt.TransformerRuntime(path) as m:
        grids, imgs = m.generate_images(cls, seeds, steps=4)
        assert np.array_equal(grids, m.generate(cls, seeds, steps=4))
        assert np.array_equal(imgs, m.decode_images(grids))
    assert grids.min() >= 0 and grids.max() < 1024 and imgs.shape == (3, 3, 8, 8)
    for b in range(3):
        want = ov.decode(v, grids[b:b + 1], 32, 32, (1, 2), 1)[0]
        assert np.abs(imgs[b] - want).max() <= 1e-4 * np.abs(want).max()
