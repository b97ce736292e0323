"""GPU parity of the dequantize-fused FC path on the quantized bytes: mgh_pack_weights_dq and
mgh_gemm_dq / _f32in / _y16 / _ln (k_gemm_fc.hip, weight forms 8 and 12: the Q8_0 / Q4_K
bytes are read on every call and decoded to fp16 as the MFMA fragments are read; k_gemv_fc
for a few activation rows).

Bars:
  * the GEMM against a float64 product of the same fp16 operands: the weights as
    mgh_pack_weights_f16 decodes them (pinned to the oracle's dequantization in
    test_gpu_h16.py) and the activations rounded to fp16, max|y - ref| <= 1e-5 * max|ref| --
    only the fp32 summation order differs, so a wrong byte, scale, nibble, sub-block or group
    shows as O(1e-3) or more;
  * where both forms run the same kernel plan (the skinny-M kernel, and the post-norm pair at
    its split-K shapes) the output equals mgh_gemm_h16's on the fp16 copy bit for bit;
  * the path as a whole: within 1e-3 * max|y| of the reference's dequantize-then-F32 product
    on the fp32 activations (oracle.gemm_q_deq_f32, mg-cpu.cpp:48-72 semantics);
  * the layout holds exactly the GGUF byte count for N % 16 == 0 (1.0625 / 0.5625 bytes per
    weight) and pads the last 16-row group otherwise.
"""
import numpy as np
import pytest

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


def _gguf_bytes(wtype, N, K):
    return N * (K // 32) * 34 if wtype == ema.WTYPE_Q8_0 else N * (K // 256) * 144


def _act64(v, act):
    from scipy.special import erf
    if act == 1:
        return 0.5 * v * (1.0 + erf(v / np.sqrt(2.0)))
    if act == 2:
        return v / (1.0 + np.exp(-v))
    return v


def _ref64(ctx, dP16, N, K, x16, bias, act, resid):
    """float64 product of the fp16 weights (downloaded from the fp16 copy) and fp16 activations"""
    w16 = ctx.download(dP16, (N, K), np.float16).astype(np.float64)
    r = _act64(x16.astype(np.float64) @ w16.T + bias, act)
    return r + resid if resid is not None else r


def _weights(ctx, wtype, N, K, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[0, :64] = 0.0                       # an all-zero block (d = 0)
    w[-1, 32:64] *= 40.0                  # a large-scale block
    wq = oracle.quantize(wtype, w)
    dW = ctx.upload(wq)
    dP16 = ctx.alloc(ema.packed_weight_bytes_f16(N, K))
    ctx.pack_weights_f16(wtype, dW, N, K, dP16)
    nb = ema.packed_weight_bytes_dq(wtype, N, K)
    dQ = ctx.alloc(nb)
    ctx.pack_weights_dq(wtype, dW, N, K, dQ)
    ctx.free(dW)
    return wq, dP16, dQ, nb


@pytest.mark.parametrize("wtype", [ema.WTYPE_Q8_0, ema.WTYPE_Q4_K])
@pytest.mark.parametrize("N,K", [(16, 256), (96, 512), (100, 768), (2304, 768), (768, 3072)])
def test_dq_layout_size(wtype, N, K):
    G = (N + 15) // 16
    got = ema.packed_weight_bytes_dq(wtype, N, K)
    assert got == _gguf_bytes(wtype, 16 * G, K)
    if N % 16 == 0:
        assert got == _gguf_bytes(wtype, N, K)


# skinny-M kernel (M <= 16, or <= 32 with K <= 1024) and tiled plans: few tiles (64 x 64 on a
# 3-deep ring, 32-row tiles), split K, 128-row tiles, fp16 operands; N = 100 and 132 end in a
# partial 16-row group
SHAPES = [(1, 2304, 768), (7, 132, 256), (16, 768, 3072), (32, 768, 768), (33, 100, 768),
          (65, 128, 768), (257, 3072, 768), (257, 768, 3072), (1025, 2304, 768), (1025, 768, 768),
          (1025, 3072, 768), (1025, 768, 3072), (4097, 2304, 768), (4112, 768, 3072),
          # the up-proj at M = 4097 / 4112: the last, partial row of 128-row tiles runs on the
          # skinny-M kernel after the tiled kernel (GELU without residual, residual without act)
          (4097, 3072, 768), (4112, 3072, 768),
          # a partial last 16-row weight group under the tiled plans (N = 1000: 62 full groups
          # and 8 rows; the buffer resources end at the packed bytes)
          (1025, 1000, 768), (4097, 1000, 768)]


@pytest.mark.parametrize("wtype", [ema.WTYPE_Q8_0, ema.WTYPE_Q4_K])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_gemm_dq_f32in(ctx, wtype, M, N, K):
    act, res = (1, False) if (M + N) % 2 else (0, True)
    print(f"gemm_dq_f32in wtype={wtype} M={M} N={N} K={K} act={act} resid={res}", flush=True)
    rng = np.random.default_rng(M + 3 * N + K + wtype)
    wq, dP16, dQ, _ = _weights(ctx, wtype, N, K, M + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    resid = rng.standard_normal((M, N)).astype(np.float32) if res else None
    dX, dB = ctx.upload(x), ctx.upload(bias)
    dR = ctx.upload(resid) if res else None
    dY, dY16 = ctx.alloc(M * N * 4), ctx.alloc(M * N * 4)
    ctx.gemm_dq_f32in(wtype, dQ, N, K, dX, M, dB, act, dR, dY)
    y = ctx.download(dY, (M, N), np.float32)
    ctx.gemm_h16_f32in(dP16, N, K, dX, M, dB, act, dR, dY16)
    y16 = ctx.download(dY16, (M, N), np.float32)
    ref = _ref64(ctx, dP16, N, K, x.astype(np.float16), bias, act, resid)
    for t in (dP16, dQ, dX, dB, dR, dY, dY16):
        if t is not None:
            ctx.free(t)
    e64 = _rel(y, ref)
    print(f"  rel err vs float64 of the fp16 operands {e64:.2e}")
    assert e64 <= 1e-5
    if M <= 32:                           # skinny-M kernel: one plan for both weight forms
        assert np.array_equal(y.view(np.uint32), y16.view(np.uint32))
    if M * N * K <= 1025 * 3072 * 768:
        ref = oracle.gemm_q_deq_f32(wtype, wq, N, K, x, bias=bias, act=act, resid=resid)
        err = _rel(y, ref)
        print(f"  rel err vs dequantize-then-F32 {err:.2e}")
        assert err <= 1e-3


# K loops whose stage count is not a multiple of the ring depth: the unrolled ring's last,
# partial iteration (2-deep ring on fp32 rows: 5 stages; 3-deep few-tile ring: 5 stages and a
# split of 14; 2-deep split-K ring: 7 stages per split; the fp16-operand 128 x 128 kernel of the
# fp16 copies: 21 stages)
ODD_STAGES = [(ema.WTYPE_Q8_0, 300, 256, 320, False), (ema.WTYPE_Q8_0, 100, 256, 320, False),
              (ema.WTYPE_Q4_K, 200, 256, 1792, False), (ema.WTYPE_Q4_K, 1025, 768, 1792, False),
              (ema.WTYPE_Q8_0, 4112, 3072, 1344, True)]


@pytest.mark.parametrize("wtype,M,N,K,x16in", ODD_STAGES)
def test_gemm_odd_stage_counts(ctx, wtype, M, N, K, x16in):
    print(f"odd stage count wtype={wtype} M={M} N={N} K={K} fp16 operand={x16in}", flush=True)
    rng = np.random.default_rng(M + N + K + wtype)
    _, dP16, dQ, _ = _weights(ctx, wtype, N, K, M * 7 + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x16 = x.astype(np.float16)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    resid = rng.standard_normal((M, N)).astype(np.float32)
    dX = ctx.upload(x16 if x16in else x)
    dB, dR = ctx.upload(bias), ctx.upload(resid)
    dY = ctx.alloc(M * N * 4)
    ref = _ref64(ctx, dP16, N, K, x16, bias, 1, resid)
    for form in ("dq", "h16"):
        if x16in:
            if form == "dq":
                ctx.gemm_dq(wtype, dQ, N, K, dX, M, dB, 1, dR, dY)
            else:
                ctx.gemm_h16(dP16, N, K, dX, M, dB, 1, dR, dY)
        elif form == "dq":
            ctx.gemm_dq_f32in(wtype, dQ, N, K, dX, M, dB, 1, dR, dY)
        else:
            ctx.gemm_h16_f32in(dP16, N, K, dX, M, dB, 1, dR, dY)
        y = ctx.download(dY, (M, N), np.float32)
        err = _rel(y, ref)
        print(f"  {form}: rel err vs float64 of the fp16 operands {err:.2e}")
        assert err <= 1e-5, form
    for t in (dP16, dQ, dX, dB, dR, dY):
        ctx.free(t)


@pytest.mark.parametrize("wtype", [ema.WTYPE_Q8_0, ema.WTYPE_Q4_K])
@pytest.mark.parametrize("M,N,K", [(12, 768, 768), (257, 2304, 768), (1025, 3072, 768), (4112, 768, 3072)])
def test_gemm_dq_fp16_operand_and_y16(ctx, wtype, M, N, K):
    """fp16 activations (the LayerNorm's operand form) and fp16 output, against the float64
    product of the fp16 operands (the fp16 output: within one fp16 rounding of it)."""
    print(f"gemm_dq/_y16 wtype={wtype} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * 5 + N + K)
    _, dP16, dQ, _ = _weights(ctx, wtype, N, K, M * 3 + N)
    x16 = rng.standard_normal((M, K)).astype(np.float16)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    dX, dB = ctx.upload(x16), ctx.upload(bias)
    dA, dB2 = ctx.alloc(M * N * 4), ctx.alloc(M * N * 4)
    for act in (0, 1):
        ctx.gemm_dq(wtype, dQ, N, K, dX, M, dB, act, None, dA)
        a = ctx.download(dA, (M, N), np.float32)
        assert _rel(a, _ref64(ctx, dP16, N, K, x16, bias, act, None)) <= 1e-5, f"act {act}"
    ctx.gemm_dq_y16(wtype, dQ, N, K, dX, M, dB, 1, None, dA)
    a = ctx.download(dA, (M, N), np.float16).astype(np.float64)
    ref = _ref64(ctx, dP16, N, K, x16, bias, 1, None)
    assert np.all(np.abs(a - ref) <= 2.0 ** -10 * np.abs(ref) + 1e-5 * np.abs(ref).max())
    for t in (dP16, dQ, dX, dB, dA, dB2):
        ctx.free(t)


@pytest.mark.parametrize("wtype", [ema.WTYPE_Q8_0, ema.WTYPE_Q4_K])
@pytest.mark.parametrize("M,N,K", [(257, 768, 3072), (1025, 768, 768), (4112, 768, 3072)])
def test_gemm_dq_ln_equals_fp16_copy(ctx, wtype, M, N, K):
    """the post-norm pair (FC + residual, then LayerNorm-affine of its rows; the split-K reduce
    normalizes the rows where the plan splits K) on the quantized bytes: y within 1e-5 of the
    float64 product, and the LayerNorm outputs equal mgh_layernorm_affine applied to that y
    (the pair's contract); at M = 257 and 1025 both weight forms run the same split-K plan, so
    the outputs also equal the fp16-copy pair's bit for bit"""
    print(f"gemm_dq_ln wtype={wtype} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + N * 7 + K)
    _, dP16, dQ, _ = _weights(ctx, wtype, N, K, M + 11)
    x16 = rng.standard_normal((M, K)).astype(np.float16)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    resid = rng.standard_normal((M, N)).astype(np.float32)
    gamma = (1 + 0.02 * rng.standard_normal(N)).astype(np.float32)
    beta = (0.01 * rng.standard_normal(N)).astype(np.float32)
    up = [ctx.upload(a) for a in (x16, bias, resid, gamma, beta)]
    dX, dB, dR, dG, dBe = up
    outs = []
    for kind in ("dq", "h16", "ln_of_y"):
        dY, dL, dC = ctx.alloc(M * N * 4), ctx.alloc(M * N * 4), ctx.alloc(M * N * 2)
        if kind == "dq":
            ctx.gemm_dq_ln(wtype, dQ, N, K, dX, M, dB, 0, dR, dY, dG, dBe, 1e-12, dL, emit=2, codes=dC)
            y_dq = dY
        elif kind == "h16":
            ctx.gemm_h16_ln(dP16, N, K, dX, M, dB, 0, dR, dY, dG, dBe, 1e-12, dL, emit=2, codes=dC)
        else:                             # the LayerNorm of the dq pair's own y
            ctx.layernorm_affine(y_dq, dG, dBe, M, N, 1e-12, dL, emit=2, codes=dC)
        outs.append([ctx.download(dY, (M, N), np.uint32), ctx.download(dL, (M, N), np.uint32),
                     ctx.download(dC, (M, N), np.uint16)])
        if kind != "dq":
            ctx.free(dY)
        for t in (dL, dC):
            ctx.free(t)
    y = outs[0][0].view(np.float32)
    assert _rel(y, _ref64(ctx, dP16, N, K, x16, bias, 0, resid)) <= 1e-5
    for t in up + [dP16, dQ, y_dq]:
        ctx.free(t)
    assert np.array_equal(outs[0][1], outs[2][1]) and np.array_equal(outs[0][2], outs[2][2])
    if M <= 1025:
        for a, b in zip(outs[0], outs[1]):
            assert np.array_equal(a, b)


# Partial tiles in both directions with a residual: the epilogue's buffer ranges end with the
# tile's last row inside M, and columns past N take an offset beyond any range, so these outputs
# (and their residual reads) rely on the hardware range check; fp32 rows (64-row tiles, the
# skinny-M kernel for a ragged last row) and fp16 rows (128-row tiles), fp32 and fp16 output.
@pytest.mark.parametrize("wtype", [ema.WTYPE_Q8_0, ema.WTYPE_Q4_K])
@pytest.mark.parametrize("M,N,K", [(65, 100, 768), (1025, 1000, 768), (4097, 1000, 768), (300, 1000, 256)])
def test_gemm_dq_ragged_tiles_with_residual(ctx, wtype, M, N, K):
    print(f"gemm_dq ragged wtype={wtype} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + N + K + wtype)
    _, dP16, dQ, _ = _weights(ctx, wtype, N, K, M + 2 * N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x16 = x.astype(np.float16)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    resid = rng.standard_normal((M, N)).astype(np.float32)
    dX, dX16, dB, dR = ctx.upload(x), ctx.upload(x16), ctx.upload(bias), ctx.upload(resid)
    # the outputs carry a guard past M x N that no store may touch
    guard = 4096
    dY = ctx.upload(np.full(M * N + guard, 7.0, np.float32))
    dY16 = ctx.upload(np.full(M * N + guard, 7.0, np.float16))
    for act in (0, 1):
        ref = _ref64(ctx, dP16, N, K, x16, bias, act, resid)
        for form, call in (("fp32 rows", lambda: ctx.gemm_dq_f32in(wtype, dQ, N, K, dX, M, dB, act, dR, dY)),
                           ("fp16 rows", lambda: ctx.gemm_dq(wtype, dQ, N, K, dX16, M, dB, act, dR, dY))):
            call()
            y = ctx.download(dY, (M * N + guard,), np.float32)
            assert _rel(y[:M * N].reshape(M, N), ref) <= 1e-5, f"{form} act {act}"
            assert np.all(y[M * N:] == 7.0), f"{form} act {act}: store past the output"
        ctx.gemm_dq_y16(wtype, dQ, N, K, dX16, M, dB, act, dR, dY16)
        y16 = ctx.download(dY16, (M * N + guard,), np.float16)
        a = y16[:M * N].reshape(M, N).astype(np.float64)
        assert np.all(np.abs(a - ref) <= 2.0 ** -10 * np.abs(ref) + 1e-5 * np.abs(ref).max()), f"y16 act {act}"
        assert np.all(y16[M * N:] == 7.0), f"y16 act {act}: store past the output"
    for t in (dP16, dQ, dX, dX16, dB, dR, dY, dY16):
        ctx.free(t)


_PLAN_CHILD = r"""
import os, sys
import numpy as np
sys.path.insert(0, os.getcwd())
import edge_maskgit_amd as ema
from tests.test_gpu_dq import _weights, _ref64, _rel
M, N, K = 1025, 2304, 768
ctx = ema.Context(0)
rng = np.random.default_rng(5)
_, dP16, dQ, _ = _weights(ctx, ema.WTYPE_Q8_0, N, K, 11)
x = rng.standard_normal((M, K)).astype(np.float32)
bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
dX, dB, dY = ctx.upload(x), ctx.upload(bias), ctx.alloc(M * N * 4)
try:
    ctx.gemm_dq_f32in(ema.WTYPE_Q8_0, dQ, N, K, dX, M, dB, 0, None, dY)
except ema.MghError as e:
    print("REFUSED", e)
    sys.exit(0)
y = ctx.download(dY, (M, N), np.float32)
print("ERR", _rel(y, _ref64(ctx, dP16, N, K, x.astype(np.float16), bias, 0, None)))
"""


@pytest.mark.parametrize("plan,ok", [("64,128,2,4", True), ("64,64,3,1,768,2304", True), ("48,128,2,1", False)])
def test_plan_override(plan, ok):
    """MGH_FC_PLAN replaces the tile plan of the tiled FC launches (read once per process, so in a
    child process): a plan the kernel set holds gives the same product (the float64 bar), one it
    does not hold is refused."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, MGH_FC_PLAN=plan)
    print(f"MGH_FC_PLAN={plan}", flush=True)
    r = subprocess.run([sys.executable, "-c", _PLAN_CHILD], cwd=root, env=env, capture_output=True, text=True,
                       timeout=300)
    print(r.stdout[-400:], r.stderr[-400:])
    assert r.returncode == 0
    if ok:
        err = float(r.stdout.split("ERR")[-1])
        assert err <= 1e-5
    else:
        assert "REFUSED" in r.stdout


def test_pack_dq_rejects_bad_shapes(ctx):
    dW = ctx.alloc(1024)
    with pytest.raises(ema.MghError):
        ctx.pack_weights_dq(ema.WTYPE_Q4_K, dW, 4, 128, dW)          # Q4_K needs K % 256 == 0
    with pytest.raises(ema.MghError):
        ctx.pack_weights_dq(7, dW, 4, 256, dW)                        # not a quantized type
    ctx.free(dW)
    assert ema.packed_weight_bytes_dq(ema.WTYPE_Q4_K, 4, 128) == 0


def test_gemm_rejects_n_past_the_epilogue_offsets(ctx):
    # the tiled epilogue addresses a tile's outputs with 32-bit offsets from its origin: N is
    # refused past 2^21 (before any pointer is touched, so a small buffer stands in)
    d = ctx.alloc(4096)
    for fn in (ctx.gemm_dq, ctx.gemm_dq_f32in):
        with pytest.raises(ema.MghError, match="N <= 2097152"):
            fn(ema.WTYPE_Q8_0, d, (1 << 21) + 4, 64, d, 1, None, 0, None, d)
    with pytest.raises(ema.MghError, match="N <= 2097152"):
        ctx.gemm_h16(d, (1 << 21) + 4, 64, d, 1, None, 0, None, d)
    ctx.free(d)


@pytest.mark.parametrize("wtype,N,K", [(ema.WTYPE_Q8_0, 1, 32), (ema.WTYPE_Q8_0, 99, 96), (ema.WTYPE_Q8_0, 768, 3072),
                                       (ema.WTYPE_Q4_K, 3, 256), (ema.WTYPE_Q4_K, 99, 512)])
def test_dequant_weights_f32_matches_oracle(ctx, wtype, N, K):
    """mgh_dequant_weights_f32 (the weights of the F32 dequant GEMM for shapes outside the fused
    kernels) equals the oracle's dequantization, itself pinned to the reference decoder, bit for
    bit; the source rows start at an odd byte offset, as Q8_0 rows of K % 64 != 0 do"""
    rng = np.random.default_rng(N + K)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[0, :32] = 0.0
    wq = oracle.quantize(wtype, w)
    buf = np.zeros(wq.nbytes + 1, np.uint8)
    buf[1:] = wq.reshape(-1)
    dW = ctx.upload(buf)
    dO = ctx.alloc(N * K * 4)
    ctx.dequant_weights_f32(wtype, dW.ptr + 1, N, K, dO)
    got = ctx.download(dO, (N, K), np.float32)
    ctx.free(dW)
    ctx.free(dO)
    want = oracle.dequant(wtype, wq, N, K)
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
