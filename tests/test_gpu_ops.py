"""GPU parity of the ops around the FC GEMMs: LayerNorm-affine (and its fused next-GEMM
operand), fp16-K/V flash attention, the fp32 GEMM of the tied head, and the graph glue.

Bars:
  * LN-affine vs the oracle (the reference CPU executor's double statistics): every element
    within 2 fp32 ulps of max|y|, and nearly all bit-exact; the fused int8-dot operand equals
    the activation quantizer applied to the kernel's own y, bit for bit.
  * Flash attention vs the oracle attention on fp16-rounded q/k/v: max|o - o_ref| <= 2e-5 *
    max|o_ref| (fp32 softmax; only summation order and the online rescaling differ).
  * fp32 GEMM vs the oracle's sequential fp32 GEMM: <= 1e-5 * max|y|.
  * get_rows / add / strided copy: exact.
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


# ---- LayerNorm-affine ------------------------------------------------------------------
@pytest.mark.parametrize("rows,D", [(1, 256), (5, 768), (1025, 768), (33, 2048)])
def test_layernorm_vs_oracle(ctx, rows, D):
    print(f"layernorm rows={rows} D={D}", flush=True)
    rng = np.random.default_rng(rows + D)
    x = (rng.standard_normal((rows, D)) * 3 + 0.5).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    b = (0.1 * rng.standard_normal(D)).astype(np.float32)
    ref = oracle.layernorm_affine(x, g, b, 1e-12)
    dX, dG, dB, dY = ctx.upload(x), ctx.upload(g), ctx.upload(b), ctx.alloc(x.nbytes)
    ctx.layernorm_affine(dX, dG, dB, rows, D, 1e-12, dY)
    y = ctx.download(dY, x.shape, np.float32)
    for t in (dX, dG, dB, dY):
        ctx.free(t)
    ulp = np.spacing(np.abs(ref).max())
    assert np.abs(y - ref).max() <= 2 * ulp
    frac = float(np.mean(y.view(np.uint32) == ref.view(np.uint32)))
    print(f"  bit-exact fraction {frac:.5f}")
    assert frac >= 0.99


def test_layernorm_emit_int8_operand(ctx):
    rows, D = 257, 768
    print("layernorm emit int8", flush=True)
    rng = np.random.default_rng(7)
    x = rng.standard_normal((rows, D)).astype(np.float32)
    x[3] = 0.0                                   # constant row: y = beta
    g = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    b = (0.1 * rng.standard_normal(D)).astype(np.float32)
    b[:32] = 0.0
    dX, dG, dB, dY = ctx.upload(x), ctx.upload(g), ctx.upload(b), ctx.alloc(x.nbytes)
    dC, dD, dS = ctx.alloc(rows * D * 2), ctx.alloc(rows * D // 32 * 4), ctx.alloc(rows * D // 32 * 4)
    ctx.layernorm_affine(dX, dG, dB, rows, D, 1e-12, dY, ema.EMIT_INT8, dC, dD, dS)
    y = ctx.download(dY, x.shape, np.float32)
    codes = ctx.download(dC, (rows, D), np.float16)
    dx = ctx.download(dD, (rows, D // 32), np.float32)
    sx = ctx.download(dS, (rows, D // 32), np.int32)
    # the same y without the operand
    ctx.layernorm_affine(dX, dG, dB, rows, D, 1e-12, dY)
    y0 = ctx.download(dY, x.shape, np.float32)
    for t in (dX, dG, dB, dY, dC, dD, dS):
        ctx.free(t)
    assert np.array_equal(y.view(np.uint32), y0.view(np.uint32))
    qx, dx_r, sx_r = oracle.quantize_act_q8(y)
    assert np.array_equal(codes.astype(np.int32), qx.astype(np.int32))
    assert np.array_equal(dx.view(np.uint32), dx_r.view(np.uint32))
    assert np.array_equal(sx, sx_r)


def test_layernorm_emit_deq_operand(ctx):
    rows, D = 65, 768
    print("layernorm emit deq-f16", flush=True)
    rng = np.random.default_rng(8)
    x = rng.standard_normal((rows, D)).astype(np.float32)
    g = np.ones(D, np.float32)
    b = np.zeros(D, np.float32)
    dX, dG, dB, dY = ctx.upload(x), ctx.upload(g), ctx.upload(b), ctx.alloc(x.nbytes)
    dC, dD, dS = ctx.alloc(rows * D * 2), ctx.alloc(rows * D // 32 * 4), ctx.alloc(rows * D // 32 * 4)
    ctx.layernorm_affine(dX, dG, dB, rows, D, 1e-12, dY, ema.EMIT_DEQ_F16, dC, dD, dS)
    y = ctx.download(dY, x.shape, np.float32)
    h = ctx.download(dC, (rows, D), np.float16)
    dx = ctx.download(dD, (rows, D // 32), np.float32)
    ux = ctx.download(dS, (rows, D // 32), np.float32)
    # the block scales and sums are optional: the fp16 operand alone, bit-identical
    dC2, dY2 = ctx.alloc(rows * D * 2), ctx.alloc(x.nbytes)
    ctx.layernorm_affine(dX, dG, dB, rows, D, 1e-12, dY2, ema.EMIT_DEQ_F16, dC2, None, None)
    y2 = ctx.download(dY2, x.shape, np.float32)
    h2 = ctx.download(dC2, (rows, D), np.float16)
    for t in (dX, dG, dB, dY, dC, dD, dS, dC2, dY2):
        ctx.free(t)
    assert np.array_equal(h2.view(np.uint16), h.view(np.uint16))
    assert np.array_equal(y2.view(np.uint32), y.view(np.uint32))
    assert np.array_equal(h, y.astype(np.float16))
    assert np.all(dx == 1.0)
    blk = h.astype(np.float64).reshape(rows, D // 32, 32).sum(-1)
    assert np.abs(ux - blk).max() <= 1e-5 * max(np.abs(blk).max(), 1.0)


# ---- flash attention -------------------------------------------------------------------
def _qkv(rng, D, S, H, B):
    shape = (B * S, H * D)                       # the FC outputs [S*B][H*D] (batch-major rows)
    return [rng.standard_normal(shape).astype(np.float32) for _ in range(3)]


# S <= 512 runs the whole-head kernel (K/V of a head resident in LDS), longer sequences the
# chunked online-softmax kernel
@pytest.mark.parametrize("D,S,H,B", [(48, 1, 2, 1), (48, 16, 2, 1), (48, 17, 2, 1), (48, 64, 3, 2), (48, 65, 2, 1),
                                     (48, 257, 16, 2), (64, 130, 4, 1), (16, 40, 1, 1), (32, 300, 2, 1),
                                     (48, 512, 2, 1), (64, 512, 1, 1), (48, 513, 2, 1), (48, 1025, 1, 1)])
def test_flash_attn_vs_oracle(ctx, D, S, H, B):
    print(f"flash_attn D={D} S={S} H={H} B={B}", flush=True)
    rng = np.random.default_rng(D * S + H + B)
    q, k, v = _qkv(rng, D, S, H, B)
    st = (1, H * D, D, H * D * S)
    scale = 1.0 / np.sqrt(D)
    ref = oracle.attention(q, k, v, st, D, S, H, B, scale, True)
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    do = ctx.alloc(D * S * H * B * 4)
    ctx.flash_attn_f16kv(dq, dk, dv, st, D, S, H, B, scale, do)
    o = ctx.download(do, (D * S * H * B,), np.float32)
    # merged-head output written directly ({D,S,H,B} -> [S*B][H*D])
    ctx.flash_attn_f16kv(dq, dk, dv, st, D, S, H, B, scale, do, o_strides=(1, H * D, D, H * D * S))
    om = ctx.download(do, (D * S * H * B,), np.float32)
    for t in (dq, dk, dv, do):
        ctx.free(t)
    err = _rel(o, ref)
    print(f"  rel err {err:.2e}")
    assert err <= 2e-5
    assert np.array_equal(om, oracle.merge_heads(o, D, S, H, B))


@pytest.mark.parametrize("D,S,H", [(48, 257, 16), (64, 130, 4), (48, 40, 1)])
def test_flash_attn_split_queries_bit_identical(ctx, D, S, H):
    """with few heads the whole-head kernel spreads a head's query tiles over several
    workgroups; one image alone (split) and the same image repeated 16 times in a batch (at
    H = 16 unsplit) give the same bits"""
    rng = np.random.default_rng(D + S + H)
    q, k, v = _qkv(rng, D, S, H, 1)
    outs = []
    for B in (1, 16):
        qb, kb, vb = (np.ascontiguousarray(np.tile(a, (B, 1))) for a in (q, k, v))
        st = (1, H * D, D, H * D * S)
        dq, dk, dv = ctx.upload(qb), ctx.upload(kb), ctx.upload(vb)
        do = ctx.alloc(D * S * H * B * 4)
        ctx.flash_attn_f16kv(dq, dk, dv, st, D, S, H, B, 1.0 / np.sqrt(D), do)
        outs.append(ctx.download(do, (B, D * S * H), np.float32))
        for t in (dq, dk, dv, do):
            ctx.free(t)
    for b in range(16):
        assert np.array_equal(outs[1][b], outs[0][0])


@pytest.mark.parametrize("S", [257, 600])
def test_flash_attn_o16_is_rounded_output(ctx, S):
    """The fp16-output variant stores exactly the fp32 attention output rounded to fp16."""
    D, H, B = 48, 4, 2
    print(f"flash_attn_o16 S={S}", flush=True)
    rng = np.random.default_rng(S)
    q, k, v = _qkv(rng, D, S, H, B)
    st, ost = (1, H * D, D, H * D * S), (1, H * D, D, H * D * S)
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    do, dh = ctx.alloc(D * S * H * B * 4), ctx.alloc(D * S * H * B * 2)
    ctx.flash_attn_f16kv(dq, dk, dv, st, D, S, H, B, 0.144, do, o_strides=ost)
    ctx.flash_attn_f16kv_o16(dq, dk, dv, st, D, S, H, B, 0.144, dh, o_strides=ost)
    o = ctx.download(do, (D * S * H * B,), np.float32)
    h = ctx.download(dh, (D * S * H * B,), np.float16)
    for t in (dq, dk, dv, do, dh):
        ctx.free(t)
    assert np.array_equal(h.view(np.uint16), o.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("D,S,H,B,pad", [(48, 257, 16, 2, 0), (48, 1, 2, 1, 0), (64, 130, 4, 1, 0), (32, 512, 2, 1, 0),
                                         (48, 257, 4, 2, 4), (16, 33, 1, 3, 4), (64, 512, 2, 1, 12)])
def test_flash_attn_f16in_equals_rounded_inputs(ctx, D, S, H, B, pad):
    """The fp16-input variant on q/k/v rounded to fp16 gives the same bits as the fp32-input
    attention (which rounds its inputs to fp16 on load), for both output types, with q/k/v
    read through the strides of one wide [S*B][3*H*D + pad] buffer (the fused QKV output; a
    pad of 4 or 12 halves leaves fp16 rows 8-byte but not 16-byte aligned)."""
    print(f"flash_attn_f16in D={D} S={S} H={H} B={B} pad={pad}", flush=True)
    rng = np.random.default_rng(7 * D + S)
    E = H * D
    R = 3 * E + pad
    wide = rng.standard_normal((B * S, R)).astype(np.float16)
    st = (1, R, D, R * S)
    ost = (1, E, D, E * S)
    d32 = ctx.upload(wide.astype(np.float32))
    d16 = ctx.upload(wide)
    n = D * S * H * B
    o_ref, o_32, o_16 = ctx.alloc(n * 4), ctx.alloc(n * 4), ctx.alloc(n * 2)
    ctx.flash_attn_f16kv(d32.ptr, d32.ptr + 4 * E, d32.ptr + 8 * E, st, D, S, H, B, 0.144, o_ref, o_strides=ost)
    ctx.flash_attn_f16in(d16.ptr, d16.ptr + 2 * E, d16.ptr + 4 * E, st, D, S, H, B, 0.144, o=o_32, o_strides=ost)
    ctx.flash_attn_f16in(d16.ptr, d16.ptr + 2 * E, d16.ptr + 4 * E, st, D, S, H, B, 0.144, o16=o_16, o_strides=ost)
    ref = ctx.download(o_ref, (n,), np.float32)
    a = ctx.download(o_32, (n,), np.float32)
    h = ctx.download(o_16, (n,), np.float16)
    for t in (d32, d16, o_ref, o_32, o_16):
        ctx.free(t)
    assert np.array_equal(a.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(h.view(np.uint16), ref.astype(np.float16).view(np.uint16))


def test_flash_attn_f16in_rejects_long_sequences(ctx):
    buf = ctx.alloc(1 << 20)
    with pytest.raises(ema.MghError):
        ctx.flash_attn_f16in(buf, buf, buf, (1, 48, 48, 48 * 600), 48, 600, 1, 1, 0.1, o=buf)
    with pytest.raises(ema.MghError):
        ctx.flash_attn_f16in(buf, buf, buf, (1, 48, 48, 48 * 4), 48, 4, 1, 1, 0.1, o=buf, o16=buf)
    ctx.free(buf)


def test_flash_attn_large_scores(ctx):
    """Peaked softmax (large logits): the running max rescaling must stay exact."""
    D, S, H, B = 48, 257, 2, 1
    print("flash_attn peaked", flush=True)
    rng = np.random.default_rng(3)
    q, k, v = _qkv(rng, D, S, H, B)
    q *= 6.0
    st = (1, H * D, D, H * D * S)
    ref = oracle.attention(q, k, v, st, D, S, H, B, 1.0 / np.sqrt(D), True)
    dq, dk, dv, do = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.alloc(D * S * H * B * 4)
    ctx.flash_attn_f16kv(dq, dk, dv, st, D, S, H, B, 1.0 / np.sqrt(D), do)
    o = ctx.download(do, (D * S * H * B,), np.float32)
    for t in (dq, dk, dv, do):
        ctx.free(t)
    assert np.isfinite(o).all()
    assert _rel(o, ref) <= 2e-5


# ---- fp32 GEMM -------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K,act,res", [(1, 2025, 768, 0, False), (257, 2025, 768, 0, False),
                                           (70, 100, 64, 1, True), (130, 768, 3072, 2, True)])
def test_gemm_f32_vs_oracle(ctx, M, N, K, act, res):
    print(f"gemm_f32 M={M} N={N} K={K} act={act} resid={res}", flush=True)
    rng = np.random.default_rng(M + N + K)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    resid = rng.standard_normal((M, N)).astype(np.float32) if res else None
    ref = oracle.gemm_f32(w, x, bias=bias, act=act, resid=resid)
    dW, dX, dB, dY = ctx.upload(w), ctx.upload(x), ctx.upload(bias), ctx.alloc(M * N * 4)
    dR = ctx.upload(resid) if res else None
    ctx.gemm_f32(dW, N, K, dX, M, dB, act, dR, dY)
    y = ctx.download(dY, (M, N), np.float32)
    for t in (dW, dX, dB, dY, dR):
        if t is not None:
            ctx.free(t)
    err = _rel(y, ref)
    print(f"  rel err {err:.2e}")
    assert err <= 1e-5


# ---- glue ------------------------------------------------------------------------------
def test_get_rows_add_copy(ctx):
    print("glue ops", flush=True)
    rng = np.random.default_rng(11)
    R, E = 2025, 768
    table = rng.standard_normal((R, E)).astype(np.float32)
    ids = rng.integers(-R, R, 3 * 257).astype(np.int32)
    dT, dI, dO = ctx.upload(table), ctx.upload(ids), ctx.alloc(ids.size * E * 4)
    ctx.get_rows(dT, E, R, dI, ids.size, dO)
    got = ctx.download(dO, (ids.size, E), np.float32)
    assert np.array_equal(got, oracle.get_rows(table, ids))
    pos = rng.standard_normal((257, E)).astype(np.float32)
    dP, dS = ctx.upload(pos), ctx.alloc(ids.size * E * 4)
    ctx.add(dO, dP, pos.size, dS, ids.size * E)
    s = ctx.download(dS, (3, 257, E), np.float32)
    assert np.array_equal(s, got.reshape(3, 257, E) + pos[None])
    # head merge: {D,S,H,B} contiguous -> permute(0,2,1,3) -> [S*B][H*D]
    D, S, H, B = 48, 257, 16, 2
    a = rng.standard_normal(D * S * H * B).astype(np.float32)
    dA, dM = ctx.upload(a), ctx.alloc(a.nbytes)
    ctx.copy_strided(dA, (D, H, S, B), (1, D * S, D, D * S * H), dM)
    m = ctx.download(dM, (a.size,), np.float32)
    assert np.array_equal(m, oracle.merge_heads(a, D, S, H, B))
    for t in (dT, dI, dO, dP, dS, dA, dM):
        ctx.free(t)
