"""The entry point that allocates nothing: mgh_gemm_h16_f32in_noalloc (scratch in the library's
fixed per-GPU array) against mgh_gemm_h16_f32in (context scratch) on the same inputs, bit for
bit, over consecutive calls that reuse the array with different shapes — a rounding pass plus
the fp16-operand plan, then a smaller call on the split-K plan, then a tiny one, then one on the
skinny-M kernel (no scratch) — and the
rejection of a shape whose scratch exceeds the array, before anything runs."""
import numpy as np
import pytest

import edge_maskgit_amd as ema
import oracle

pytestmark = pytest.mark.gpu


def _case(ctx, rng, M, N, K, act, resid):
    x = rng.standard_normal((M, K)).astype(np.float32)
    wq = oracle.quantize(ema.WTYPE_Q8_0, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    dW, dX, dB = ctx.upload(wq), ctx.upload(x), ctx.upload(bias)
    dR = ctx.upload(rng.standard_normal((M, N)).astype(np.float32)) if resid else None
    dP = ctx.alloc(ema.packed_weight_bytes_f16(N, K))
    ctx.pack_weights_f16(ema.WTYPE_Q8_0, dW, N, K, dP)
    dY0, dY1 = ctx.alloc(M * N * 4), ctx.alloc(M * N * 4)
    ctx.gemm_h16_f32in(dP, N, K, dX, M, dB, act, dR, dY0)
    ctx.gemm_h16_f32in_noalloc(dP, N, K, dX, M, dB, act, dR, dY1)
    y0 = ctx.download(dY0, (M, N), np.float32)
    y1 = ctx.download(dY1, (M, N), np.float32)
    for b in (dW, dX, dB, dR, dP, dY0, dY1):
        if b is not None:
            ctx.free(b)
    return y0, y1


def test_noalloc_equals_allocating_entry_point():
    rng = np.random.default_rng(77)
    with ema.Context(0) as ctx:
        # a rounding pass into the array (4200 x 3072 outputs take the separate pass), then a
        # split-K call with fp32 rows (partials in the array), then a tiny one, then a skinny-M call
        for M, N, K, act, resid in ((4200, 3072, 768, ema.ACT_GELU, True), (1025, 768, 3072, 0, True),
                                    (37, 96, 512, ema.ACT_GELU, False),
                                    (12, 768, 768, ema.ACT_GELU, True)):
            print(f"noalloc M={M} N={N} K={K}", flush=True)
            y0, y1 = _case(ctx, rng, M, N, K, act, resid)
            assert np.isfinite(y0).all()
            assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))


def test_noalloc_two_streams_share_the_array_in_order():
    """Two contexts (two streams) on one GPU call the no-allocation entry point back to back with
    no host synchronization between them: both need the shared array (a rounding pass and
    split-K partials), and the library's per-GPU event orders the second call after the first,
    so each result equals the allocating entry point's bit for bit, twice in a row."""
    rng = np.random.default_rng(5)
    shapes = [(4200, 3072, 768, 0), (1025, 768, 3072, 0)]
    with ema.Context(0) as c0, ema.Context(0) as c1:
        bufs = []
        for (M, N, K, act), c in zip(shapes, (c0, c1)):
            x = rng.standard_normal((M, K)).astype(np.float32)
            wq = oracle.quantize(ema.WTYPE_Q8_0, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
            dW, dX = c.upload(wq), c.upload(x)
            dP = c.alloc(ema.packed_weight_bytes_f16(N, K))
            c.pack_weights_f16(ema.WTYPE_Q8_0, dW, N, K, dP)
            dR = c.upload(rng.standard_normal((M, N)).astype(np.float32))
            d0, d1 = c.alloc(M * N * 4), c.alloc(M * N * 4)
            c.gemm_h16_f32in(dP, N, K, dX, M, None, act, dR, d0)
            c.sync()
            bufs.append((c, M, N, K, act, dP, dX, dR, d0, d1))
        for rep in range(2):
            print(f"noalloc two streams, round {rep}", flush=True)
            for c, M, N, K, act, dP, dX, dR, d0, d1 in bufs:
                c.gemm_h16_f32in_noalloc(dP, N, K, dX, M, None, act, dR, d1)
            for c, M, N, K, act, dP, dX, dR, d0, d1 in bufs:
                y0 = c.download(d0, (M, N), np.float32)
                y1 = c.download(d1, (M, N), np.float32)
                assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))


def test_noalloc_rejects_shapes_beyond_the_array():
    """M = 16448, K = 3072 needs a 101 MB rounded copy of x: refused before any launch (the
    dummy buffers below are never touched)"""
    with ema.Context(0) as ctx:
        d = ctx.alloc(1 << 12)
        with pytest.raises(ema.MghError, match="maximum"):
            ctx.gemm_h16_f32in_noalloc(d, 768, 3072, d, 16448, None, 0, None, d)
