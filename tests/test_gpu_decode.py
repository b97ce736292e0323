"""GPU parity of the on-device decoding step (mgh_decode_step, k_decode.hip) and of the
whole device-resident decode loop (mgr_generate).

Bars (integer outputs, so bit-exact):
  * mgh_decode_step against the oracle step (oracle/mg_oracle_decode.cpp, pinned by
    tests/test_oracle_decode.py) on the same logits: token grids and step samples identical at
    every step of an 8-step schedule, for several images and seeds, random logits of varying
    sharpness, the closed-form cases (uniform logits, ties at the last step), known tokens,
    one or no unknown position left, zero temperature, a 64-entry codebook,
    and more than 64 images (several seeding workgroups);
  * mgr_generate (forward in HBM -> decode step, 8 times) against the same loop run from the
    host: TransformerRuntime.forward (the same kernels, read back) followed by the oracle step;
    final grids identical; repeated runs identical.
"""
import numpy as np
import pytest

import edge_maskgit_amd as ema
import oracle
from edge_maskgit_amd import runtime as rt
from tests import mg_gguf

pytestmark = pytest.mark.gpu

MASK = 2024


@pytest.fixture(scope="module")
def ctx():
    c = ema.Context(0)
    yield c
    c.close()


def _start(B, S, rng):
    tok = np.full((B, S), MASK, np.int32)
    tok[:, 0] = 1024 + rng.integers(0, 1000, B)
    return tok


def _run(ctx, logits_fn, tok0, seeds, n_steps, CB=1024, n_tokens=256, choice_temp=4.5,
         mask_id=MASK, steps=None):
    """Device and oracle side by side; logits_fn(step, tokens) gives [B][S][V] logits."""
    B, S = tok0.shape
    state = ctx.alloc(ema.decode_state_bytes(B))
    work = ctx.alloc(ema.decode_work_bytes(B, S))
    d_tok = ctx.upload(tok0)
    d_res = ctx.alloc(tok0.nbytes)
    ctx.decode_init(seeds, state)
    d_log = None
    tok_ref = tok0.copy()
    for i, step in enumerate(range(n_steps) if steps is None else steps):
        logits = logits_fn(step, tok_ref)
        V = logits.shape[2]
        if d_log is None:
            d_log = ctx.alloc(logits.nbytes)
        ctx.write(d_log, logits)
        ctx.decode_step(state, work, d_log, B, S, V, CB, mask_id, n_tokens, step, n_steps,
                        choice_temp, d_tok, d_res)
        got_tok = ctx.download(d_tok, tok0.shape, np.int32)
        got_res = ctx.download(d_res, tok0.shape, np.int32)
        draws_before = 2 * S * i          # the device engines advance once per call
        tok_ref, res_ref = oracle.decode_step(logits, tok_ref, step, n_steps, seeds, draws_before,
                                              codebook=CB, mask_id=mask_id, n_tokens=n_tokens,
                                              choice_temp=choice_temp)
        bad_t = int((got_tok != tok_ref).sum())
        bad_r = int((got_res != res_ref).sum())
        print(f"  step {step}: masked {int((tok_ref == mask_id).sum())}  "
              f"token mismatches {bad_t}  sample mismatches {bad_r}", flush=True)
        assert bad_t == 0 and bad_r == 0
    for b in (state, work, d_tok, d_res, d_log):
        ctx.free(b)
    return tok_ref


@pytest.mark.parametrize("B,seeds", [(1, [42]), (3, [0, 42, 2**63 + 5])])
def test_decode_steps_vs_oracle(ctx, B, seeds):
    print(f"decode B={B} S=257 V=2025 random logits", flush=True)
    rng = np.random.default_rng(B)

    def logits(step, _):
        scale = 1.0 + step                                    # sharper every step
        return (rng.standard_normal((B, 257, 2025)) * scale).astype(np.float32)

    _run(ctx, logits, _start(B, 257, rng), seeds, 8)


def test_decode_uniform_logits_and_ties(ctx):
    print("decode uniform logits (closed form, last-step ties)", flush=True)
    rng = np.random.default_rng(1)
    z = np.zeros((2, 257, 2025), np.float32)
    z[:, :, 1024:] = 100.0
    _run(ctx, lambda s, t: z, _start(2, 257, rng), [7, 12345], 8)


def test_decode_known_tokens_and_edges(ctx):
    print("decode known tokens / one or no unknown / zero temperature", flush=True)
    rng = np.random.default_rng(2)
    tok0 = _start(3, 257, rng)
    known = rng.random((3, 257)) < 0.4
    known[:, 0] = False
    tok0[known] = rng.integers(0, 1024, known.sum())
    tok0[1, 1:] = rng.integers(0, 1024, 256)
    tok0[1, 17] = MASK                                        # one unknown
    tok0[2, 1:] = rng.integers(0, 1024, 256)                  # none
    lg = (rng.standard_normal((3, 257, 2025)) * 3).astype(np.float32)
    _run(ctx, lambda s, t: lg, tok0, [1, 2, 3], 8, steps=[5, 6, 7])
    _run(ctx, lambda s, t: lg, _start(3, 257, rng), [4, 5, 6], 8, choice_temp=0.0, steps=[0, 1])


def test_decode_small_shapes_and_many_images(ctx):
    print("decode S=65 CB=64 V=65 and B=70", flush=True)
    rng = np.random.default_rng(3)
    tok0 = np.full((2, 65), 64, np.int32)
    tok0[:, 0] = 5
    lg = (rng.standard_normal((2, 65, 65)) * 2).astype(np.float32)
    _run(ctx, lambda s, t: lg, tok0, [9, 10], 6, CB=64, n_tokens=64, mask_id=64)
    B = 70
    seeds = list(range(1000, 1000 + B))

    def logits(step, _):
        return (rng.standard_normal((B, 257, 1024)) * 2).astype(np.float32)

    _run(ctx, logits, _start(B, 257, rng), seeds, 8, steps=[0, 1, 2])


def test_decode_rejects_bad_args(ctx):
    state = ctx.alloc(ema.decode_state_bytes(1))
    work = ctx.alloc(ema.decode_work_bytes(1, 600))
    buf = ctx.alloc(600 * 2025 * 4)
    ctx.decode_init([1], state)
    for args in [dict(S=513, CB=1024, step=0), dict(S=257, CB=100, step=0),
                 dict(S=257, CB=2048, step=0), dict(S=257, CB=1024, step=8)]:
        with pytest.raises(ema.MghError):
            ctx.decode_step(state, work, buf, 1, args["S"], 2025, args["CB"], MASK, 256,
                            args["step"], 8, 4.5, buf, buf)
    for b in (state, work, buf):
        ctx.free(b)


@pytest.fixture(scope="module")
def q4_model(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("gen") / "m_q4.gguf")
    mg_gguf.write_model(p, n_layer=2, quant="q4_k", seed=8)
    return p


@pytest.mark.parametrize("algo", [1, 2, 3])
def test_generate_matches_host_loop(q4_model, algo):
    classes, seeds, steps = [207, 3], [42, 2**40 + 1], 8
    print(f"generate B=2 (q4_k, 2 layers, algo {algo}) vs host loop", flush=True)
    with rt.TransformerRuntime(q4_model, algo=algo) as m:
        got = m.generate(classes, seeds, steps)
        again = m.generate(classes, seeds, steps)
        other = m.generate(classes, [7, 8], steps)
        S = m.hparams["n_tokens"] + 1
        tok = np.full((2, S), MASK, np.int32)
        tok[:, 0] = np.asarray(classes) + 1024
        for step in range(steps):
            logits = m.forward(tok)
            tok, res = oracle.decode_step(logits, tok, step, steps, seeds, 2 * S * step,
                                          choice_temp=4.5)
    print(f"  mismatches {int((got != res[:, 1:]).sum())}")
    assert np.array_equal(got, res[:, 1:])
    assert np.array_equal(got, again)
    assert not np.array_equal(got, other)
    assert got.min() >= 0 and got.max() < 1024


def test_generate_full_cfg5(tmp_path):
    """cfg5 at full size: 24 Q4_K layers, 64 images x 257 tokens, 8 steps from all-masked,
    dequant-fp16 path. The device-resident generate equals the same loop run from the host
    (the runtime's forward read back, then the oracle step) token for token, repeats
    bit-identically, and ends with every position a codebook id."""
    path = str(tmp_path / "cfg5.gguf")
    mg_gguf.write_model(path, n_layer=24, quant="q4_k", seed=9)
    B, steps = 64, 8
    rng = np.random.default_rng(5)
    classes = [int(c) for c in rng.integers(0, 1000, B)]
    seeds = [int(s) for s in rng.integers(0, 2**62, B)]
    print("generate cfg5 full size: 24 layers q4_k, B=64, 8 steps", flush=True)
    with rt.TransformerRuntime(path, algo=2) as m:
        got = m.generate(classes, seeds, steps)
        again = m.generate(classes, seeds, steps)
        S = m.hparams["n_tokens"] + 1
        tok = np.full((B, S), MASK, np.int32)
        tok[:, 0] = np.asarray(classes) + 1024
        for step in range(steps):
            logits = m.forward(tok)
            tok, res = oracle.decode_step(logits, tok, step, steps, seeds, 2 * S * step,
                                          choice_temp=4.5)
    print(f"  mismatches {int((got != res[:, 1:]).sum())}", flush=True)
    assert np.array_equal(got, res[:, 1:])
    assert np.array_equal(got, again)
    assert got.min() >= 0 and got.max() < 1024
