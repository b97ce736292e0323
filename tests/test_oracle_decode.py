"""Pins of the oracle's iterative-decoding step (oracle/mg_oracle_decode.cpp), CPU only.

The oracle restates src/mg-generate.cpp:82-121 with the same standard-library engine and
distributions, so what needs pinning is (a) the engine and the draw-to-double conversion the
device restates, and (b) that the step consumes the stream and applies the schedule as the
reference text says. Each check below is a closed form or an invariant a plausible mistake
breaks (wrong draw index or order, an off-by-one in the categorical search, a wrong schedule
term, known tokens treated as unknown):
  * the C++ standard's known answer for mt19937_64 ([rand.predef]: the 10000th output of a
    default-seeded engine is 9981545732273789042);
  * uniform_real_distribution<double>(a, b) == generate_canonical(x) * (b - a) + a with
    generate_canonical(x) = x / 2^64 over the engine's raw outputs;
  * uniform logits over the codebook: every probability is exactly 2^-10, so position s samples
    ceil(1024 u_s) - 1 with u_s the s-th draw of the step, and the re-masked positions are the
    ones with the smallest Gumbel noise, drawn from stream positions S..2S-1;
  * a code boosted by +60 is always sampled (argmax limit); logits past the codebook are ignored;
  * choice temperature 0: the re-masked samples are the least probable ones;
  * cosine schedule counts over 8 steps: 251, 236, 212, 181, 142, 97, 49 positions masked, and
    at the last step (zero temperature, all confidences tied) none;
  * known tokens keep their value and are never re-masked; one unknown left is re-masked (the
    cutoff is then +inf), none left changes nothing;
  * the reference's own generate() (src/mg-generate.cpp:39-123, compiled from its source into
    oracle/_ref) driven through its TransformerFwd / VqganFwd hooks with the same logits: the
    oracle loop feeds every step's forward the same tokens and ends on the same grid, over
    several seeds, class ids and choice temperatures.
"""
import math

import numpy as np
import pytest

import oracle
from oracle import ref

S, V, CB, MASK, NT = 257, 2025, 1024, 2024, 256


def _start(B, rng=None, cls=None):
    tok = np.full((B, S), MASK, np.int32)
    tok[:, 0] = 1024 + (np.arange(B) * 37 % 1000 if cls is None else np.asarray(cls))
    return tok


def test_mt19937_64_known_answer():
    assert int(oracle.mt64_draws(5489, 10000)[-1]) == 9981545732273789042


@pytest.mark.parametrize("seed", [0, 42, 5489, 2**63 + 99])
@pytest.mark.parametrize("a,b", [(0.0, 1.0), (1e-12, 1.0)])
def test_uniform_draws_are_canonical(seed, a, b):
    x = oracle.mt64_draws(seed, 4096)
    u = x.astype(np.float64) / 2.0**64
    u[u >= 1.0] = np.nextafter(1.0, 0.0)
    want = u * (b - a) + a
    got = oracle.uniform_draws(seed, a, b, 4096)
    assert np.array_equal(got.view(np.uint64), want.view(np.uint64))


@pytest.mark.parametrize("seed", [7, 12345])
def test_uniform_logits_closed_form(seed):
    logits = np.zeros((1, S, V), np.float32)
    logits[:, :, CB:] = 100.0                      # outside the codebook: never sampled
    tok0 = _start(1)
    tok, res = oracle.decode_step(logits, tok0, 0, 8, [seed], 0)
    u = oracle.uniform_draws(seed, 0.0, 1.0, 2 * S)[:S]
    want = np.maximum(np.ceil(u * 1024.0).astype(np.int64) - 1, 0)
    assert res[0, 0] == tok0[0, 0]                 # known class token kept
    assert np.array_equal(res[0, 1:], want[1:])
    # re-masked: the 251 unknown positions with the smallest Gumbel noise
    g = -np.log(-np.log(oracle.uniform_draws(seed, 1e-12, 1.0, 2 * S)[S:]))
    masked = tok[0] == MASK
    assert masked.sum() == 251 and not masked[0]
    assert g[masked].max() < g[1:][~masked[1:]].min()
    assert np.array_equal(tok[0][~masked], res[0][~masked])


def test_draws_continue_across_steps():
    """Step t starts 2*S draws into the stream: the categorical draws of step 1 are stream
    positions 2S..3S-1."""
    seed = 99
    logits = np.zeros((1, S, V), np.float32)
    tok, _ = oracle.decode_step(logits, _start(1), 0, 8, [seed], 0)
    _, res = oracle.decode_step(logits, tok, 1, 8, [seed], 2 * S)
    u = oracle.uniform_draws(seed, 0.0, 1.0, 3 * S)[2 * S:]
    want = np.maximum(np.ceil(u * 1024.0).astype(np.int64) - 1, 0)
    unknown = tok[0] == MASK
    assert np.array_equal(res[0][unknown], want[unknown])
    assert np.array_equal(res[0][~unknown], tok[0][~unknown])


def test_argmax_limit_and_known_tokens():
    rng = np.random.default_rng(3)
    B = 2
    logits = rng.standard_normal((B, S, V)).astype(np.float32)
    code = rng.integers(0, CB, (B, S))
    np.put_along_axis(logits, code[..., None], 60.0, axis=2)
    tok0 = _start(B)
    known = rng.random((B, S)) < 0.3
    known[:, 0] = False
    tok0[known] = rng.integers(0, CB, known.sum())
    tok, res = oracle.decode_step(logits, tok0, 2, 8, [5, 6], 4 * S)
    for b in range(B):
        unk = tok0[b] == MASK
        assert np.array_equal(res[b][unk], code[b][unk])
        assert np.array_equal(res[b][~unk], tok0[b][~unk])
        assert np.array_equal(tok[b][~unk], tok0[b][~unk])   # known: never re-masked


def test_temperature_zero_remasks_least_probable():
    rng = np.random.default_rng(4)
    logits = (rng.standard_normal((1, S, V)) * 2).astype(np.float32)
    tok, res = oracle.decode_step(logits, _start(1), 3, 8, [11], 6 * S, choice_temp=0.0)
    x = logits[0, :, :CB].astype(np.float64)
    p = np.exp(x - x.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    ps = p[np.arange(1, S), res[0, 1:]]           # position 0 holds the class token
    masked = tok[0, 1:] == MASK
    n = int(math.floor(NT * math.cos(math.pi / 2 * 4 / 8)))
    assert masked.sum() == n and tok[0, 0] == res[0, 0]
    assert ps[masked].max() <= ps[~masked].min()


def test_cosine_schedule_counts():
    seed = 2024
    logits = np.zeros((1, S, V), np.float32)
    tok = _start(1)
    counts = []
    for t in range(8):
        tok, res = oracle.decode_step(logits, tok, t, 8, [seed], 2 * S * t)
        counts.append(int((tok[0] == MASK).sum()))
    want = []
    unknown = NT
    for t in range(8):
        ml = math.floor(NT * math.cos(math.pi / 2 * (t + 1) / 8))
        ml = max(1, min(ml, unknown - 1))
        want.append(ml)
        unknown = ml
    assert want == [251, 236, 212, 181, 142, 97, 49, 1]
    assert counts[:7] == want[:7]
    # last step: temperature * (1 - ratio) = 0, so every unknown position has the same
    # confidence log(2^-10); the cutoff (2nd smallest) equals them all and `conf < cutoff`
    # re-masks none
    assert counts[7] == 0
    assert not (res[0] == MASK).any()              # the step's samples fill every position


def test_one_or_no_unknown_left():
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((2, S, V)).astype(np.float32)
    tok0 = rng.integers(0, CB, (2, S)).astype(np.int32)
    tok0[:, 0] = 1500
    tok0[0, 17] = MASK                             # image 0: one unknown, image 1: none
    tok, res = oracle.decode_step(logits, tok0, 6, 8, [1, 2], 12 * S)
    assert tok[0, 17] == MASK and res[0, 17] != MASK
    keep = np.ones(S, bool)
    keep[17] = False
    assert np.array_equal(tok[0][keep], tok0[0][keep])
    assert np.array_equal(tok[1], tok0[1]) and np.array_equal(res[1], tok0[1])


@pytest.fixture(scope="module")
def gen_model(tmp_path_factory):
    from tests import mg_gguf
    p = str(tmp_path_factory.mktemp("gen") / "gen.gguf")
    mg_gguf.write_model(p, n_layer=1, quant="f32", seed=9)
    return p


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref/libmgref.so not built (needs /root/reference)")
@pytest.mark.parametrize("seed,cls,temp,scale", [(42, 207, 4.5, 3.0), (7, 0, 1.0, 3.0), (2024, 999, -1.0, 1.0),
                                                 (1, 512, 0.0, 6.0), (123456789, 88, 4.5, 0.3)])
def test_decode_loop_equals_reference_generate(gen_model, seed, cls, temp, scale):
    """8 steps of the oracle step against the reference's generate() on the same per-step
    logits: identical tokens into every forward and the identical final grid (a negative
    temperature selects the model's 4.5, as the reference does)"""
    steps = 8
    rng = np.random.default_rng(seed % 1000)
    logits = (rng.standard_normal((steps, S, V)) * scale).astype(np.float32)
    ref_tok, ref_grid = ref.generate(gen_model, cls, seed, steps, temp, logits)
    tok = _start(1, cls=[cls])
    ct = 4.5 if temp < 0 else temp
    for step in range(steps):
        assert np.array_equal(tok[0], ref_tok[step]), f"tokens into step {step}"
        tok, res = oracle.decode_step(logits[step][None], tok, step, steps, [seed], 2 * S * step, choice_temp=ct)
    assert np.array_equal(res[0, 1:], ref_grid)
