"""The device sampler (mcpm_sample_device, and the engine's sampled decode)
against the oracle's statement of its arithmetic (or_sample_blocked: the
steps of src/sampler.cpp:8-73 with running sums in blocked double), which
tests/test_oracle.py pins against exact arithmetic and against the
reference-order sampler.  Bar: the same token for every case and draw."""
import numpy as np
import pytest

import mcpm
import oracle as O
from conftest import P, announce

pytestmark = pytest.mark.gpu

# (n, logit scale, temperature, top_p): a full vocabulary, ragged sizes (one
# position, one past a block), flat and peaked distributions, no temperature
# (T = 1 and T <= 0), no cut (top_p 1 and 0) and a cut at the first token.
CASES = [
    (130560, 3.0, 0.8, 0.95), (130560, 0.02, 1.0, 0.95), (130560, 8.0, 1.3, 0.5),
    (4000, 3.0, 1.0, 1.0), (4000, 3.0, 0.0, 0.0), (4000, 1.0, 0.7, 1e-6),
    (257, 2.0, 0.9, 0.9), (1, 1.0, 0.8, 0.95), (300, 0.0, 1.0, 0.5),
    # the sort-free top-p path at its limits (top_p 0.998, the largest
    # vocabulary), one bucket of 130,560 equal p (ordered by id alone), and
    # just past the limit (the sorted path)
    (130560, 3.0, 1.0, 0.998), (524288, 2.0, 1.0, 0.95), (130560, 0.0, 1.0, 0.7), (130560, 3.0, 1.0, 0.999),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"n{c[0]}-s{c[1]}-T{c[2]}-p{c[3]}")
def test_device_sampler_matches_spec(ctx, case):
    n, scale, T, top_p = case
    orc = O.oracle()
    rng = np.random.default_rng(n + int(100 * scale))
    lg = (rng.standard_normal(n) * scale).astype(np.float32)
    if n > 10:
        lg[rng.integers(0, n, 16)] = lg[3]  # ties: ordered by id
    announce(f"device sampler {case}")
    dev = ctx.upload(lg)
    out = ctx.zeros(4)
    draws = [0.0, float(np.nextafter(np.float32(1), np.float32(0)))] + [float(np.float32(x)) for x in rng.random(10)]
    try:
        for r in draws:
            mcpm.check(ctx.lib.mcpm_sample_device(ctx.h, dev.ptr, n, T, top_p, r, out.ptr))
            got = int(ctx.download(out, np.int32, 1)[0])
            assert got == orc.or_sample_blocked(P(lg), n, T, top_p, r), r
    finally:
        ctx.sync()
        dev.free()
        out.free()


def test_device_sampler_rejects_bad_arguments(ctx):
    dev = ctx.upload(np.zeros(8, np.float32))
    out = ctx.zeros(4)
    try:
        for n, r in [(0, 0.5), (8, 1.0), (8, -0.1), (8, float("nan")), (524289, 0.5)]:
            with pytest.raises(mcpm.McpmError):
                mcpm.check(ctx.lib.mcpm_sample_device(ctx.h, dev.ptr, n, 1.0, 0.9, r, out.ptr))
    finally:
        ctx.sync()
        dev.free()
        out.free()


def _oracle_sampled(img, prompt, n_gen, T, top_p, seed, vocab, cont=None):
    """Greedy-loop twin with or_sample_blocked and the host's mt19937 draws;
    cont = (n_more, seed2) continues with a freshly seeded generator."""
    orc = O.oracle()
    om = O.OracleModel(img)
    om.init_kv(len(prompt) + n_gen + (cont[0] if cont else 0) + 4)
    lg = np.empty(vocab, np.float32)
    for p, t in enumerate(prompt):
        om.forward(int(t), p, lg)
    out, pos = [], len(prompt)
    plan = [(n_gen, seed)] + ([cont] if cont else [])
    for n, sd in plan:
        gen = np.zeros(625, np.uint32)
        orc.or_mt_seed(P(gen), sd)
        for _ in range(n):
            if out:
                om.forward(out[-1], pos, lg)
                pos += 1
            out.append(orc.or_sample_blocked(P(lg), vocab, T, top_p, orc.or_mt_uniform01(P(gen))))
    om.close()
    return out


def test_engine_sampled_and_continuation_match_oracle(ctx):
    cfg = mcpm.make_config(2, 512, 8, 2, 64, 1400, 3000)
    img = mcpm.synth_gguf(cfg, seed=77, mix=0)
    prompt = [int(t) for t in np.random.default_rng(8).integers(0, 3000, 20)]
    announce("engine sampled + continuation")
    eng = mcpm.Engine(ctx, image=img)
    try:
        eng.init_kv_cache(64)
        first = list(eng.generate_sampled(prompt, 12, 0.9, 0.9, 99))
        eng.decode_sampled(0, 0.9, 0.9, 5)  # nothing to do
        with pytest.raises(mcpm.McpmError):
            eng.decode_sampled(4, 0.9, 0.9, 5)  # the list holds 12 tokens
        eng.generate_sampled(prompt, 20, 0.9, 0.9, 99)
        eng.sync()
    finally:
        eng.free()
    assert first == _oracle_sampled(img, prompt, 12, 0.9, 0.9, 99, 3000)
    eng = mcpm.Engine(ctx, image=img)
    try:
        eng.init_kv_cache(64)
        eng.set_prefill(False)
        eng.generate_sampled(prompt, 20, 0.9, 0.9, 99)  # room for 20
        eng.init_kv_cache(64)
        eng.generate_sampled(prompt, 6, 0.9, 0.9, 99)
        eng.decode_sampled(6, 0.9, 0.9, 123)
        got = list(eng.tokens(12))
        # greedy continuation after a sampled run follows the argmax
        eng.decode_steps(2)
        both = list(eng.tokens(14))
    finally:
        eng.free()
    assert got == _oracle_sampled(img, prompt, 6, 0.9, 0.9, 99, 3000, cont=(6, 123))
    assert both[:12] == got
