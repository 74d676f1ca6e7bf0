"""Batched prompt processing (mcpm_engine_prefill, MFMA GEMMs) against the
per-token decode path: the KV cache rows of every layer must be bit-identical
to those left by one forward per token, and the generated continuation the
same.  The per-token path itself is checked against the oracle elsewhere;
the greedy test below also checks prefill + decode against the oracle."""
import numpy as np
import pytest

import mcpm
import oracle as O
from conftest import announce, assert_bits

pytestmark = pytest.mark.gpu

# (layers, dim, heads, kv heads, head_dim, ffn, vocab, mix, prompt length)
CASES = [
    (2, 2304, 32, 8, 64, 5760, 4096, 0, 100),   # 2.4B layer shape, Q6_K v/down, crosses a 64-position chunk
    (3, 2304, 32, 8, 64, 5760, 4096, 1, 40),    # llama-style mix: Q4_K down in some layers
    (2, 512, 8, 2, 64, 1400, 2000, 0, 300),     # q-dim 512 (2 blocks), 5 attention chunks
    (2, 256, 4, 2, 64, 512, 300, 0, 130),       # q-dim 256 (1 block), ffn padded 512
    (2, 512, 8, 2, 64, 1400, 2000, 0, 1100),    # two batched passes (1024 + 75 tokens), 18 chunks
]


def _run(eng, prompt, n_gen, prefill):
    eng.set_prefill(prefill)
    eng.init_kv_cache(len(prompt) + n_gen + 4)
    toks = list(eng.generate_greedy(prompt, n_gen))
    kv = [eng.read_kv(l, 0, len(prompt) - 1) for l in range(eng.cfg.n_layers)]
    return toks, kv


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"L{c[0]}-d{c[1]}-h{c[2]}-mix{c[7]}-p{c[8]}")
def test_prefill_kv_and_tokens_match_per_token(ctx, case):
    L, D, NH, NKV, HD, F, V, mix, n_prompt = case
    cfg = mcpm.make_config(L, D, NH, NKV, HD, F, V)
    img = mcpm.synth_gguf(cfg, seed=4242, mix=mix)
    prompt = np.random.default_rng(7).integers(0, V, n_prompt).astype(np.int32)
    announce(f"prefill case {case}")
    eng = mcpm.Engine(ctx, image=img)
    try:
        want_toks, want_kv = _run(eng, prompt, 6, prefill=False)
        got_toks, got_kv = _run(eng, prompt, 6, prefill=True)
    finally:
        eng.free()
    for l in range(L):
        assert_bits(got_kv[l][0], want_kv[l][0])
        assert_bits(got_kv[l][1], want_kv[l][1])
    assert got_toks == want_toks


def test_prefill_greedy_matches_oracle(ctx):
    cfg = mcpm.make_config(2, 512, 8, 2, 64, 1400, 2000)
    img = mcpm.synth_gguf(cfg, seed=31, mix=0)
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, 2000, 70)]
    announce("prefill greedy vs oracle")
    eng = mcpm.Engine(ctx, image=img)
    try:
        eng.set_prefill(True)
        eng.init_kv_cache(96)
        got = list(eng.generate_greedy(prompt, 10))
    finally:
        eng.free()
    om = O.OracleModel(img)
    want = list(om.generate_greedy(prompt, 10))
    om.close()
    assert got == want


def test_prefill_sampled_matches_per_token(ctx):
    cfg = mcpm.make_config(2, 512, 8, 2, 64, 1400, 2000)
    img = mcpm.synth_gguf(cfg, seed=5, mix=0)
    prompt = np.random.default_rng(11).integers(0, 2000, 90).astype(np.int32)
    announce("prefill sampled")
    eng = mcpm.Engine(ctx, image=img)
    try:
        out = []
        for pf in (False, True):
            eng.set_prefill(pf)
            eng.init_kv_cache(128)
            out.append(list(eng.generate_sampled(prompt, 16, 0.8, 0.95, 1234)))
    finally:
        eng.free()
    assert out[0] == out[1]


def test_prefill_rejects_bad_arguments(ctx):
    cfg = mcpm.make_config(1, 256, 4, 2, 64, 512, 300)
    eng = mcpm.Engine(ctx, image=mcpm.synth_gguf(cfg, seed=1))
    try:
        with pytest.raises(mcpm.McpmError):
            eng.prefill([1, 2, 3])  # no KV cache yet
        eng.init_kv_cache(8)
        with pytest.raises(mcpm.McpmError):
            eng.prefill(list(range(9)))  # past the capacity
        with pytest.raises(mcpm.McpmError):
            eng.prefill([0, 300])  # token out of range
        eng.prefill([])
    finally:
        eng.free()
