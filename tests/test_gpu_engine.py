"""The decode engine (GGUF load, KV cache, graph-captured forward, decode loops)
against the CPU oracle and the reference's golden tokens."""
import hashlib
import os
import tempfile

import numpy as np
import pytest

import mcpm
import oracle as O
from conftest import announce, assert_bits, golden

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=4, dim=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=1400, vocab=4000)
SMALL_MIX = 2  # the reference file's layout: Q4_K token_embd, untied Q6_K output


@pytest.fixture(scope="module")
def small_image():
    g = golden("small_model_greedy.npz")
    assert int(g["mix"]) == SMALL_MIX
    img = mcpm.synth_gguf(mcpm.make_config(**SMALL), seed=int(g["seed"]), mix=SMALL_MIX)
    assert hashlib.sha256(img.tobytes()).hexdigest() == str(g["image_sha"]), "model generator changed"
    return img


@pytest.fixture(scope="module")
def small_engine(ctx, small_image):
    e = mcpm.Engine(ctx, image=small_image)
    e.init_kv_cache(256)
    yield e
    e.free()


def test_config_from_gguf(small_engine):
    c = small_engine.cfg
    assert (c.n_layers, c.dim, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn, c.ffn_pad, c.vocab) == \
        (4, 512, 8, 2, 64, 1400, 1536, 4000)
    assert c.tied_embeddings == 0  # separate output.weight
    assert abs(c.rope_base - 10000.0) < 1e-3


def test_forward_logits_bit_exact(small_engine, small_image):
    om = O.OracleModel(small_image)
    om.init_kv(256)
    rng = np.random.default_rng(11)
    toks = rng.integers(0, 4000, 70)
    want = np.empty(4000, np.float32)
    for pos, t in enumerate(toks):
        announce(f"small forward pos={pos}")
        got, am = small_engine.forward(int(t), pos)
        om.forward(int(t), pos, want)
        assert_bits(got, want)
        assert am == int(np.argmax(want))


@pytest.mark.parametrize("graph", [True, False])
def test_greedy_matches_oracle_and_reference(small_engine, small_image, graph):
    g = golden("small_model_greedy.npz")
    small_engine.set_graph(graph)
    announce(f"small greedy graph={graph}")
    got = small_engine.generate_greedy(g["prompt"], len(g["tokens"]))
    om = O.OracleModel(small_image)
    want = om.generate_greedy(g["prompt"], len(g["tokens"]))
    np.testing.assert_array_equal(got, want)
    assert len(set(got.tolist())) > 8, "a degenerate (near-constant) token sequence pins little"
    # the reference's own ops (one thread), for as long as the oracle agrees
    # with them: the untied head's top-2 margins are small, and the
    # reference's -ffast-math RMS and lane sums flip an argmax after that
    k = int(g["reference_agree_steps"])
    assert k >= 16
    np.testing.assert_array_equal(got[:k], g["tokens"][:k])
    small_engine.set_graph(True)


def test_forward_context_errors(small_engine):
    with pytest.raises(mcpm.McpmError) as ei:
        small_engine.forward(1, 256)
    assert ei.value.code == -4
    with pytest.raises(mcpm.McpmError) as ei:
        small_engine.forward(1, 10, max_seq_len=10)
    assert ei.value.code == -4
    with pytest.raises(mcpm.McpmError):
        small_engine.forward(4000, 0)


def test_load_from_file_and_errors(ctx, small_image):
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "m.gguf")
        small_image.tofile(p)
        e = mcpm.Engine(ctx, gguf_path=p)
        assert e.cfg.n_layers == 4
        e.free()
        bad = os.path.join(d, "bad.gguf")
        small_image[: len(small_image) // 2].tofile(bad)
        with pytest.raises(mcpm.McpmError) as ei:
            mcpm.Engine(ctx, gguf_path=bad)
        assert ei.value.code == -6
    with pytest.raises(mcpm.McpmError) as ei:
        mcpm.Engine(ctx, gguf_path="/nonexistent/model.gguf")
    assert ei.value.code == -5


def _oracle_sampled(image, prompt, n, temperature, top_p, seed):
    om = O.OracleModel(image)
    om.init_kv(64)
    orc = O.oracle()
    gen = np.zeros(625, np.uint32)  # or_mt19937 state
    orc.or_mt_seed(gen.ctypes.data, seed)
    lg = np.empty(4000, np.float32)
    for p, t in enumerate(prompt):
        om.forward(int(t), p, lg)
    out = []
    for i in range(n):
        nxt = orc.or_sample_blocked(lg.ctypes.data, 4000, temperature, top_p, orc.or_mt_uniform01(gen.ctypes.data))
        out.append(nxt)
        if i < n - 1:
            om.forward(nxt, len(prompt) + i, lg)
    return np.array(out, np.int32)


def test_sampled_matches_oracle_sampler(small_engine, small_image):
    """Sampled generation against the oracle's model and sampler, one after
    another on one engine: settings whose sampler runs inside the captured
    token graph (a cut at 0.95 and at 0.5, no cut, a temperature of 1, the
    draw read on the device per step) and a cut above 0.998 (the sort, after
    the graph), each change of settings capturing the graph again."""
    prompt = np.arange(10, 26, dtype=np.int32)
    for temperature, top_p, seed in [(0.8, 0.95, 1234), (0.9, 0.999, 77), (1.0, 1.0, 5), (0.7, 0.5, 9),
                                     (0.8, 0.95, 1234)]:
        announce(f"small sampled T={temperature} top_p={top_p}")
        got = small_engine.generate_sampled(prompt, 24, temperature, top_p, seed)
        np.testing.assert_array_equal(got, _oracle_sampled(small_image, prompt, 24, temperature, top_p, seed))


@pytest.mark.parametrize("prefill", [False, True])
def test_kernel_timing_counts(small_engine, prefill):
    small_engine.set_prefill(prefill)
    small_engine.set_kernel_timing(mcpm.KC_GATE_UP)
    small_engine.generate_greedy(np.array([1, 2, 3], np.int32), 2)
    t, n = small_engine.kernel_time()
    small_engine.set_kernel_timing(-1)
    small_engine.set_prefill(True)
    # per-token path: 3 prompt positions + 1 decode step, one gate/up launch
    # per layer each; with prefill the first two prompt tokens go through the
    # batched GEMMs (not timed classes)
    assert n == (2 if prefill else 4) * small_engine.cfg.n_layers and t > 0


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).view(np.uint8).tobytes()).hexdigest()


@pytest.fixture(scope="module", params=["persistent", "five-launch"])
def full_engine(ctx, request):
    """The 2.4B-shaped model of the benchmark (40 layers, 2304 hidden, 32/8
    heads of 64, FFN 5760, vocab 130560, tied Q6_K head, Q6_K v/down), KV
    capacity 1536: through the default decode path (every layer of a token
    in one persistent launch, the instance compiled for this shape) and
    through five launches per layer."""
    g = golden("full_model_oracle.npz")
    announce(f"full model synth ({request.param})")
    img = mcpm.synth_gguf(mcpm.config_2p4b(), seed=int(g["seed"]), mix=0)
    assert _sha(img) == str(g["image_sha"]), "model generator changed"
    e = mcpm.Engine(ctx, image=img)
    del img
    if request.param == "five-launch":
        e.set_persistent(False)
    e.init_kv_cache(1536)
    if request.param == "persistent":
        assert e.uses_persistent() and e.persistent_fixed_shape(), "the default decode path of the 2.4B shape"
    else:
        assert not e.uses_persistent()
    yield e
    e.free()


def test_full_model_greedy_256(full_engine):
    """The benchmark's greedy workload: the 32-token prompt and 256 greedy
    steps reproduce the CPU oracle bit for bit -- every token, and every
    step's logits (SHA-256) through per-token forwards."""
    g = golden("full_model_oracle.npz")
    e = full_engine
    n = len(g["tokens"])
    assert n == 256
    announce("full model greedy 32+256 (device loop)")
    toks = e.generate_greedy(g["prompt"], n)
    np.testing.assert_array_equal(toks, g["tokens"])
    announce("full model per-step logits")
    prompt = [int(t) for t in g["prompt"]]
    feed = prompt + [int(t) for t in g["tokens"][:-1]]
    n_p = len(prompt)
    for pos, t in enumerate(feed):
        logits, am = e.forward(t, pos)
        if pos >= n_p - 1:
            step = pos - (n_p - 1)
            assert _sha(logits) == str(g["logits_sha"][step]), f"logits differ at step {step}"
            assert am == int(g["tokens"][step])


def test_full_model_long_context_sampled(full_engine):
    """The long-context sampled workload at full size: a 1024-token random
    prompt through the batched MFMA prefill, then 512 tokens sampled at
    temperature 0.8 / top-p 0.95 by the device sampler, the KV cache reaching
    1535 of 1536 rows.  Against the CPU oracle (per-token forwards,
    or_sample_blocked on the same std::mt19937 draws): every token, the K and
    V rows of three layers (SHA-256 over all 1535 positions), and the logits
    (SHA-256) of every 32nd step and the last."""
    g = golden("c5_long_sampled.npz")
    e = full_engine
    assert e.uses_prefill()
    prompt = g["prompt"]
    n_gen = len(g["tokens"])
    announce(f"full model prefill {len(prompt)} + sampled {n_gen}")
    toks = e.generate_sampled(prompt, n_gen, float(g["temperature"]), float(g["top_p"]), int(g["sample_seed"]))
    np.testing.assert_array_equal(toks, g["tokens"])
    rows = int(g["kv_rows"])
    for i, l in enumerate(g["kv_layers"]):
        announce(f"full model KV rows layer {int(l)}")
        k, v = e.read_kv(int(l), 0, rows)
        assert _sha(k) == str(g["k_sha"][i]), f"K rows of layer {int(l)} differ"
        assert _sha(v) == str(g["v_sha"][i]), f"V rows of layer {int(l)} differ"
    # a forward at an already-written position rewrites its K/V row with the
    # same values and returns that step's logits
    announce("full model sampled-step logits")
    n_p = len(prompt)
    for i, step in enumerate(g["logits_steps"]):
        step = int(step)
        tok = int(prompt[-1]) if step == 0 else int(g["tokens"][step - 1])
        logits, _ = e.forward(tok, n_p - 1 + step)
        assert _sha(logits) == str(g["logits_sha"][i]), f"logits differ at step {step}"


@pytest.mark.parametrize("name", ["refshape_1layer_greedy.npz", "refshape_3layer_greedy.npz",
                                  "refshape_layout_greedy.npz"])
def test_reference_geometry_tokens(ctx, name):
    """The reference's own MiniCPM5-2B geometry (hidden 2048, 16/2 heads of
    128, FFN 6144, rope base 5e6) at reduced depth: tokens equal the
    reference's for as long as the oracle's do (all 64 steps for one layer
    and for the reference file's layout), and equal the oracle's for all 64
    steps.  refshape_layout_greedy.npz is the reference file's own layout
    (include/minicpm_metadata.h:30-32): a Q4_K token_embd, a separate Q6_K
    output.weight at the full 130560 rows, use_more_bits v/down types."""
    g = golden(name)
    L, D, NH, NKV, HD, F, V = [int(v) for v in g["config"]]
    mix = int(g["mix"]) if "mix" in g else 0
    cfg = mcpm.make_config(L, D, NH, NKV, HD, F, V, rope_base=float(g["rope_base"]))
    img = mcpm.synth_gguf(cfg, seed=int(g["seed"]), mix=mix)
    assert _sha(img) == str(g["image_sha"]), "model generator changed"
    e = mcpm.Engine(ctx, image=img)
    if mix == 2:
        assert e.cfg.tied_embeddings == 0
    e.init_kv_cache(96)
    n = len(g["tokens"])
    announce(f"{name} greedy")
    got = e.generate_greedy(g["prompt"], n)
    k = int(g["reference_agree_steps"])
    np.testing.assert_array_equal(got[:k], g["tokens"][:k])
    want = O.OracleModel(img).generate_greedy(g["prompt"], n)
    np.testing.assert_array_equal(got, want)
    e.free()


@pytest.mark.parametrize("n_prompt", [1100, 2200])
def test_long_context_greedy_matches_oracle(ctx, n_prompt):
    """Prompts of 1100 and 2200 tokens (18 and 35 attention chunks per head)
    and 8 greedy tokens on a model whose O projection combines the attention
    partials in its prologue (q dim 1024: 4 blocks), against the oracle: the
    combine's preloaded chunks, its first batch, and (2200) its later batches
    of partials and maxima."""
    cfg = mcpm.make_config(2, 1024, 16, 4, 64, 2048, 1000)
    img = mcpm.synth_gguf(cfg, seed=404, mix=0)
    prompt = [int(t) for t in np.random.default_rng(17).integers(0, 1000, n_prompt)]
    announce(f"long context greedy vs oracle ({n_prompt}-token prompt)")
    eng = mcpm.Engine(ctx, image=img)
    try:
        eng.init_kv_cache(n_prompt + 20)
        got = list(eng.generate_greedy(prompt, 8))
    finally:
        eng.free()
    om = O.OracleModel(img)
    want = list(om.generate_greedy(prompt, 8))
    om.close()
    assert got == want


def test_per_head_attention_matches_oracle(ctx, monkeypatch):
    """Short contexts run one attention work group per kv head that combines
    its chunks and hands the O projection Q8_K blocks; longer ones run the
    splits and the O projection's combine.  With the per-head path allowed up
    to its limit (MCPM_ATTN_Q8K=8: 8 chunks, two rounds of its four chunk
    groups), logits bit-identical to the oracle at every position 0..519
    (both paths, and the switch between their graphs at 512); greedy tokens
    across 512 and across the default switch (192) equal to the oracle's and
    to the split path's alone (MCPM_ATTN_Q8K=0)."""
    cfg = mcpm.make_config(2, 1024, 16, 4, 64, 2048, 1000)
    img = mcpm.synth_gguf(cfg, seed=515, mix=0)
    rng = np.random.default_rng(23)
    toks = [int(t) for t in rng.integers(0, 1000, 520)]
    om = O.OracleModel(img)
    om.init_kv(600)
    want = np.empty(1000, np.float32)
    monkeypatch.setenv("MCPM_ATTN_Q8K", "8")
    eng = mcpm.Engine(ctx, image=img)
    try:
        eng.init_kv_cache(600)
        announce("per-kv-head attention: forward at positions 0..519")
        for pos, t in enumerate(toks):
            got, _ = eng.forward(t, pos)
            om.forward(t, pos, want)
            assert_bits(got, want)
    finally:
        eng.free()
    om.close()
    om = O.OracleModel(img)
    want_long = list(om.generate_greedy(toks[:490], 30))
    om.close()
    om = O.OracleModel(img)
    want_short = list(om.generate_greedy(toks[:170], 40))
    om.close()
    for mode in ("8", None, "0"):
        if mode is None:
            monkeypatch.delenv("MCPM_ATTN_Q8K", raising=False)
        else:
            monkeypatch.setenv("MCPM_ATTN_Q8K", mode)
        announce(f"per-kv-head attention: greedy, MCPM_ATTN_Q8K={mode}")
        eng = mcpm.Engine(ctx, image=img)
        try:
            eng.init_kv_cache(600)
            eng.set_prefill(False)
            assert list(eng.generate_greedy(toks[:490], 30)) == want_long
            assert list(eng.generate_greedy(toks[:170], 40)) == want_short
        finally:
            eng.free()


@pytest.mark.parametrize("prefill", [True, False])
def test_generate_at_reuses_cached_rows(ctx, prefill):
    """mcpm_engine_generate_{greedy,sampled}_at: a second turn that keeps the
    first turn's KV rows (conversation + response but its last token) and
    runs only its new tokens, or keeps a shorter prefix, generates the tokens
    of the whole conversation run from position 0 and leaves bit-identical
    KV rows."""
    cfg = mcpm.make_config(2, 512, 8, 2, 64, 1400, 2000)
    img = mcpm.synth_gguf(cfg, seed=606, mix=0)
    rng = np.random.default_rng(9)
    turn1 = [int(t) for t in rng.integers(0, 2000, 70)]
    user2 = [int(t) for t in rng.integers(0, 2000, 90)]
    announce(f"generate_at reuse (prefill={prefill})")
    eng = mcpm.Engine(ctx, image=img)
    try:
        eng.set_prefill(prefill)
        cap = 400
        eng.init_kv_cache(cap)
        resp1 = list(eng.generate_greedy(turn1, 12))
        conv2 = turn1 + resp1 + user2
        n2 = len(conv2)
        keep = len(turn1) + len(resp1) - 1
        got = list(eng.generate_greedy_at(conv2[keep:], keep, 10))
        kv_got = [eng.read_kv(l, 0, n2 + 9) for l in range(cfg.n_layers)]
        # a shorter kept prefix (an edited turn): positions 30.. rerun
        got_short = list(eng.generate_greedy_at(conv2[30:], 30, 10))
        sampled = list(eng.generate_sampled_at(conv2[keep:], keep, 10, 0.9, 0.9, 77))
        eng.init_kv_cache(cap)
        want = list(eng.generate_greedy(conv2, 10))
        kv_want = [eng.read_kv(l, 0, n2 + 9) for l in range(cfg.n_layers)]
        want_sampled = list(eng.generate_sampled(conv2, 10, 0.9, 0.9, 77))
        with pytest.raises(mcpm.McpmError):
            eng.generate_greedy_at(conv2, cap - len(conv2) + 1, 2)  # past the cache
    finally:
        eng.free()
    assert got == want and got_short == want and sampled == want_sampled
    for (kg, vg), (kw, vw) in zip(kv_got, kv_want):
        assert_bits(kg, kw)
        assert_bits(vg, vw)


def test_fused_ffn_block_matches_oracle(ctx, small_image, monkeypatch):
    """MCPM_FUSED_FFN=1: each layer's FFN block (gate/up, then down) as one
    launch with a grid barrier between the phases, the down weights loaded
    before the barrier.  Same tokens and bit-identical logits as the oracle,
    on the small model and on the first 32 steps of the 2.4B-shaped model."""
    monkeypatch.setenv("MCPM_FUSED_FFN", "1")
    g = golden("small_model_greedy.npz")
    announce("fused FFN: small model greedy")
    e = mcpm.Engine(ctx, image=small_image)
    try:
        e.init_kv_cache(256)
        got = e.generate_greedy(g["prompt"], len(g["tokens"]))
        want = O.OracleModel(small_image).generate_greedy(g["prompt"], len(g["tokens"]))
        np.testing.assert_array_equal(got, want)
        om = O.OracleModel(small_image)
        om.init_kv(64)
        lg = np.empty(4000, np.float32)
        for pos, t in enumerate(g["prompt"]):
            logits, _ = e.forward(int(t), pos)
            om.forward(int(t), pos, lg)
            assert_bits(logits, lg)
    finally:
        e.free()
    gf = golden("full_model_oracle.npz")
    announce("fused FFN: 2.4B-shaped model greedy 32+32")
    img = mcpm.synth_gguf(mcpm.config_2p4b(), seed=int(gf["seed"]), mix=0)
    e = mcpm.Engine(ctx, image=img)
    del img
    try:
        e.set_persistent(False)  # the fused FFN runs on the five-launch path
        e.init_kv_cache(128)
        np.testing.assert_array_equal(e.generate_greedy(gf["prompt"], 32), gf["tokens"][:32])
    finally:
        e.free()


@pytest.mark.parametrize("env", ["MCPM_FUSED_FFN", "MCPM_FUSED_ATTN"])
def test_grid_barrier_give_up_then_recovers(ctx, small_image, monkeypatch, env):
    """The fused kernels' grid barrier with a spin limit of 1 poll: a wait
    gives up, every work group leaves through its own bounded wait, and the
    call returns MCPM_ERR_HIP with the barrier state reset; with the default
    limit restored, the next calls give the oracle's logits bit for bit."""
    monkeypatch.setenv(env, "1")
    e = mcpm.Engine(ctx, image=small_image)
    try:
        e.init_kv_cache(64)
        prompt = np.arange(5, 21, dtype=np.int32)
        e.set_spin_limit(1)
        codes = []
        for i in range(6):
            announce(f"{env}: spin limit 1, call {i}")
            try:
                e.generate_greedy(prompt, 4)
            except mcpm.McpmError as err:
                codes.append(err.code)
                break
        assert codes == [mcpm.ERR_HIP], "no wait gave up at a spin limit of 1"
        e.set_spin_limit(0)
        announce(f"{env}: default spin limit after the give-up")
        om = O.OracleModel(small_image)
        om.init_kv(64)
        want = np.empty(4000, np.float32)
        for pos, t in enumerate(prompt):
            got, _ = e.forward(int(t), pos)
            om.forward(int(t), pos, want)
            assert_bits(got, want)
        np.testing.assert_array_equal(e.generate_greedy(prompt, 8),
                                      O.OracleModel(small_image).generate_greedy(prompt, 8))
    finally:
        e.free()


@pytest.mark.parametrize("case", ["small", "full32", "refshape", "long_8kv"])
def test_fused_qkv_attention_matches_oracle(ctx, small_image, monkeypatch, case):
    """MCPM_FUSED_ATTN=1: each layer's QKV GEMV and attention as one launch
    (q and the new K and V rows written through, a grid barrier, then the
    attention splits; each work group's first split's K and V rows loaded
    before the barrier and the row at pos read again after it).  Against the
    oracle: the small model's tokens and bit-identical logits at 70
    positions (two chunks), the 2.4B-shaped model's first 32 steps, the
    reference geometry (heads of 128, groups of 8, Q6_K v), and 2208
    per-token positions of a model with 8 kv heads, whose 35 chunks give
    280 splits: more than one per work group."""
    monkeypatch.setenv("MCPM_FUSED_ATTN", "1")
    if case == "small":
        g = golden("small_model_greedy.npz")
        announce("fused QKV+attention: small model")
        e = mcpm.Engine(ctx, image=small_image)
        try:
            e.init_kv_cache(256)
            # one launch per layer for QKV and attention together
            e.set_kernel_timing(mcpm.KC_ATTN)
            e.forward(1, 0)
            assert e.kernel_time()[1] == 0
            e.set_kernel_timing(mcpm.KC_QKV)
            e.forward(1, 0)
            assert e.kernel_time()[1] == e.cfg.n_layers
            e.set_kernel_timing(-1)
            got = e.generate_greedy(g["prompt"], len(g["tokens"]))
            np.testing.assert_array_equal(got, O.OracleModel(small_image).generate_greedy(g["prompt"], len(got)))
            om = O.OracleModel(small_image)
            om.init_kv(256)
            lg = np.empty(4000, np.float32)
            toks = np.random.default_rng(11).integers(0, 4000, 70)
            for pos, t in enumerate(toks):
                logits, _ = e.forward(int(t), pos)
                om.forward(int(t), pos, lg)
                assert_bits(logits, lg)
        finally:
            e.free()
    elif case == "full32":
        gf = golden("full_model_oracle.npz")
        announce("fused QKV+attention: 2.4B-shaped model greedy 32+32")
        img = mcpm.synth_gguf(mcpm.config_2p4b(), seed=int(gf["seed"]), mix=0)
        e = mcpm.Engine(ctx, image=img)
        del img
        try:
            e.set_persistent(False)  # the fused launch runs on the five-launch path
            e.init_kv_cache(128)
            np.testing.assert_array_equal(e.generate_greedy(gf["prompt"], 32), gf["tokens"][:32])
        finally:
            e.free()
    elif case == "refshape":
        g = golden("refshape_layout_greedy.npz")
        L, D, NH, NKV, HD, F, V = [int(v) for v in g["config"]]
        cfg = mcpm.make_config(L, D, NH, NKV, HD, F, V, rope_base=float(g["rope_base"]))
        img = mcpm.synth_gguf(cfg, seed=int(g["seed"]), mix=int(g["mix"]))
        announce("fused QKV+attention: reference geometry")
        e = mcpm.Engine(ctx, image=img)
        try:
            e.init_kv_cache(96)
            got = e.generate_greedy(g["prompt"], len(g["tokens"]))
        finally:
            e.free()
        np.testing.assert_array_equal(got, O.OracleModel(img).generate_greedy(g["prompt"], len(g["tokens"])))
    else:
        cfg = mcpm.make_config(2, 1024, 16, 8, 64, 2048, 1000)
        img = mcpm.synth_gguf(cfg, seed=405, mix=0)
        prompt = [int(t) for t in np.random.default_rng(18).integers(0, 1000, 2200)]
        announce("fused QKV+attention: 8 kv heads, 2200-token prompt per token")
        e = mcpm.Engine(ctx, image=img)
        try:
            e.set_prefill(False)
            e.init_kv_cache(2220)
            got = list(e.generate_greedy(prompt, 8))
        finally:
            e.free()
        om = O.OracleModel(img)
        want = list(om.generate_greedy(prompt, 8))
        om.close()
        assert got == want


# 32 query heads of 64 over 8 kv heads (the 2.4B shape's head geometry): the
# O projection's 64 work groups (8 per XCD) take 4 heads each; and 16 over 4
# with 8 work groups per XCD taking 2 heads each
IN_O_SHAPES = {"kv8": (2, 1024, 32, 8, 64, 2816, 1000), "kv4": (2, 1024, 16, 4, 64, 2048, 1000)}


@pytest.mark.parametrize("shape", sorted(IN_O_SHAPES))
def test_attention_in_o_projection_matches_oracle(ctx, monkeypatch, shape):
    """Contexts of one chunk (at most 64 positions) form the attention in the
    O projection: each XCD's work groups split the query heads and share the
    outputs through tagged records in the XCD's L2, with no attention launch
    (counted: no attention launch below 64 positions, one per layer past it).
    Logits bit-identical to the oracle at positions 0..79 (across the switch
    at 64), and greedy and sampled tokens identical to the engine with the
    attention as its own launch (MCPM_ATTN_IN_O=0)."""
    cfg = mcpm.make_config(*IN_O_SHAPES[shape])
    img = mcpm.synth_gguf(cfg, seed=77, mix=0)
    rng = np.random.default_rng(5)
    toks = [int(t) for t in rng.integers(0, 1000, 80)]
    om = O.OracleModel(img)
    om.init_kv(128)
    want = np.empty(1000, np.float32)
    eng = mcpm.Engine(ctx, image=img)
    try:
        eng.init_kv_cache(128)
        for pos, t in enumerate(toks):
            announce(f"attention in the O projection ({shape}): forward pos={pos}")
            got, _ = eng.forward(t, pos)
            om.forward(t, pos, want)
            assert_bits(got, want)
        eng.set_prefill(False)
        for n_prompt in (20, 70):
            # positions 0..n_prompt-1 (one generated token): an attention
            # launch per layer only at positions 64 and past
            eng.set_kernel_timing(mcpm.KC_ATTN)
            eng.generate_greedy(np.array(toks[:n_prompt], np.int32), 1)
            _, n = eng.kernel_time()
            eng.set_kernel_timing(-1)
            assert n == max(0, n_prompt - 64) * cfg.n_layers, (n_prompt, n)
        prompt = np.array(toks[:24], np.int32)
        got = (eng.generate_greedy(prompt, 60), eng.generate_sampled(prompt, 60, 0.9, 0.95, 7))
    finally:
        eng.free()
    om.close()
    monkeypatch.setenv("MCPM_ATTN_IN_O", "0")
    ref = mcpm.Engine(ctx, image=img)
    try:
        ref.init_kv_cache(128)
        announce(f"attention as its own launch ({shape})")
        want_toks = (ref.generate_greedy(prompt, 60), ref.generate_sampled(prompt, 60, 0.9, 0.95, 7))
    finally:
        ref.free()
    np.testing.assert_array_equal(got[0], want_toks[0])
    np.testing.assert_array_equal(got[1], want_toks[1])


def test_attention_in_o_give_up_then_recovers(ctx):
    """The O projection's wait for its XCD's attention records with a spin
    limit of 1 poll: the call returns MCPM_ERR_HIP; with the default limit
    restored the next calls give the oracle's logits bit for bit (the token
    epoch moved on, so no record of the abandoned calls matches a later
    tag)."""
    cfg = mcpm.make_config(*IN_O_SHAPES["kv8"])
    img = mcpm.synth_gguf(cfg, seed=78, mix=0)
    e = mcpm.Engine(ctx, image=img)
    try:
        e.init_kv_cache(64)
        prompt = np.arange(5, 21, dtype=np.int32)
        e.set_spin_limit(1)
        codes = []
        for i in range(6):
            announce(f"attention in the O projection: spin limit 1, call {i}")
            try:
                e.generate_greedy(prompt, 4)
            except mcpm.McpmError as err:
                codes.append(err.code)
                break
        assert codes == [mcpm.ERR_HIP], "no wait gave up at a spin limit of 1"
        e.set_spin_limit(0)
        announce("attention in the O projection: default spin limit after the give-up")
        om = O.OracleModel(img)
        om.init_kv(64)
        want = np.empty(1000, np.float32)
        for pos, t in enumerate(prompt):
            got, _ = e.forward(int(t), pos)
            om.forward(int(t), pos, want)
            assert_bits(got, want)
        om.close()
    finally:
        e.free()
