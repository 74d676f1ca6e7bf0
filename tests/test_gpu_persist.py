"""The persistent decode launch (all layers of a token in one launch, one work
group per CU, hand-offs through tagged records) against the CPU oracle and
against the five-launch-per-layer path, bit for bit."""
import numpy as np
import pytest

import mcpm
import oracle as O
from conftest import announce, assert_bits

pytestmark = pytest.mark.gpu

# 8 kv heads of 64 and head groups of 4 query heads: the shape the persistent
# launch takes (kv head h on XCD h)
KV8 = dict(n_layers=3, dim=1024, n_heads=32, n_kv_heads=8, head_dim=64, ffn=2816, vocab=4096)


@pytest.fixture(scope="module")
def kv8_image():
    return mcpm.synth_gguf(mcpm.make_config(**KV8), seed=11, mix=0)


@pytest.fixture(scope="module")
def engines(ctx, kv8_image):
    a = mcpm.Engine(ctx, image=kv8_image)
    b = mcpm.Engine(ctx, image=kv8_image)
    a.set_persistent(True)
    b.set_persistent(False)
    yield a, b
    a.free()
    b.free()


def test_default_mode_and_taken_when_asked(ctx, kv8_image, engines):
    """The default mode takes the persistent launch only for a shape it has
    a compiled instance of: not this one, which mode 1 takes."""
    e = mcpm.Engine(ctx, image=kv8_image)
    e.init_kv_cache(64)
    assert not e.uses_persistent()
    e.set_persistent(True)
    assert e.uses_persistent() and not e.persistent_fixed_shape()
    e.set_persistent(mcpm.PERSIST_AUTO)
    assert not e.uses_persistent()
    with pytest.raises(mcpm.McpmError):
        e.set_persistent(3)
    e.free()
    a, b = engines
    a.init_kv_cache(256)
    b.init_kv_cache(256)
    assert a.uses_persistent(), "the 8-kv-head model fits the persistent launch on a 256-CU device"
    assert not b.uses_persistent()
    # work group b on the XCD of b % 8 (the device dispatches work groups
    # round-robin over its 8 XCDs): the XCD-local records are taken
    assert a.persistent_xcd_local()


def test_logits_bit_exact_vs_oracle(engines, kv8_image):
    a, _ = engines
    a.init_kv_cache(256)
    assert a.uses_persistent()
    om = O.OracleModel(kv8_image)
    om.init_kv(256)
    rng = np.random.default_rng(5)
    toks = rng.integers(0, KV8["vocab"], 80)
    want = np.empty(KV8["vocab"], np.float32)
    for pos, t in enumerate(toks):
        announce(f"persistent forward pos={pos}")
        got, am = a.forward(int(t), pos)
        om.forward(int(t), pos, want)
        assert_bits(got, want)
        assert am == int(np.argmax(want))


@pytest.mark.parametrize("graph", [True, False])
def test_generation_matches_five_launch_path(engines, graph):
    a, b = engines
    prompt = np.arange(3, 19, dtype=np.int32)
    outs = []
    for e in (a, b):
        e.init_kv_cache(512)
        e.set_graph(graph)
        announce(f"greedy graph={graph} persistent={e.uses_persistent()}")
        outs.append((e.generate_greedy(prompt, 200), e.generate_sampled(prompt, 200, 0.9, 0.95, 21)))
        e.set_graph(True)
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])
    assert len(set(outs[0][1].tolist())) > 8, "a near-constant token sequence pins little"


def test_agent_scope_hand_offs_match(ctx, kv8_image, engines, monkeypatch):
    """MCPM_PD_XCD_LOCAL=0: every record at agent scope; the same tokens as
    the five-launch path."""
    _, b = engines
    monkeypatch.setenv("MCPM_PD_XCD_LOCAL", "0")
    e = mcpm.Engine(ctx, image=kv8_image)
    try:
        e.set_persistent(True)
        e.init_kv_cache(512)
        assert e.uses_persistent() and not e.persistent_xcd_local()
        prompt = np.arange(5, 21, dtype=np.int32)
        b.init_kv_cache(512)
        announce("greedy and sampled, agent-scope hand-offs")
        got = (e.generate_greedy(prompt, 150), e.generate_sampled(prompt, 150, 0.9, 0.95, 33))
        want = (b.generate_greedy(prompt, 150), b.generate_sampled(prompt, 150, 0.9, 0.95, 33))
    finally:
        e.free()
    np.testing.assert_array_equal(got[0], want[0])
    np.testing.assert_array_equal(got[1], want[1])


@pytest.mark.parametrize("ffn", [2780, 2600])
def test_first_chunk_owners_light_ffn_share(ctx, ffn):
    """FFN sizes whose spare pairs leave the eight first-chunk owners fewer
    gate/up rows than the plan's 11 (7 at 2780; none at 2600) in a gate/up
    layout of their own: the generic instance against the oracle and the
    five launches."""
    generic_vs_oracle(ctx, ffn, "light FFN share")


@pytest.mark.parametrize("ffn", [5120, 5888])
def test_ffn_activation_quantize_rounds(ctx, ffn):
    """The down phase's Q8_K blocks of the FFN activations past the 16th:
    staged in the O weights' region and quantized in the same round where
    that region holds them (20 blocks at 5120 against 5 KiB of O weights per
    work group), in a second round where it does not (23 blocks at 5888):
    the generic instance against the oracle and the five launches."""
    generic_vs_oracle(ctx, ffn, "h quantize rounds")


def generic_vs_oracle(ctx, ffn, label):
    cfg = dict(KV8, n_layers=2, ffn=ffn, vocab=2048)
    img = mcpm.synth_gguf(mcpm.make_config(**cfg), seed=ffn, mix=0)
    a = mcpm.Engine(ctx, image=img)
    b = mcpm.Engine(ctx, image=img)
    try:
        a.set_persistent(True)
        b.set_persistent(False)
        a.init_kv_cache(256)
        b.init_kv_cache(256)
        assert a.uses_persistent() and not a.persistent_fixed_shape() and not b.uses_persistent()
        om = O.OracleModel(img)
        om.init_kv(256)
        rng = np.random.default_rng(ffn)
        want = np.empty(cfg["vocab"], np.float32)
        for pos, t in enumerate(rng.integers(0, cfg["vocab"], 24)):
            announce(f"{label} ffn={ffn} pos={pos}")
            got, _ = a.forward(int(t), pos)
            om.forward(int(t), pos, want)
            assert_bits(got, want)
        prompt = rng.integers(0, cfg["vocab"], 40).astype(np.int32)
        announce(f"{label} ffn={ffn}: greedy and sampled vs five launches")
        np.testing.assert_array_equal(a.generate_greedy(prompt, 48), b.generate_greedy(prompt, 48))
        np.testing.assert_array_equal(a.generate_sampled(prompt, 48, 0.9, 0.95, 7),
                                      b.generate_sampled(prompt, 48, 0.9, 0.95, 7))
    finally:
        a.free()
        b.free()


def test_long_context_two_chunks_per_work_group(engines):
    """Positions past 32 chunks of 64 per kv head (the work groups of one
    XCD): the first work groups take two chunks each, and the combiner reads
    every partial, its own two from LDS."""
    a, b = engines
    rng = np.random.default_rng(9)
    prompt = rng.integers(0, KV8["vocab"], 2300).astype(np.int32)
    outs = []
    for e in (a, b):
        e.init_kv_cache(4096)
        announce(f"long context persistent={e.uses_persistent()}")
        outs.append(e.generate_greedy_at(prompt, 0, 48))
    np.testing.assert_array_equal(outs[0], outs[1])
    # the caches now hold the same rows: one more position's logits, bit for bit
    pos = 2300 + 48
    la, _ = a.forward(int(outs[0][-1]), pos)
    lb, _ = b.forward(int(outs[1][-1]), pos)
    assert_bits(la, lb)


def test_prefill_scratch_growth_then_decode(engines):
    """Prompts of growing length on one engine: each call grows the prefill
    scratch (freed and allocated again, zeroed), then decodes through the
    persistent launch; against the five-launch path with every prompt token
    decoded one at a time (no prefill scratch at all)."""
    a, b = engines
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, KV8["vocab"], 1100).astype(np.int32)
    b.set_prefill(False)
    try:
        for T in (100, 300, 577, 1000):
            for e in (a, b):
                e.init_kv_cache(4096)
            announce(f"prefill growth T={T}")
            got = a.generate_greedy_at(prompt[:T], 0, 4)
            want = b.generate_greedy_at(prompt[:T], 0, 4)
            np.testing.assert_array_equal(got, want)
    finally:
        b.set_prefill(True)


def test_hand_off_give_up_then_recovers(engines, kv8_image):
    """Hand-off waits with a spin limit of 1 poll: a wait gives up, every
    work group leaves, the call returns MCPM_ERR_HIP and the records and
    launch count are reset; with the default limit restored the next calls
    give the oracle's logits bit for bit."""
    a, _ = engines
    a.init_kv_cache(256)
    assert a.uses_persistent()
    prompt = np.arange(40, 56, dtype=np.int32)
    a.set_spin_limit(1)
    codes = []
    try:
        for i in range(6):
            announce(f"persistent: spin limit 1, call {i}")
            try:
                a.generate_greedy(prompt, 4)
            except mcpm.McpmError as err:
                codes.append(err.code)
                break
    finally:
        a.set_spin_limit(0)
    assert codes == [mcpm.ERR_HIP], "no wait gave up at a spin limit of 1"
    announce("persistent: default spin limit after the give-up")
    om = O.OracleModel(kv8_image)
    om.init_kv(256)
    want = np.empty(KV8["vocab"], np.float32)
    for pos, t in enumerate(prompt):
        got, _ = a.forward(int(t), pos)
        om.forward(int(t), pos, want)
        assert_bits(got, want)


# The 2.4B shape's own plan (hidden 2304, FFN 5760: 23 blocks of h, the
# single-wait down prologue, staging in the down region) on 3 layers: the
# shape the launch has an instance compiled for (every plan field but the
# layer and chunk counts a constant), taken by default
SHAPE24 = dict(n_layers=3, dim=2304, n_heads=32, n_kv_heads=8, head_dim=64, ffn=5760, vocab=4096)


@pytest.fixture(scope="module")
def shape24_image():
    return mcpm.synth_gguf(mcpm.make_config(**SHAPE24), seed=23, mix=0)


def test_2p4b_shape_vs_oracle_and_five_launch_path(ctx, shape24_image):
    img = shape24_image
    a = mcpm.Engine(ctx, image=img)
    b = mcpm.Engine(ctx, image=img)
    try:
        b.set_persistent(False)
        a.init_kv_cache(512)
        b.init_kv_cache(512)
        assert a.uses_persistent() and not b.uses_persistent()
        assert a.persistent_fixed_shape() and a.persistent_xcd_local()
        om = O.OracleModel(img)
        om.init_kv(512)
        rng = np.random.default_rng(8)
        toks = rng.integers(0, SHAPE24["vocab"], 40)
        want = np.empty(SHAPE24["vocab"], np.float32)
        for pos, t in enumerate(toks):
            announce(f"2.4B-shaped persistent forward pos={pos}")
            got, _ = a.forward(int(t), pos)
            om.forward(int(t), pos, want)
            assert_bits(got, want)
        # past 192 positions (several chunks per head), sampled, against the
        # five launches
        prompt = rng.integers(0, SHAPE24["vocab"], 200).astype(np.int32)
        announce("2.4B-shaped persistent vs five launches, 200-token prompt")
        np.testing.assert_array_equal(a.generate_sampled(prompt, 96, 0.9, 0.95, 5),
                                      b.generate_sampled(prompt, 96, 0.9, 0.95, 5))
        # off frees the slab and runs the five launches; on builds it again
        a.set_persistent(False)
        assert not a.uses_persistent()
        a.set_persistent(True)
        assert a.uses_persistent() and a.persistent_fixed_shape()
        np.testing.assert_array_equal(a.generate_greedy(prompt[:50], 32), b.generate_greedy(prompt[:50], 32))
        # past 4096 positions (three chunks for some work groups) the default
        # mode runs the five launches and holds no slab
        a.init_kv_cache(4160)
        assert not a.uses_persistent()
        a.init_kv_cache(512)
        assert a.uses_persistent()
    finally:
        a.free()
        b.free()


def test_2p4b_shape_agent_scope_hand_offs(ctx, shape24_image, monkeypatch):
    """MCPM_PD_XCD_LOCAL=0 on the compiled shape: every record at agent
    scope, the same greedy and sampled tokens as the five launches."""
    monkeypatch.setenv("MCPM_PD_XCD_LOCAL", "0")
    a = mcpm.Engine(ctx, image=shape24_image)
    b = mcpm.Engine(ctx, image=shape24_image)
    try:
        b.set_persistent(False)
        a.init_kv_cache(512)
        b.init_kv_cache(512)
        assert a.uses_persistent() and a.persistent_fixed_shape() and not a.persistent_xcd_local()
        prompt = np.arange(7, 40, dtype=np.int32)
        announce("2.4B-shaped persistent, agent-scope hand-offs, vs five launches")
        np.testing.assert_array_equal(a.generate_greedy(prompt, 64), b.generate_greedy(prompt, 64))
        np.testing.assert_array_equal(a.generate_sampled(prompt, 100, 0.9, 0.95, 3),
                                      b.generate_sampled(prompt, 100, 0.9, 0.95, 3))
    finally:
        a.free()
        b.free()
