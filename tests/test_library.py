"""Host-side checks of libmcpm_hip.so that need no GPU: the C ABI exports, the
GGUF writer/reader, the block encoders and the host sampler."""
import hashlib
import os
import subprocess

import numpy as np
import pytest

import mcpm
import oracle as O
from conftest import P, ROOT
from helpers import header_functions




def test_library_exports_every_header_function(lib):
    declared = header_functions(os.path.join(ROOT, "include", "mcpm_hip.h"))
    assert len(declared) >= 50
    missing = [f for f in declared if not hasattr(lib, f)]
    assert not missing, missing
    assert set(declared) == set(mcpm.exported_symbols())


def test_library_has_gfx950_code_object():
    so = open(os.path.join(ROOT, "minicpm5.cpp_amd", "libmcpm_hip.so"), "rb").read()
    assert b"gfx950" in so


def test_gguf_roundtrip_independent_reader():
    cfg = mcpm.make_config(3, 512, 8, 2, 64, 1400, 1000, rope_base=5e6, eps=1e-5)
    img = mcpm.synth_gguf(cfg, seed=3, mix=1)
    kv, T = O.read_gguf(img)
    assert kv["general.architecture"] == "llama"
    assert kv["llama.block_count"] == 3 and kv["llama.embedding_length"] == 512
    assert kv["llama.feed_forward_length"] == 1400 and kv["llama.attention.head_count_kv"] == 2
    assert abs(kv["llama.rope.freq_base"] - 5e6) < 1 and abs(kv["llama.attention.layer_norm_rms_epsilon"] - 1e-5) < 1e-9
    assert "output.weight" not in T  # tied
    assert T["token_embd.weight"][0] == mcpm.TYPE_Q6_K and T["token_embd.weight"][1] == [512, 1000]
    assert T["blk.0.ffn_down.weight"][1] == [1536, 512]  # FFN padded to whole 256-blocks
    assert T["blk.1.attn_norm.weight"][0] == mcpm.TYPE_F32
    # mix 1 (llama.cpp use_more_bits: l < n/8, l >= 7n/8 or (l - n/8) % 3 == 2):
    # with 3 layers only layer 2 takes Q6_K v/down
    assert [T[f"blk.{l}.attn_v.weight"][0] for l in range(3)] == [mcpm.TYPE_Q4_K, mcpm.TYPE_Q4_K, mcpm.TYPE_Q6_K]
    assert len(T) == 2 + 9 * 3


def test_gguf_mix_literal_vs_llama():
    cfg = mcpm.make_config(16, 256, 4, 2, 64, 512, 300)
    kv0, T0 = O.read_gguf(mcpm.synth_gguf(cfg, seed=1, mix=0))
    kv1, T1 = O.read_gguf(mcpm.synth_gguf(cfg, seed=1, mix=1))
    lit = [T0[f"blk.{l}.ffn_down.weight"][0] for l in range(16)]
    ll = [T1[f"blk.{l}.ffn_down.weight"][0] for l in range(16)]
    assert all(t == mcpm.TYPE_Q6_K for t in lit)
    more = [l < 2 or l >= 14 or (l - 2) % 3 == 2 for l in range(16)]
    assert ll == [mcpm.TYPE_Q6_K if m else mcpm.TYPE_Q4_K for m in more]


def test_generator_is_deterministic_and_normal():
    a = mcpm.synth_normal(42, 7, 1 << 20, 0.0, 0.02)
    b = mcpm.synth_normal(42, 7, 1 << 20, 0.0, 0.02)
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 1e-4 and abs(a.std() - 0.02) < 1e-4
    assert not np.array_equal(a, mcpm.synth_normal(42, 8, 1 << 20, 0.0, 0.02))
    # any sub-range regenerates identically (counter-based)
    img1 = mcpm.synth_gguf(mcpm.make_config(1, 256, 4, 2, 64, 256, 64), seed=9)
    img2 = mcpm.synth_gguf(mcpm.make_config(1, 256, 4, 2, 64, 256, 64), seed=9)
    assert hashlib.sha256(img1.tobytes()).digest() == hashlib.sha256(img2.tobytes()).digest()


@pytest.mark.parametrize("gtype,block", [(mcpm.TYPE_Q4_K, 256), (mcpm.TYPE_Q6_K, 256), (mcpm.TYPE_Q8_0, 32)])
def test_encoder_reconstruction_bounds(orc, gtype, block):
    rng = np.random.default_rng(gtype)
    x = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    x[3] = 0.0
    x[5, :256] = np.linspace(-1, 1, 256)
    enc = mcpm.quantize_rows(gtype, x)
    deq = np.zeros_like(x)
    rb = enc.reshape(64, -1)
    for r in range(64):
        orc.or_dequant_row(gtype, P(np.ascontiguousarray(rb[r])), 1024, P(deq[r]))
    assert (deq[3] == 0).all()
    err = np.abs(deq - x).reshape(64, -1, block)
    rng_b = np.abs(x).reshape(64, -1, block).max(-1)
    levels = {mcpm.TYPE_Q4_K: 15, mcpm.TYPE_Q6_K: 31, mcpm.TYPE_Q8_0: 127}[gtype]
    # a step of the block's range over the code levels, plus the 6/8-bit scale rounding
    assert (err.max(-1) <= 2.2 * rng_b / levels + 1e-7).all()


def test_host_sampler_matches_oracle(orc):
    rng = np.random.default_rng(5)
    for i in range(40):
        lg = (rng.standard_normal(5000) * 4).astype(np.float32)
        T, top_p = [(0.8, 0.95), (1.0, 1.0), (0.3, 0.5), (2.0, 0.99)][i % 4]
        r = float(rng.random())
        assert mcpm.sample_logits(lg, T, top_p, r) == orc.or_sample(P(lg), lg.size, T, top_p, r)


def test_c_abi_rejects_bad_arguments(lib):
    # no device needed: argument checks fail before any HIP call
    assert lib.mcpm_quantize_rows(99, None, 1, 256, None) == -2
    cfg = mcpm.make_config(1, 100, 4, 2, 64, 256, 64)  # dim not a multiple of 256
    img = mcpm.C.c_void_p()
    n = mcpm.C.c_size_t()
    assert lib.mcpm_synth_gguf(mcpm.C.byref(cfg), 1, 0, None, mcpm.C.byref(img), mcpm.C.byref(n)) == -2
    assert b"invalid config" in lib.mcpm_last_error()


REF = "/root/reference"


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src")), reason="the reference's sources are not here")
def test_reference_sources_link_against_the_mirror(tmp_path):
    """The two drop-in levels build from the reference's sources, unmodified
    and compiled against their own include/ (oracle/Makefile `dropin`): its
    CLI with src/model.cpp and src/ops/*.cpp replaced by libmcpm_model.so,
    and with only src/ops/*.cpp replaced by libmcpm_ops.so; the order driver
    against the reference's include/model.h both ways.  The operator-level
    CLI takes matmul, execute_attention, ... from libmcpm_ops.so (undefined in
    the executable), the engine-level CLI takes MiniCPM5Engine's calls from
    libmcpm_model.so; --help runs without a GPU."""
    out = str(tmp_path)
    r = subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "dropin", f"DROPIN_OUT={out}"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    names = ["minicpm5-cli-engine", "minicpm5-cli-ops", "dropin_driver_engine", "dropin_driver_ops"]
    for n in names:
        assert os.access(os.path.join(out, n), os.X_OK), n

    def undefined(prog):
        nm = subprocess.run(["nm", "-D", "-C", "--undefined-only", os.path.join(out, prog)],
                            capture_output=True, text=True, check=True).stdout
        return nm

    ops_undef = undefined("minicpm5-cli-ops")
    for fn in ("matmul(", "matmul_qkv_q8k(", "matmul_gate_up_q8k(", "execute_attention(", "get_embedding(",
               "rmsnorm_and_quantize_q8k(", "swiglu_and_quantize_q8k(", "apply_rope("):
        assert fn in ops_undef, fn
    assert "MiniCPM5Engine::forward" not in ops_undef  # the reference's own src/model.cpp
    eng_undef = undefined("minicpm5-cli-engine")
    for fn in ("MiniCPM5Engine::init_kv_cache(int)", "MiniCPM5Engine::load_model(", "MiniCPM5Engine::forward(int, int, int)"):
        assert fn in eng_undef, fn
    r = subprocess.run([os.path.join(out, "minicpm5-cli-engine"), "--help"], capture_output=True, text=True)
    assert r.returncode == 0 and "Usage" in r.stdout


def test_persistent_decode_plan_checks():
    """The persistent decode launch's host-side plan (tests/cpp/persist_check):
    LDS budget, slab regions and their sources, the rows each work group's
    tasks read, and the shapes it refuses."""
    prog = os.path.join(ROOT, "tests", "cpp", "persist_check")
    assert os.access(prog, os.X_OK), f"{prog} not built (make -C tests/cpp)"
    r = subprocess.run([prog], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "all persistent-kernel plan checks passed" in r.stdout
