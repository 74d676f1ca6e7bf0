"""The C++ mirror of the reference's host interfaces (minicpm5.cpp_amd/host/):
ops.h functions and MiniCPM5Engine, driven from C++ programs and compared with
the CPU oracle.  Bar: bit-identical to the oracle, as the C ABI they wrap."""
import os
import subprocess

import numpy as np
import pytest

import mcpm
from conftest import P, announce

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "tests", "cpp", "ops_wrapper_check")
DECODE = os.path.join(ROOT, "minicpm5.cpp_amd", "mcpm_decode")
SEED = 99  # tests/cpp/ops_wrapper_check.cpp
COLS = 512


def test_programs_built_and_usage():
    """Both programs exist and reject bad usage before touching a GPU."""
    for path in (CHECK, DECODE):
        assert os.access(path, os.X_OK), f"{path} not built (make -C minicpm5.cpp_amd host; make -C tests/cpp)"
    assert subprocess.run([DECODE, "--help"], capture_output=True).returncode == 0
    assert subprocess.run([DECODE, "--synth", "1", "--prompt-ids", "1,x"], capture_output=True).returncode == 2
    assert subprocess.run([CHECK], capture_output=True).returncode == 2


def _records(path):
    out = {}
    with open(path, "rb") as f:
        data = f.read()
    i = 0
    while i < len(data):
        n = int.from_bytes(data[i:i + 4], "little")
        name = data[i + 4:i + 4 + n].decode()
        i += 4 + n
        nb = int.from_bytes(data[i:i + 8], "little")
        out[name] = np.frombuffer(data[i + 8:i + 8 + nb], np.uint8).copy()
        i += 8 + nb
    return out


def _normal(tid, n, mean=0.0, sd=1.0):
    return mcpm.synth_normal(SEED, tid, n, mean, sd)


def _weight(tid, gtype, rows, cols=COLS):
    w = _normal(tid, rows * cols, 0.0, 0.02).reshape(rows, cols)
    return w if gtype == mcpm.TYPE_F32 else mcpm.quantize_rows(gtype, w)


def _f32(rec):
    return rec.view(np.float32)


@pytest.mark.gpu
def test_ops_mirror_matches_oracle(orc, tmp_path):
    out = str(tmp_path / "ops.bin")
    announce("ops_wrapper_check")
    r = subprocess.run([CHECK, out], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    got = _records(out)

    x, gamma = _normal(5, COLS), _normal(6, COLS, 1.0, 0.1)
    g, u = _normal(7, COLS), _normal(8, COLS)
    want = np.empty(300, np.float32)
    for name, gtype, tid in [("matmul_q4k", mcpm.TYPE_Q4_K, 1), ("matmul_q6k", mcpm.TYPE_Q6_K, 2),
                             ("matmul_q8_0", mcpm.TYPE_Q8_0, 3)]:
        orc.or_matmul(gtype, P(_weight(tid, gtype, 300)), P(x), P(want), 300, COLS)
        np.testing.assert_array_equal(_f32(got[name]), want, err_msg=name)
    wf = np.ascontiguousarray(_weight(4, mcpm.TYPE_F32, 40))
    want40 = np.empty(40, np.float32)
    orc.or_matmul(mcpm.TYPE_F32, P(wf), P(x), P(want40), 40, COLS)
    np.testing.assert_array_equal(_f32(got["matmul_f32"]), want40)
    np.testing.assert_array_equal(_f32(got["matmul_unsupported"]), np.full(300, 0.001, np.float32))

    xq = np.zeros(COLS // 256 * 292, np.uint8)
    orc.or_quantize_row_q8_K(P(x), COLS, P(xq), 0)
    np.testing.assert_array_equal(got["quantize_row_q8_K"], xq)
    for name, gtype, tid in [("matmul_q8k_q4k", mcpm.TYPE_Q4_K, 1), ("matmul_q8k_q6k", mcpm.TYPE_Q6_K, 2)]:
        orc.or_matmul_q8k(gtype, P(_weight(tid, gtype, 300)), P(xq), P(want), 300, COLS)
        np.testing.assert_array_equal(_f32(got[name]), want, err_msg=name)

    q, k, v = np.empty(256, np.float32), np.empty(64, np.float32), np.empty(64, np.float32)
    orc.or_gemv_qkv_q8_K(P(_weight(9, mcpm.TYPE_Q4_K, 256)), P(_weight(10, mcpm.TYPE_Q4_K, 64)),
                         P(_weight(11, mcpm.TYPE_Q6_K, 64)), mcpm.TYPE_Q6_K, P(xq), P(q), P(k), P(v), 256, 64, COLS)
    for name, arr in [("qkv_q", q), ("qkv_k", k), ("qkv_v", v)]:
        np.testing.assert_array_equal(_f32(got[name]), arr, err_msg=name)
    gate, up = np.empty(300, np.float32), np.empty(300, np.float32)
    orc.or_gemv_gate_up_q4_K_q8_K(P(_weight(12, mcpm.TYPE_Q4_K, 300)), P(_weight(13, mcpm.TYPE_Q4_K, 300)), P(xq),
                                  P(gate), P(up), 300, COLS)
    np.testing.assert_array_equal(_f32(got["gate"]), gate)
    np.testing.assert_array_equal(_f32(got["up"]), up)

    rn = np.empty(COLS, np.float32)
    orc.or_rmsnorm(P(rn), P(x), P(gamma), COLS, np.float32(1e-6))
    np.testing.assert_array_equal(_f32(got["rmsnorm"]), rn)
    nq = np.zeros_like(xq)
    orc.or_rmsnorm_and_quantize_q8k(P(nq), P(x), P(gamma), COLS, np.float32(1e-6))
    np.testing.assert_array_equal(got["rmsnorm_and_quantize_q8k"], nq)
    sq = np.zeros_like(xq)
    orc.or_swiglu_and_quantize_q8k(P(sq), P(g), P(u), COLS)
    np.testing.assert_array_equal(got["swiglu_and_quantize_q8k"], sq)

    rv = _normal(14, 4 * 64)
    orc.or_apply_rope(P(rv[128:]), 17, 1, 64, np.float32(10000.0))  # head 2 only
    np.testing.assert_array_equal(_f32(got["apply_rope"]), rv)

    pos, max_seq, nh, nkv, hd = 70, 96, 8, 2, 64
    kc_all, vc_all = _normal(18, max_seq * nkv * hd), _normal(19, max_seq * nkv * hd)
    aq, kc, vc = _normal(15, nh * hd), _normal(16, nkv * hd), _normal(17, nkv * hd)
    att = np.empty(nh * hd, np.float32)
    assert orc.or_attention(P(att), P(aq), P(kc), P(vc), P(kc_all), P(vc_all), pos, max_seq, nh, nkv, hd) == 0
    np.testing.assert_array_equal(_f32(got["attention"]), att)
    np.testing.assert_array_equal(_f32(got["attention_kcache_row"]), kc)

    emb = np.empty(COLS, np.float32)
    orc.or_get_embedding(P(emb), mcpm.TYPE_Q6_K, P(_weight(20, mcpm.TYPE_Q6_K, 50)), COLS, 5)
    np.testing.assert_array_equal(_f32(got["embedding"]), emb)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["forward", "prefill", "device-loop"])
def test_engine_mirror_greedy_matches_oracle(mode):
    import oracle as O
    cfg = mcpm.make_config(2, 2304, 32, 8, 64, 5760, 4096)
    seed, prompt, n_gen = 7, [5, 1000, 77, 4095, 12], 12
    announce(f"mcpm_decode {mode}")
    cmd = [DECODE, "--synth", str(seed), "--layers", "2", "--vocab", "4096",
           "--prompt-ids", ",".join(map(str, prompt)), "--tokens", str(n_gen)]
    if mode != "forward":
        cmd.append("--" + mode)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    line = next(l for l in r.stdout.splitlines() if l.startswith("tokens:"))
    got = [int(t) for t in line.split()[1:]]
    om = O.OracleModel(mcpm.synth_gguf(cfg, seed=seed, mix=0))
    want = om.generate_greedy(prompt, n_gen)
    om.close()
    assert got == list(want)


@pytest.mark.gpu
def test_engine_mirror_sampled_matches_oracle():
    """mcpm_decode --sample: MiniCPM5Engine::generate_sampled against the
    oracle model with the device sampler's arithmetic and the same draws."""
    import oracle as O
    orc = O.oracle()
    cfg = mcpm.make_config(2, 2304, 32, 8, 64, 5760, 4096)
    seed, prompt, n_gen, T, top_p, sseed = 7, [5, 1000, 77, 4095, 12], 10, 0.9, 0.9, 31
    announce("mcpm_decode --sample")
    cmd = [DECODE, "--synth", str(seed), "--layers", "2", "--vocab", "4096",
           "--prompt-ids", ",".join(map(str, prompt)), "--tokens", str(n_gen), "--sample", f"{T},{top_p},{sseed}"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    line = next(l for l in r.stdout.splitlines() if l.startswith("tokens:"))
    got = [int(t) for t in line.split()[1:]]
    om = O.OracleModel(mcpm.synth_gguf(cfg, seed=seed, mix=0))
    om.init_kv(len(prompt) + n_gen + 2)
    lg = np.empty(4096, np.float32)
    for p, t in enumerate(prompt):
        om.forward(int(t), p, lg)
    gen = np.zeros(625, np.uint32)
    orc.or_mt_seed(P(gen), sseed)
    want = []
    for i in range(n_gen):
        if want:
            om.forward(want[-1], len(prompt) + i - 1, lg)
        want.append(orc.or_sample_blocked(P(lg), 4096, T, top_p, orc.or_mt_uniform01(P(gen))))
    om.close()
    assert got == want


@pytest.mark.gpu
def test_session_turns_reuse_cache_and_match_oracle():
    """mcpm_decode --turns: KVSession keeps the KV rows of the conversation
    between turns and runs only each turn's new tokens; every turn's tokens
    equal those of the same conversation run from position 0 (--no-reuse,
    the reference's way) and the oracle's greedy continuation."""
    import oracle as O
    cfg = mcpm.make_config(2, 2304, 32, 8, 64, 5760, 4096)
    seed, prompt, n_gen = 7, [5, 1000, 77, 4095, 12], 6
    announce("mcpm_decode --turns")
    base = [DECODE, "--synth", str(seed), "--layers", "2", "--vocab", "4096",
            "--prompt-ids", ",".join(map(str, prompt)), "--tokens", str(n_gen), "--turns", "3,40"]
    runs = {}
    for reuse in (True, False):
        r = subprocess.run(base + ([] if reuse else ["--no-reuse"]), capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stderr
        runs[reuse] = [l for l in r.stdout.splitlines() if l.startswith("turn ")]
    assert len(runs[True]) == 3

    def parse(line):
        head, toks = line.split("tokens:")
        f = dict(kv.strip().split(" ", 1) for kv in head.split(":", 1)[1].split(",")[:3])
        return int(f["conversation"]), int(f["reused"]), int(f["processed"]), [int(t) for t in toks.split()]

    turns = [parse(l) for l in runs[True]]
    fresh = [parse(l) for l in runs[False]]
    prev = None  # (conversation length, response) of the previous turn
    for (n, reused, processed, toks), (n2, reused2, _, toks2) in zip(turns, fresh):
        assert toks == toks2 and n == n2 and reused2 == 0
        # the previous turn's conversation and response but its last token
        # (never fed back) are cached
        assert reused == (0 if prev is None else prev[0] + len(prev[1]) - 1)
        assert processed == n - reused
        prev = (n, toks)
    # turn 0 against the oracle; the later turns' new ids come from the
    # program's generator, and the run from position 0 checks them
    om = O.OracleModel(mcpm.synth_gguf(cfg, seed=seed, mix=0))
    assert list(om.generate_greedy(prompt, n_gen)) == turns[0][3]
    om.close()


# ------------------------------------------------------------------------
# The reference's own sources linked against this build (oracle/Makefile
# `dropin`, built where the reference's sources are; the programs travel as
# built files).

REF_BIN = os.path.join(ROOT, "oracle", "_ref")
DRIVER_NATIVE = os.path.join(ROOT, "tests", "cpp", "dropin_driver")


def _ref_program(name):
    path = os.path.join(REF_BIN, name)
    if not os.access(path, os.X_OK):
        pytest.skip(f"{name} not built (make -C oracle dropin needs the reference's sources)")
    return path


def _tokens(stdout):
    line = next(l for l in stdout.splitlines() if l.startswith("tokens:"))
    return [int(t) for t in line.split()[1:]]


@pytest.mark.gpu
def test_reference_cli_runs_on_the_engine(tmp_path):
    """The reference's own CLI -- src/main.cpp, chat_session.cpp, sampler.cpp,
    tokenizer.cpp, chat_template.cpp and tool.cpp compiled unmodified against
    its own include/ -- linked against libmcpm_model.so in place of
    src/model.cpp and src/ops/*.cpp: it allocates the KV cache before loading
    (main.cpp:107-111), reads the vocabulary from a reference-layout GGUF,
    tokenizes the chat template, runs forward() per prompt token and samples
    --n tokens on the GPU engine."""
    cli = _ref_program("minicpm5-cli-engine")
    cfg = mcpm.make_config(2, 512, 8, 2, 64, 1400, 4000)
    path = str(tmp_path / "m.gguf")
    mcpm.synth_gguf(cfg, seed=5, mix=2, path=path)
    announce("reference CLI on libmcpm_model.so")
    # the CLI seeds its sampler from std::random_device, and a sampled token of
    # the synthetic vocabulary can be a lone byte: its output is read as bytes
    r = subprocess.run([cli, "-m", path, "--text", "Hello, world", "-n", "8", "-c", "512", "-v"],
                       capture_output=True, text=True, encoding="utf-8", errors="replace", timeout=300,
                       cwd=str(tmp_path))
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "tokens) direto do arquivo GGUF" in r.stdout  # the reference tokenizer read the vocabulary
    prompt_line = next(l for l in r.stdout.splitlines() if l.startswith("Prompt:"))
    assert int(prompt_line.split()[1]) > 10  # the rendered chat template, tokenized


@pytest.fixture(scope="module")
def refgeom_file(tmp_path_factory):
    """A synthetic model at the reference's own geometry and file layout
    (42 layers, hidden 2048, 16/2 heads of 128, FFN 6144, vocab 130560, Q4_K
    token_embd, Q6_K output, tensor data at the reference file's offsets)."""
    cfg = mcpm.make_config(42, 2048, 16, 2, 128, 6144, 130560, rope_base=5e6)
    path = str(tmp_path_factory.mktemp("refgeom") / "minicpm5-2b-synthetic.gguf")
    announce("synthesize the reference-geometry model")
    mcpm.synth_gguf(cfg, seed=20260115, mix=2, path=path)
    return cfg, path


@pytest.mark.gpu
def test_dropin_drivers_match_native_engine(refgeom_file, tmp_path):
    """MiniCPM5Engine driven in main.cpp's order (init_kv_cache, load_model,
    forward per token) three ways on the reference-geometry file: this
    build's header + libmcpm_model.so; the reference's include/model.h +
    libmcpm_model.so (engine drop-in); the reference's include/model.h and
    its own src/model.cpp -- loading by the tensor offsets compiled into it --
    + libmcpm_ops.so (operator drop-in).  Each gives the native engine's
    greedy tokens and bit-identical first-step logits."""
    import oracle as O
    cfg, path = refgeom_file
    prompt, n_gen, ctx = [1, 3, 500, 70000, 130559, 42, 9, 1234], 8, 64
    announce("native engine on the reference-geometry file")
    c = mcpm.Context(0)
    e = mcpm.Engine(c, gguf_path=path)
    try:
        assert e.cfg.tied_embeddings == 0 and e.cfg.n_layers == 42
        e.init_kv_cache(ctx)
        want = [int(t) for t in e.generate_greedy(prompt, n_gen)]
        e.init_kv_cache(ctx)
        for p, t in enumerate(prompt):
            want_logits, _ = e.forward(t, p)
    finally:
        e.free()
        c.close()
    programs = [DRIVER_NATIVE, os.path.join(REF_BIN, "dropin_driver_engine"), os.path.join(REF_BIN, "dropin_driver_ops")]
    ran = 0
    for prog in programs:
        if not os.access(prog, os.X_OK):
            assert prog != DRIVER_NATIVE, "tests/cpp/dropin_driver not built"
            continue
        announce(f"{os.path.basename(prog)} on the reference-geometry file")
        out = str(tmp_path / (os.path.basename(prog) + ".f32"))
        r = subprocess.run([prog, path, str(ctx), str(n_gen), ",".join(map(str, prompt)), out],
                           capture_output=True, text=True, timeout=600)
        assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
        assert _tokens(r.stdout) == want, os.path.basename(prog)
        np.testing.assert_array_equal(np.fromfile(out, np.float32).view(np.uint32), want_logits.view(np.uint32))
        ran += 1
    if ran < len(programs):
        pytest.skip("the reference-header drivers are not built here (no reference sources)")
    # and the native engine against the oracle on the first steps
    announce("oracle on the reference-geometry file")
    om = O.OracleModel(np.fromfile(path, np.uint8))
    assert list(om.generate_greedy(prompt, 3)) == want[:3]
    om.close()


@pytest.mark.gpu
def test_reference_cli_runs_on_the_operators(refgeom_file, tmp_path):
    """The reference's CLI with its own src/model.cpp (tensor offsets
    compiled in for its file) and libmcpm_ops.so in place of src/ops/*.cpp:
    it loads the reference-geometry file by those offsets and runs its
    forward() through this build's operators on the GPU."""
    cli = _ref_program("minicpm5-cli-ops")
    cfg, path = refgeom_file
    announce("reference CLI on libmcpm_ops.so")
    r = subprocess.run([cli, "-m", path, "--text", "Hi", "-n", "4", "-c", "256", "-v"],
                       capture_output=True, text=True, encoding="utf-8", errors="replace", timeout=600,
                       cwd=str(tmp_path))
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    prompt_line = next(l for l in r.stdout.splitlines() if l.startswith("Prompt:"))
    assert int(prompt_line.split()[1]) > 10
