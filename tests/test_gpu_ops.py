"""Per-op parity of the HIP kernels through the C ABI.

Bar: bit-identical to the CPU oracle (which reproduces the reference's AVX2
GEMV arithmetic exactly, see tests/test_oracle.py), and within 1e-3 of the
reference's own outputs stored in tests/golden/.
"""
import numpy as np
import pytest

import mcpm
from conftest import P, announce, assert_bits, assert_close, golden
from helpers import q8k_from, rand_act, rand_q4k, rand_q6k, rand_q8_0

pytestmark = pytest.mark.gpu



# Device buffers made by up() stay alive until the test ends (after a sync),
# so a pointer taken inline in a call never outlives its allocation.
_KEEP = []


@pytest.fixture(autouse=True)
def _keep_uploads(ctx):
    yield
    ctx.sync()
    _KEEP.clear()


def up(ctx, a):
    buf = ctx.upload(np.ascontiguousarray(a))
    _KEEP.append(buf)
    return buf


def test_tensor_roundtrip(ctx):
    rng = np.random.default_rng(0)
    for gtype, gen, cols in [(mcpm.TYPE_Q4_K, rand_q4k, 2304), (mcpm.TYPE_Q6_K, rand_q6k, 5888),
                             (mcpm.TYPE_Q8_0, rand_q8_0, 512)]:
        rows = 40
        blk = gen(rng, rows * cols // (32 if gtype == mcpm.TYPE_Q8_0 else 256))
        announce(f"roundtrip type={gtype} {rows}x{cols}")
        t = ctx.tensor(blk, gtype, cols, rows)
        assert_bits(t.download(), blk.view(np.uint8))


@pytest.mark.parametrize("gtype", [mcpm.TYPE_Q4_K, mcpm.TYPE_Q6_K, mcpm.TYPE_Q8_0])
def test_dequant_bit_exact(ctx, orc, gtype):
    rng = np.random.default_rng(1)
    rows, cols = 24, 1024
    per = 32 if gtype == mcpm.TYPE_Q8_0 else 256
    blk = {mcpm.TYPE_Q4_K: lambda: rand_q4k(rng, rows * cols // per, extreme=True),
           mcpm.TYPE_Q6_K: lambda: rand_q6k(rng, rows * cols // per, extreme=True),
           mcpm.TYPE_Q8_0: lambda: rand_q8_0(rng, rows * cols // per)}[gtype]()
    announce(f"dequant type={gtype}")
    t = ctx.tensor(blk, gtype, cols, rows)
    got = t.dequantize()
    want = np.zeros((rows, cols), np.float32)
    rb = blk.view(np.uint8).reshape(rows, -1)
    for r in range(rows):
        row = np.ascontiguousarray(rb[r])
        orc.or_dequant_row(gtype, P(row), cols, want[r].ctypes.data)
    assert_bits(got, want)


def test_fp16_conversion_exhaustive_on_device(ctx, orc):
    """fp16_to_fp32 (include/ops.h:14-31) on the GPU for all 65,536 inputs:
    Q8_0 blocks whose d runs through every half-precision bit pattern (zeros,
    subnormals, normals, infinities, NaNs), codes +1 and -1, dequantized by
    the device (the conversion the GEMV and embedding kernels use) against the
    oracle's conversion, which is pinned against the reference's on the same
    65,536 inputs.  Bit-exact for every non-NaN input (d*1 and d*-1 are exact);
    NaN stays NaN (the reference's portable converter keeps a signalling
    payload, the hardware conversion and F16C quiet it)."""
    n_blk = 65536
    rows = 64
    cols = n_blk // rows * 32  # 1024 blocks per row
    blk = np.zeros(n_blk, mcpm.Q8_0)
    blk["d"] = np.arange(n_blk, dtype=np.uint32).astype(np.uint16)  # block (r, b) holds d = r*1024 + b
    blk["qs"][:, 0::2] = 1
    blk["qs"][:, 1::2] = -1
    announce("fp16 exhaustive via Q8_0 dequant")
    t = ctx.tensor(blk, mcpm.TYPE_Q8_0, cols, rows)
    got = t.dequantize().reshape(n_blk, 32)
    conv = np.array([orc.or_fp16_to_fp32(h) for h in range(n_blk)], np.float32)
    nan = np.isnan(conv)
    assert nan.sum() == 2 * 1023  # both signs, every non-zero mantissa
    assert np.isnan(got[nan]).all()
    want = np.stack([conv, -conv], axis=1)[~nan]
    assert_bits(np.ascontiguousarray(got[~nan][:, 0:2]), np.ascontiguousarray(want))
    assert_bits(np.ascontiguousarray(got[~nan][:, 30:32]), np.ascontiguousarray(want))


def test_quantize_row_q8k(ctx, orc):
    rng = np.random.default_rng(2)
    x = rand_act(rng, 256 * 12, 3.0)
    x[256:512] = 0.0
    x[512:768] = np.round(rng.standard_normal(256) * 20) / 2
    x[512] = 127.0
    announce("quantize_row_q8_K")
    xd = up(ctx, x)
    yd = ctx.zeros(12 * 292)
    mcpm.check(ctx.lib.mcpm_quantize_row_q8_K(ctx.h, xd.ptr, x.size, yd.ptr))
    got = ctx.download(yd, mcpm.Q8_K, 12)
    assert_bits(got, q8k_from(orc, x, 0))


def test_quantize_golden(ctx, orc):
    g = golden("q8k_quant.npz")
    x = g["x"]
    announce("quantize golden")
    yd = ctx.zeros(16 * 292)
    mcpm.check(ctx.lib.mcpm_quantize_row_q8_K(ctx.h, up(ctx, x).ptr, x.size, yd.ptr))
    assert_bits(ctx.download(yd, mcpm.Q8_K, 16), g["even"].view(mcpm.Q8_K))


@pytest.mark.parametrize("dim", [256, 2304, 5888])
def test_rmsnorm_ops(ctx, orc, dim):
    rng = np.random.default_rng(3 + dim)
    x = rand_act(rng, dim, 2.0)
    w = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    announce(f"rmsnorm dim={dim}")
    xd, wd = up(ctx, x), up(ctx, w)
    od = ctx.zeros(dim * 4)
    mcpm.check(ctx.lib.mcpm_rmsnorm(ctx.h, od.ptr, xd.ptr, wd.ptr, dim, 1e-6))
    want = np.zeros(dim, np.float32)
    orc.or_rmsnorm(P(want), P(x), P(w), dim, 1e-6)
    assert_bits(ctx.download(od, np.float32, dim), want)
    qd = ctx.zeros(dim // 256 * 292)
    mcpm.check(ctx.lib.mcpm_rmsnorm_and_quantize_q8k(ctx.h, qd.ptr, xd.ptr, wd.ptr, dim, 1e-6))
    wq = np.zeros(dim // 256, mcpm.Q8_K)
    orc.or_rmsnorm_and_quantize_q8k(P(wq), P(x), P(w), dim, 1e-6)
    assert_bits(ctx.download(qd, mcpm.Q8_K, dim // 256), wq)


def test_swiglu_quant(ctx, orc):
    rng = np.random.default_rng(4)
    dim = 5888
    g = rand_act(rng, dim, 3.0)
    u = rand_act(rng, dim, 1.0)
    g[-128:] = 0.0
    u[-128:] = 0.0
    announce("swiglu_and_quantize")
    od = ctx.zeros(23 * 292)
    mcpm.check(ctx.lib.mcpm_swiglu_and_quantize_q8k(ctx.h, od.ptr, up(ctx, g).ptr, up(ctx, u).ptr, dim))
    want = np.zeros(23, mcpm.Q8_K)
    orc.or_swiglu_and_quantize_q8k(P(want), P(g), P(u), dim)
    assert_bits(ctx.download(od, mcpm.Q8_K, 23), want)


GEMV_SHAPES = [(8, 256), (37, 2304), (512, 2048), (2304, 5888), (130, 8192), (1000, 2304)]


@pytest.mark.parametrize("rows,cols", GEMV_SHAPES)
@pytest.mark.parametrize("gtype", [mcpm.TYPE_Q4_K, mcpm.TYPE_Q6_K])
def test_gemv_q8k_bit_exact(ctx, orc, gtype, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    nb = cols // 256
    blk = (rand_q4k if gtype == mcpm.TYPE_Q4_K else rand_q6k)(rng, rows * nb, extreme=True)
    x = rand_act(rng, cols)
    xq = q8k_from(orc, x)
    announce(f"gemv q8k type={gtype} {rows}x{cols}")
    t = ctx.tensor(blk, gtype, cols, rows)
    od = ctx.zeros(rows * 4)
    fn = ctx.lib.mcpm_gemv_q4_K_q8_K if gtype == mcpm.TYPE_Q4_K else ctx.lib.mcpm_gemv_q6_K_q8_K
    mcpm.check(fn(ctx.h, t.h, up(ctx, xq).ptr, od.ptr, rows, cols))
    want = np.zeros(rows, np.float32)
    (orc.or_gemv_q4_K_q8_K if gtype == mcpm.TYPE_Q4_K else orc.or_gemv_q6_K_q8_K)(P(blk), P(xq), P(want), rows, cols)
    assert_bits(ctx.download(od, np.float32, rows), want)
    # fp32-activation entry (quantize ties-even inside the kernel)
    od2 = ctx.zeros(rows * 4)
    fn2 = ctx.lib.mcpm_gemv_q4_K if gtype == mcpm.TYPE_Q4_K else ctx.lib.mcpm_gemv_q6_K
    mcpm.check(fn2(ctx.h, t.h, up(ctx, x).ptr, od2.ptr, rows, cols))
    assert_bits(ctx.download(od2, np.float32, rows), want)


# Work-group items forced through the shape override ("-KB,S": S rows, KB
# steps per wave): a ragged last item (37 rows), one row per group with each
# group looping over many items, two steps per wave, and 32 blocks per row.
GRP_SHAPES = [(37, 2304, "-1,11"), (2304, 5888, "-1,1"), (2304, 5888, "-2,22"), (130, 8192, "-1,8"),
              (1000, 2304, "-2,56")]


@pytest.mark.parametrize("rows,cols,shape", GRP_SHAPES)
@pytest.mark.parametrize("gtype", [mcpm.TYPE_Q4_K, mcpm.TYPE_Q6_K])
def test_gemv_group_items_bit_exact(ctx, orc, monkeypatch, gtype, rows, cols, shape):
    monkeypatch.setenv("MCPM_GEMV_SHAPE_OTHER", shape)
    rng = np.random.default_rng(rows * 11 + cols)
    nb = cols // 256
    blk = (rand_q4k if gtype == mcpm.TYPE_Q4_K else rand_q6k)(rng, rows * nb, extreme=True)
    x = rand_act(rng, cols)
    xq = q8k_from(orc, x)
    announce(f"gemv group items type={gtype} {rows}x{cols} shape={shape}")
    t = ctx.tensor(blk, gtype, cols, rows)
    want = np.zeros(rows, np.float32)
    (orc.or_gemv_q4_K_q8_K if gtype == mcpm.TYPE_Q4_K else orc.or_gemv_q6_K_q8_K)(P(blk), P(xq), P(want), rows, cols)
    od = ctx.zeros(rows * 4)
    fn = ctx.lib.mcpm_gemv_q4_K_q8_K if gtype == mcpm.TYPE_Q4_K else ctx.lib.mcpm_gemv_q6_K_q8_K
    mcpm.check(fn(ctx.h, t.h, up(ctx, xq).ptr, od.ptr, rows, cols))
    assert_bits(ctx.download(od, np.float32, rows), want)
    od2 = ctx.zeros(rows * 4)
    fn2 = ctx.lib.mcpm_gemv_q4_K if gtype == mcpm.TYPE_Q4_K else ctx.lib.mcpm_gemv_q6_K
    mcpm.check(fn2(ctx.h, t.h, up(ctx, x).ptr, od2.ptr, rows, cols))
    assert_bits(ctx.download(od2, np.float32, rows), want)


@pytest.mark.parametrize("v_type", [mcpm.TYPE_Q4_K, mcpm.TYPE_Q6_K])
def test_qkv(ctx, orc, v_type):
    rng = np.random.default_rng(5 + v_type)
    H, QR, KR = 2304, 2048, 512
    nb = H // 256
    wq, wk = rand_q4k(rng, QR * nb), rand_q4k(rng, KR * nb)
    wv = (rand_q4k if v_type == mcpm.TYPE_Q4_K else rand_q6k)(rng, KR * nb)
    xq = q8k_from(orc, rand_act(rng, H))
    announce(f"qkv v_type={v_type}")
    tq, tk, tv = ctx.tensor(wq, 12, H, QR), ctx.tensor(wk, 12, H, KR), ctx.tensor(wv, v_type, H, KR)
    qd, kd, vd = ctx.zeros(QR * 4), ctx.zeros(KR * 4), ctx.zeros(KR * 4)
    mcpm.check(ctx.lib.mcpm_gemv_qkv_q8_K(ctx.h, tq.h, tk.h, tv.h, up(ctx, xq).ptr, qd.ptr, kd.ptr, vd.ptr, QR, KR, H))
    q, k, v = np.zeros(QR, np.float32), np.zeros(KR, np.float32), np.zeros(KR, np.float32)
    orc.or_gemv_qkv_q8_K(P(wq), P(wk), P(wv), v_type, P(xq), P(q), P(k), P(v), QR, KR, H)
    assert_bits(ctx.download(qd, np.float32, QR), q)
    assert_bits(ctx.download(kd, np.float32, KR), k)
    assert_bits(ctx.download(vd, np.float32, KR), v)


@pytest.mark.parametrize("rows", [5760, 13])
def test_gate_up(ctx, orc, rows):
    rng = np.random.default_rng(6 + rows)
    H = 2304
    nb = H // 256
    wg, wu = rand_q4k(rng, rows * nb), rand_q4k(rng, rows * nb)
    xq = q8k_from(orc, rand_act(rng, H), 1)
    announce(f"gate_up rows={rows}")
    tg, tu = ctx.tensor(wg, 12, H, rows), ctx.tensor(wu, 12, H, rows)
    gd, ud = ctx.zeros(rows * 4), ctx.zeros(rows * 4)
    mcpm.check(ctx.lib.mcpm_gemv_gate_up_q4_K_q8_K(ctx.h, tg.h, tu.h, up(ctx, xq).ptr, gd.ptr, ud.ptr, rows, H))
    g, u = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
    orc.or_gemv_gate_up_q4_K_q8_K(P(wg), P(wu), P(xq), P(g), P(u), rows, H)
    assert_bits(ctx.download(gd, np.float32, rows), g)
    assert_bits(ctx.download(ud, np.float32, rows), u)


def test_matmul_dispatch(ctx, orc):
    rng = np.random.default_rng(7)
    rows, cols = 300, 1024
    x = rand_act(rng, cols)
    cases = [(mcpm.TYPE_F32, rng.standard_normal((rows, cols)).astype(np.float32).ravel()),
             (mcpm.TYPE_Q8_0, rand_q8_0(rng, rows * cols // 32)),
             (mcpm.TYPE_Q4_K, rand_q4k(rng, rows * cols // 256)),
             (mcpm.TYPE_Q6_K, rand_q6k(rng, rows * cols // 256))]
    xd = up(ctx, x)
    for gtype, blk in cases:
        announce(f"matmul type={gtype}")
        t = ctx.tensor(blk, gtype, cols, rows)
        od = ctx.zeros(rows * 4)
        mcpm.check(ctx.lib.mcpm_matmul(ctx.h, t.h, xd.ptr, od.ptr))
        want = np.zeros(rows, np.float32)
        assert orc.or_matmul(gtype, P(blk), P(x), P(want), rows, cols) == 0
        assert_bits(ctx.download(od, np.float32, rows), want)


def test_unsupported_type_rejected(ctx):
    with pytest.raises(mcpm.McpmError) as ei:
        ctx.tensor(np.zeros(256 * 2, np.uint8), 1, 256, 1)  # F16
    assert ei.value.code == -3


@pytest.mark.parametrize("pos", [0, 1, 77, 1535, 4095])
def test_rope(ctx, orc, pos):
    rng = np.random.default_rng(pos)
    v = rand_act(rng, 2048)
    announce(f"rope pos={pos}")
    vd = up(ctx, v)
    mcpm.check(ctx.lib.mcpm_apply_rope(ctx.h, vd.ptr, pos, 32, 64, 10000.0))
    want = v.copy()
    orc.or_apply_rope(P(want), pos, 32, 64, 10000.0)
    assert_bits(ctx.download(vd, np.float32, 2048), want)


# (position, KV capacity): the launch covers the splits of every chunk count
# up to the capacity's, which is not monotonic (64 chunks take 64 splits, 66
# take 33), so positions well below a capacity of 65-128 chunks are included
ATTN_CASES = [(c, c + 3) for c in (0, 1, 63, 64, 65, 511, 2048, 4096)] + [(700, 1152), (1000, 1536), (960, 2000),
                                                                         (3000, 4600), (4200, 8192)]


@pytest.mark.parametrize("case", ATTN_CASES, ids=lambda c: f"pos{c[0]}-cap{c[1]}")
@pytest.mark.parametrize("heads", [(32, 8, 64), (16, 2, 128)])
def test_attention(ctx, orc, case, heads):
    nh, nkv, hd = heads
    ctxlen, ms = case
    rng = np.random.default_rng(ctxlen * 3 + nh)
    q = rand_act(rng, nh * hd)
    k = rand_act(rng, nkv * hd)
    v = rand_act(rng, nkv * hd)
    kc = rand_act(rng, ms * nkv * hd)
    vc = rand_act(rng, ms * nkv * hd)
    announce(f"attention ctx={ctxlen} heads={heads}")
    qd, kd, vd, kcd, vcd = up(ctx, q), up(ctx, k), up(ctx, v), up(ctx, kc), up(ctx, vc)
    od = ctx.zeros(nh * hd * 4)
    mcpm.check(ctx.lib.mcpm_execute_attention(ctx.h, od.ptr, qd.ptr, kd.ptr, vd.ptr, kcd.ptr, vcd.ptr, ctxlen, ms, nh,
                                              nkv, hd))
    want = np.zeros(nh * hd, np.float32)
    kc2, vc2 = kc.copy(), vc.copy()
    assert orc.or_attention(P(want), P(q), P(k), P(v), P(kc2), P(vc2), ctxlen, ms, nh, nkv, hd) == 0
    assert_bits(ctx.download(od, np.float32, nh * hd), want)
    assert_bits(ctx.download(kcd, np.float32, kc.size), kc2)
    assert_bits(ctx.download(vcd, np.float32, vc.size), vc2)


def test_attention_context_overflow(ctx):
    od = ctx.upload(np.full(2048, 7.0, np.float32))
    z = ctx.zeros(64 * 512 * 4)
    rc = ctx.lib.mcpm_execute_attention(ctx.h, od.ptr, z.ptr, z.ptr, z.ptr, z.ptr, z.ptr, 64, 64, 32, 8, 64)
    assert rc == -4
    assert np.all(ctx.download(od, np.float32, 2048) == 7.0)  # untouched, as the reference returns early


@pytest.mark.parametrize("gtype", [mcpm.TYPE_Q4_K, mcpm.TYPE_Q6_K])
def test_embedding(ctx, orc, gtype):
    rng = np.random.default_rng(8)
    vocab, dim = 300, 2304
    blk = (rand_q4k if gtype == mcpm.TYPE_Q4_K else rand_q6k)(rng, vocab * dim // 256, extreme=True)
    t = ctx.tensor(blk, gtype, dim, vocab)
    od = ctx.zeros(dim * 4)
    for tok in (0, 1, 157, vocab - 1):
        announce(f"embedding type={gtype} token={tok}")
        mcpm.check(ctx.lib.mcpm_get_embedding(ctx.h, od.ptr, t.h, tok))
        want = np.zeros(dim, np.float32)
        assert orc.or_get_embedding(P(want), gtype, P(blk), dim, tok) == 0
        assert_bits(ctx.download(od, np.float32, dim), want)


def test_argmax_first_index(ctx):
    x = np.zeros(130560, np.float32)
    x[[5, 77777, 130000]] = 3.0
    od = ctx.zeros(4)
    announce("argmax")
    mcpm.check(ctx.lib.mcpm_argmax(ctx.h, up(ctx, x).ptr, x.size, od.ptr))
    assert ctx.download(od, np.int32, 1)[0] == 5
    x = np.random.default_rng(9).standard_normal(1000).astype(np.float32)
    mcpm.check(ctx.lib.mcpm_argmax(ctx.h, up(ctx, x).ptr, x.size, od.ptr))
    assert ctx.download(od, np.int32, 1)[0] == int(np.argmax(x))


# ------------------------------------ single-op workloads C1-C3 (2.4B shapes)

def _weights(seed, tid, rows, cols, gtype, real_cols=None):
    real_cols = real_cols or cols
    w = mcpm.synth_normal(seed, tid, rows * real_cols, 0.0, 0.02).reshape(rows, real_cols)
    if real_cols < cols:
        w = np.concatenate([w, np.zeros((rows, cols - real_cols), np.float32)], axis=1)
    return mcpm.quantize_rows(gtype, w)


def test_c1_single_gemv_golden(ctx, orc):
    g = golden("c1_q4k_gemv.npz")
    s = int(g["seed"])
    W = _weights(s, 1, 5760, 2304, mcpm.TYPE_Q4_K)
    import hashlib
    assert hashlib.sha256(W.tobytes()).hexdigest() == str(g["w_sha"]), "weight generator changed"
    x = mcpm.synth_normal(s, 2, 2304)
    announce("C1 Q4_K GEMV 5760x2304")
    t = ctx.tensor(W, 12, 2304, 5760)
    od = ctx.zeros(5760 * 4)
    mcpm.check(ctx.lib.mcpm_gemv_q4_K(ctx.h, t.h, up(ctx, x).ptr, od.ptr, 5760, 2304))
    got = ctx.download(od, np.float32, 5760)
    assert_bits(got, g["y"])  # the reference's AVX2 matmul, bit for bit
    assert_close(got, g["y"], 1e-3)


def test_c2_ffn_block_golden(ctx, orc):
    g = golden("c2_ffn_block.npz")
    s = int(g["seed"])
    H, F, FP = 2304, 5760, 5888
    x = mcpm.synth_normal(s, 1, H)
    gamma = mcpm.synth_normal(s, 2, H, 1.0, 0.1)
    Wg = _weights(s, 3, F, H, mcpm.TYPE_Q4_K)
    Wu = _weights(s, 4, F, H, mcpm.TYPE_Q4_K)
    Wd = _weights(s, 5, H, FP, mcpm.TYPE_Q6_K, real_cols=F)
    announce("C2 FFN block")
    tg, tu, td = ctx.tensor(Wg, 12, H, F), ctx.tensor(Wu, 12, H, F), ctx.tensor(Wd, 14, FP, H)
    xd, gd = up(ctx, x), up(ctx, gamma)
    xq = ctx.zeros(9 * 292)
    mcpm.check(ctx.lib.mcpm_rmsnorm_and_quantize_q8k(ctx.h, xq.ptr, xd.ptr, gd.ptr, H, 1e-6))
    gt, ut = ctx.zeros(FP * 4), ctx.zeros(FP * 4)
    mcpm.check(ctx.lib.mcpm_gemv_gate_up_q4_K_q8_K(ctx.h, tg.h, tu.h, xq.ptr, gt.ptr, ut.ptr, F, H))
    hq = ctx.zeros(23 * 292)
    mcpm.check(ctx.lib.mcpm_swiglu_and_quantize_q8k(ctx.h, hq.ptr, gt.ptr, ut.ptr, FP))
    dd = ctx.zeros(H * 4)
    mcpm.check(ctx.lib.mcpm_matmul_q8k(ctx.h, td.h, hq.ptr, FP, dd.ptr))
    gate = ctx.download(gt, np.float32, F)
    upv = ctx.download(ut, np.float32, F)
    down = ctx.download(dd, np.float32, H)
    assert_close(gate, g["gate"])
    assert_close(upv, g["up"])
    assert_close(down, g["down"])
    # given the reference's own Q8_K inputs, the GEMVs match it bit for bit
    xq_ref = g["xq"].view(mcpm.Q8_K)
    mcpm.check(ctx.lib.mcpm_gemv_gate_up_q4_K_q8_K(ctx.h, tg.h, tu.h, up(ctx, xq_ref).ptr, gt.ptr, ut.ptr, F, H))
    assert_bits(ctx.download(gt, np.float32, F), g["gate"])
    assert_bits(ctx.download(ut, np.float32, F), g["up"])
    mcpm.check(ctx.lib.mcpm_matmul_q8k(ctx.h, td.h, up(ctx, g["hq"].view(mcpm.Q8_K)).ptr, FP, dd.ptr))
    assert_bits(ctx.download(dd, np.float32, H), g["down"])


@pytest.mark.parametrize("ctxlen", [512, 2048, 4096])
def test_c3_attention_golden(ctx, orc, ctxlen):
    g = golden("c3_attention.npz")
    s = int(g["seed"])
    H, NH, NKV, HD = 2304, 32, 8, 64
    x = mcpm.synth_normal(s, 1, H)
    Wq = _weights(s, 2, NH * HD, H, mcpm.TYPE_Q4_K)
    Wk = _weights(s, 3, NKV * HD, H, mcpm.TYPE_Q4_K)
    Wv = _weights(s, 4, NKV * HD, H, mcpm.TYPE_Q4_K)
    announce(f"C3 attention ctx={ctxlen}")
    tq, tk, tv = ctx.tensor(Wq, 12, H, NH * HD), ctx.tensor(Wk, 12, H, NKV * HD), ctx.tensor(Wv, 12, H, NKV * HD)
    xq = ctx.zeros(9 * 292)
    mcpm.check(ctx.lib.mcpm_quantize_row_q8_K(ctx.h, up(ctx, x).ptr, H, xq.ptr))
    qd, kd, vd = ctx.zeros(NH * HD * 4), ctx.zeros(NKV * HD * 4), ctx.zeros(NKV * HD * 4)
    mcpm.check(ctx.lib.mcpm_gemv_qkv_q8_K(ctx.h, tq.h, tk.h, tv.h, xq.ptr, qd.ptr, kd.ptr, vd.ptr, NH * HD, NKV * HD,
                                          H))
    assert_bits(ctx.download(qd, np.float32, NH * HD), g["q"])
    assert_bits(ctx.download(kd, np.float32, NKV * HD), g["k"])
    assert_bits(ctx.download(vd, np.float32, NKV * HD), g["v"])
    mcpm.check(ctx.lib.mcpm_apply_rope(ctx.h, qd.ptr, ctxlen, NH, HD, 10000.0))
    mcpm.check(ctx.lib.mcpm_apply_rope(ctx.h, kd.ptr, ctxlen, NKV, HD, 10000.0))
    # fp32 RoPE angles pos*theta carry up to pos*2^-24 rad of rounding, so two
    # fp32 implementations agree normwise but not on near-zero elements.
    assert_close(ctx.download(qd, np.float32, NH * HD), g[f"q_rope_{ctxlen}"], floor=0.2)
    assert_close(ctx.download(kd, np.float32, NKV * HD), g[f"k_rope_{ctxlen}"], floor=0.2)
    ms = ctxlen + 1
    kc = mcpm.synth_normal(s, 10 + ctxlen, ms * NKV * HD)
    vc = mcpm.synth_normal(s, 20000 + ctxlen, ms * NKV * HD)
    # the reference's roped q/k as inputs isolate the attention itself
    qr, kr = up(ctx, g[f"q_rope_{ctxlen}"]), up(ctx, g[f"k_rope_{ctxlen}"])
    od = ctx.zeros(NH * HD * 4)
    mcpm.check(ctx.lib.mcpm_execute_attention(ctx.h, od.ptr, qr.ptr, kr.ptr, vd.ptr, up(ctx, kc).ptr,
                                              up(ctx, vc).ptr, ctxlen, ms, NH, NKV, HD))
    assert_close(ctx.download(od, np.float32, NH * HD), g[f"attn_{ctxlen}"])


def test_op_timing_counts_gemv_kernels(ctx):
    """mcpm_set_op_timing / mcpm_op_time: each timed GEMV launch adds one
    event pair, the count restarts after each read, and the results of a
    timed launch are those of an untimed one."""
    W = _weights(20260105, 7, 512, 768, mcpm.TYPE_Q4_K)
    x = mcpm.synth_normal(20260105, 8, 768)
    announce("op timing")
    t = ctx.tensor(W, mcpm.TYPE_Q4_K, 768, 512)
    xd = up(ctx, x)
    o0, o1 = ctx.zeros(512 * 4), ctx.zeros(512 * 4)
    try:
        mcpm.check(ctx.lib.mcpm_gemv_q4_K(ctx.h, t.h, xd.ptr, o0.ptr, 512, 768))
        ctx.set_op_timing(True)
        for _ in range(3):
            mcpm.check(ctx.lib.mcpm_gemv_q4_K(ctx.h, t.h, xd.ptr, o1.ptr, 512, 768))
        ms, n = ctx.op_time()
        assert n == 3 and ms > 0.0
        assert ctx.op_time() == (0.0, 0)
        ctx.set_op_timing(False)
        mcpm.check(ctx.lib.mcpm_gemv_q4_K(ctx.h, t.h, xd.ptr, o1.ptr, 512, 768))
        assert ctx.op_time() == (0.0, 0)
        assert_bits(ctx.download(o1, np.float32, 512), ctx.download(o0, np.float32, 512))
    finally:
        ctx.set_op_timing(False)
        ctx.sync()


def test_stream_read_covers_every_word(ctx):
    """mcpm_stream_read (the read floor's kernel): work group b xors the
    16-byte words i with (i // 256) % grid == b, so every word is read once;
    bad sizes, alignment and grids are refused before any launch."""
    rng = np.random.default_rng(20260105)
    n16 = 3 * 4096 + 17
    words = rng.integers(0, 2**32, size=n16 * 4, dtype=np.uint64).astype(np.uint32)
    announce("stream read")
    src = ctx.upload(words)
    for grid in (1, 7, 64, 300):
        sink = ctx.zeros(grid * 4)
        try:
            mcpm.check(ctx.lib.mcpm_stream_read(ctx.h, src.ptr, n16 * 16, grid, sink.ptr))
            got = ctx.download(sink, np.uint32, grid)
            per16 = np.bitwise_xor.reduce(words.reshape(n16, 4), axis=1)
            owner = (np.arange(n16) // 256) % grid
            want = np.zeros(grid, np.uint32)
            np.bitwise_xor.at(want, owner, per16)
            assert np.array_equal(got, want), grid
        finally:
            sink.free()
    sink = ctx.zeros(64 * 4)
    try:
        for ptr, nbytes, grid in ((src.ptr, 40, 4), (src.ptr + 4, 64, 4), (src.ptr, 64, 0), (src.ptr, 0, 4),
                                  (src.ptr, 64, 65537)):
            assert ctx.lib.mcpm_stream_read(ctx.h, ptr, nbytes, grid, sink.ptr) == -2  # MCPM_ERR_ARG
    finally:
        sink.free()
        src.free()
        ctx.sync()
