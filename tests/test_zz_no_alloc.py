"""mcpm_execute_attention_noalloc (the allocation-free entry point) against
mcpm_execute_attention, the entry point whose kernels it shares: the same
output and cache rows bit for bit, on two calls in a row (the second on a
smaller shape, so stale records of the first stay in the shared scratch
array beyond what the second reads), and the size limit rejected cleanly."""
import numpy as np
import pytest

import mcpm
from conftest import announce, assert_bits

pytestmark = pytest.mark.gpu

LIMIT_FLOATS = 64 * 64 * (128 + 2)  # include/mcpm_hip.h


def _up(ctx, a):
    return ctx.upload(np.ascontiguousarray(a))


def _run(ctx, fn, q, k, v, kc, vc, pos, cap, nh, nkv, hd):
    qd, kd, vd, kcd, vcd = _up(ctx, q), _up(ctx, k), _up(ctx, v), _up(ctx, kc), _up(ctx, vc)
    od = ctx.zeros(nh * hd * 4)
    mcpm.check(fn(ctx.h, od.ptr, qd.ptr, kd.ptr, vd.ptr, kcd.ptr, vcd.ptr, pos, cap, nh, nkv, hd))
    return (ctx.download(od, np.float32, nh * hd), ctx.download(kcd, np.float32, kc.size),
            ctx.download(vcd, np.float32, vc.size))


@pytest.mark.parametrize("cases", [
    [((32, 8, 64), 4000, 4096), ((32, 8, 64), 100, 256)],     # 64 chunks, then 4
    [((16, 2, 128), 2047, 2048), ((64, 8, 128), 700, 900)],  # another geometry, then a larger head count
])
def test_noalloc_attention_matches_allocating_entry(ctx, cases):
    for i, ((nh, nkv, hd), pos, cap) in enumerate(cases):
        rng = np.random.default_rng(100 + 7 * i + pos)
        q = rng.standard_normal(nh * hd).astype(np.float32)
        k = rng.standard_normal(nkv * hd).astype(np.float32)
        v = rng.standard_normal(nkv * hd).astype(np.float32)
        kc = rng.standard_normal(cap * nkv * hd).astype(np.float32)
        vc = rng.standard_normal(cap * nkv * hd).astype(np.float32)
        announce(f"noalloc attention call {i}: heads {nh}/{nkv}x{hd} pos {pos} cap {cap}")
        got = _run(ctx, ctx.lib.mcpm_execute_attention_noalloc, q, k, v, kc, vc, pos, cap, nh, nkv, hd)
        want = _run(ctx, ctx.lib.mcpm_execute_attention, q, k, v, kc, vc, pos, cap, nh, nkv, hd)
        for g, w in zip(got, want):
            assert_bits(g, w)


def test_noalloc_attention_rejects_sizes_beyond_the_scratch(ctx):
    nh, nkv, hd = 64, 8, 128
    cap = 64 * 65  # 65 chunks: 64 * 65 * 130 floats > the limit
    assert nh * (cap // 64) * (hd + 2) > LIMIT_FLOATS
    z = ctx.zeros(cap * nkv * hd * 4)
    od = ctx.upload(np.full(nh * hd, 3.0, np.float32))
    announce("noalloc attention over the limit")
    rc = ctx.lib.mcpm_execute_attention_noalloc(ctx.h, od.ptr, z.ptr, z.ptr, z.ptr, z.ptr, z.ptr, 10, cap, nh, nkv, hd)
    assert rc == -2  # MCPM_ERR_ARG
    assert np.all(ctx.download(od, np.float32, nh * hd) == 3.0)
    # the largest shape that fits runs
    cap = 64 * 64
    z = ctx.zeros(cap * nkv * hd * 4)
    od = ctx.zeros(nh * hd * 4)
    assert ctx.lib.mcpm_execute_attention_noalloc(ctx.h, od.ptr, z.ptr, z.ptr, z.ptr, z.ptr, z.ptr, cap - 1, cap, nh,
                                                  nkv, hd) == 0
