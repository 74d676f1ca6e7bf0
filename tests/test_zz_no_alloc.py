"""mcpm_execute_attention_noalloc (the allocation-free entry point) against
mcpm_execute_attention, the entry point whose kernels it shares: the same
output and cache rows bit for bit, on two calls in a row (the second on a
smaller shape, so stale records of the first stay in the shared scratch
array beyond what the second reads), a second call after one over NaN
inputs against the oracle, and the size limit rejected cleanly."""
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


@pytest.mark.parametrize("second", [((32, 8, 64), 100, 256), ((16, 2, 128), 700, 1024)])
def test_noalloc_attention_never_reads_a_previous_calls_records(ctx, orc, second):
    """A first call over NaN queries, keys and values leaves NaN partial
    records over 64 chunks of 32 heads in the shared scratch; the second,
    smaller call reads fewer records, and must equal the oracle's attention
    and the allocating entry point bit for bit, so a read of a leftover
    record would show as a NaN or a mismatch."""
    nh, nkv, hd = 32, 8, 64
    cap = 4096
    nan = np.full(cap * nkv * hd, np.nan, np.float32)
    announce("noalloc attention: NaN call, 64 chunks")
    out, _, _ = _run(ctx, ctx.lib.mcpm_execute_attention_noalloc, np.full(nh * hd, np.nan, np.float32),
                     np.full(nkv * hd, np.nan, np.float32), np.full(nkv * hd, np.nan, np.float32), nan, nan.copy(),
                     4000, cap, nh, nkv, hd)
    assert np.isnan(out).any()  # the records it left hold NaNs
    (nh, nkv, hd), pos, cap = second
    rng = np.random.default_rng(77 + pos)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    v = rng.standard_normal(nkv * hd).astype(np.float32)
    kc = rng.standard_normal(cap * nkv * hd).astype(np.float32)
    vc = rng.standard_normal(cap * nkv * hd).astype(np.float32)
    announce(f"noalloc attention after the NaN call: heads {nh}/{nkv}x{hd} pos {pos} cap {cap}")
    got = _run(ctx, ctx.lib.mcpm_execute_attention_noalloc, q, k, v, kc, vc, pos, cap, nh, nkv, hd)
    want = np.zeros(nh * hd, np.float32)
    kc2, vc2 = kc.copy(), vc.copy()
    P = lambda a: a.ctypes.data
    assert orc.or_attention(P(want), P(q), P(k), P(v), P(kc2), P(vc2), pos, cap, nh, nkv, hd) == 0
    assert not np.isnan(got[0]).any()
    assert_bits(got[0], want)
    assert_bits(got[1], kc2)
    assert_bits(got[2], vc2)
    alloc = _run(ctx, ctx.lib.mcpm_execute_attention, q, k, v, kc, vc, pos, cap, nh, nkv, hd)
    for g, w in zip(got, alloc):
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
