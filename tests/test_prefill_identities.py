"""The exact fp16 / fp32 identities the prefill GEMM's operand builds rely on
(csrc/mcpm_prefill.hip), checked exhaustively on the CPU: every scale, code
and field position the Q4_K and Q6_K formats allow.  A byte permute reads a
code byte t as the fp16 number 1024 + t; one fused multiply-add then forms
the A operand.  Each check computes the fused operation exactly (float64
holds every intermediate here exactly) and rounds once to fp16, as
v_pk_fma_f16 does, and compares with the exact product the reference's
integer arithmetic uses."""
import numpy as np

F16 = np.float16


def r16(x):
    """Round a float64 (exact here) once to fp16, back to float64."""
    return np.float64(F16(x))


def fma16(a, b, c):
    return r16(np.float64(a) * np.float64(b) + np.float64(c))


def test_q4k_operands_exact():
    """Q4_K, scales 0..63: sc from fp16 (1024 + sc) - 1024, sc/16 from
    (1024 + sc)/16 - 64, offsets -1024*s; low nibble t = q, high nibble read
    in place t = 16q: fma(1024 + t, s, -1024*s) == q*sc for every q."""
    for sc in range(64):
        h = 1024 + sc
        s_lo = r16(h - 1024.0)
        s_hi = fma16(h, r16(1.0 / 16), r16(-64.0))
        m_lo, m_hi = r16(s_lo * -1024.0), r16(s_hi * -1024.0)
        assert (s_lo, s_hi, m_lo, m_hi) == (sc, sc / 16, -1024 * sc, -64 * sc)
        for q in range(16):
            assert fma16(1024 + q, s_lo, m_lo) == q * sc
            assert fma16(1024 + 16 * q, s_hi, m_hi) == q * sc


def test_q6k_operands_exact():
    """Q6_K, signed scales -128..127 as u = sc + 128: a field at bit p of its
    byte reads as t = code*2^p and takes s = sc*2^-p/64 = (1024 + u)*(2^-p/64)
    - 18*2^-p and m = -16*sc*2^-p = (1024 + u)*(-16*2^-p) + 18432*2^-p; then
    fma(1024 + t, s, m) == code*sc/64 for the low nibbles (p = 0, 4) and the
    2-bit high fields (p = 0, 2, 4, 6)."""
    for sc in range(-128, 128):
        h = 1024 + sc + 128
        for p, codes in ((0, 16), (4, 16), (0, 4), (2, 4), (4, 4), (6, 4)):
            f = 2.0 ** -p
            c1, c2, o1, o2 = r16(f / 64), r16(-18 * f), r16(-16 * f), r16(18432 * f)
            assert (c1, c2, o1, o2) == (f / 64, -18 * f, -16 * f, 18432 * f)  # constants exact in fp16
            s = fma16(h, c1, c2)
            m = fma16(h, o1, o2)
            assert s == sc * f / 64 and m == -16 * sc * f
            for q in range(codes):
                assert fma16(1024 + q * 2 ** p, s, m) == q * sc / 64
        # the offset operand's pair entries: -sc/32 = (1024 + u)*(-1/32) + 36
        assert fma16(h, r16(-1 / 32), r16(36.0)) == -sc / 32


def test_q6k_scaled_chain_is_the_unscaled_chain():
    """With every Q6_K MFMA sum divided by 64 (exactly), the chain step
    fma(d*64, fma(16, T/64, S/64), acc) equals fma(d, fma(16, T, S), acc) in
    fp32: the 64 is a power of two, so it commutes with each rounding."""
    rng = np.random.default_rng(7)
    f32 = np.float32
    for _ in range(20000):
        S = f32(rng.integers(-(1 << 23), 1 << 23))
        T = f32(rng.integers(-(1 << 22), 1 << 22))
        d = f32(rng.standard_normal() * 10.0 ** rng.integers(-8, 2))
        acc = f32(rng.standard_normal() * 10.0 ** rng.integers(-3, 3))

        def fma32(a, b, c):
            return f32(np.float64(a) * np.float64(b) + np.float64(c))  # exact product, one rounding

        v = fma32(f32(16.0), T, S)
        v64 = fma32(f32(16.0), f32(T / f32(64)), f32(S / f32(64)))
        assert v64 == v / f32(64)
        assert fma32(f32(d * f32(64)), v64, acc) == fma32(d, v, acc)
