"""Random ggml blocks and small utilities shared by the CPU and GPU tests."""
import numpy as np

import mcpm


def fp16_bits(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def rand_q4k(rng, n, extreme=False):
    """n random Q4_K blocks.  Any byte pattern is a valid block; d/dmin are
    kept finite.  extreme=True mixes in q in {0,15}, scales/mins in {0,63},
    subnormal and maximal d."""
    b = np.zeros(n, mcpm.Q4_K)
    b["d"] = fp16_bits(rng.uniform(1e-4, 3e-3, n))
    b["dmin"] = fp16_bits(rng.uniform(1e-4, 3e-3, n))
    b["scales"] = rng.integers(0, 256, (n, 12))
    b["qs"] = rng.integers(0, 256, (n, 128))
    if extreme:
        k = n // 4
        b["qs"][:k] = rng.choice(np.array([0x00, 0xff, 0x0f, 0xf0], np.uint8), (k, 128))
        b["scales"][:k] = rng.choice(np.array([0x00, 0xff, 0x3f, 0xc0], np.uint8), (k, 12))
        b["d"][k:2 * k] = rng.choice(np.array([0x0001, 0x03ff, 0x7bff, 0x0400, 0x8001], np.uint16), k)
        b["dmin"][k:2 * k] = rng.choice(np.array([0x0001, 0x03ff, 0x7bff, 0x0000], np.uint16), k)
    return b


def rand_q6k(rng, n, extreme=False):
    b = np.zeros(n, mcpm.Q6_K)
    b["d"] = fp16_bits(rng.uniform(1e-5, 3e-4, n))
    b["scales"] = rng.integers(-128, 128, (n, 16))
    b["ql"] = rng.integers(0, 256, (n, 128))
    b["qh"] = rng.integers(0, 256, (n, 64))
    if extreme:
        k = n // 4
        b["ql"][:k] = rng.choice(np.array([0x00, 0xff], np.uint8), (k, 128))
        b["qh"][:k] = rng.choice(np.array([0x00, 0xff, 0x55, 0xaa], np.uint8), (k, 64))
        b["scales"][:k] = rng.choice(np.array([-128, 127, 0, -1], np.int8), (k, 16))
        b["d"][k:2 * k] = rng.choice(np.array([0x0001, 0x03ff, 0x7bff, 0x0400, 0x8400], np.uint16), k)
    return b


def rand_q8_0(rng, n):
    b = np.zeros(n, mcpm.Q8_0)
    b["d"] = fp16_bits(rng.uniform(1e-4, 3e-3, n))
    b["qs"] = rng.integers(-128, 128, (n, 32))
    return b


def rand_act(rng, n, scale=1.0):
    return (rng.standard_normal(n) * scale).astype(np.float32)


def q8k_from(orc, x, ties_away=0):
    out = np.zeros(x.size // 256, mcpm.Q8_K)
    orc.or_quantize_row_q8_K(x.ctypes.data, x.size, out.ctypes.data, ties_away)
    return out


def deq_q8k(b):
    return (b["qs"].astype(np.float64) * b["d"][:, None].astype(np.float64)).ravel()


def header_functions(path):
    """Function names declared in a C header (mcpm_* entry points)."""
    import re
    txt = open(path).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(mcpm_[a-zA-Z0-9_]+)\s*\(", txt)))
