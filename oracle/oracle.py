"""ctypes access to the CPU oracle (libmcpm_oracle.so) and to the reference's
own ops (_ref/librefops.so).  TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product.

Also holds an independent GGUF v3 reader (numpy) so the oracle can run a model
image without the product's C++ parser.
"""
from __future__ import annotations

import ctypes as C
import os
import struct
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libmcpm_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "librefops.so")

F32, Q8_0, Q4_K, Q6_K = 0, 8, 12, 14
Q8_K = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])

_P, _I, _F = C.c_void_p, C.c_int, C.c_float


def build(reference: bool = True):
    """Builds the oracle (and oracle/_ref when the reference sources exist)."""
    subprocess.run(["make", "-C", HERE, "liboracle"], check=True, capture_output=True)
    if reference:
        subprocess.run(["make", "-C", HERE, "ref"], check=True, capture_output=True)


class OrConfig(C.Structure):
    _fields_ = [("n_layers", _I), ("dim", _I), ("n_heads", _I), ("n_kv_heads", _I), ("head_dim", _I),
                ("ffn", _I), ("ffn_pad", _I), ("vocab", _I), ("rope_base", _F), ("eps", _F)]


class OrLayer(C.Structure):
    _fields_ = [("attn_norm", _P), ("wq", _P), ("wk", _P), ("wv", _P), ("wv_type", _I), ("wo", _P),
                ("wo_type", _I), ("ffn_norm", _P), ("wg", _P), ("wu", _P), ("wd", _P), ("wd_type", _I)]


_ORACLE_SIGS = {
    "or_fp16_to_fp32": (_F, [C.c_uint16]),
    "or_q4k_scales_mins": (None, [_P, _P, _P]),
    "or_expf": (_F, [_F]),
    "or_quantize_row_q8_K": (None, [_P, _I, _P, _I]),
    "or_dequant_row": (None, [_I, _P, _I, _P]),
    "or_q4k_block_lanes": (None, [_P, _P, _P, _P]),
    "or_q6k_block_lanes": (None, [_P, _P, _P]),
    "or_gemv_q4_K_q8_K": (None, [_P, _P, _P, _I, _I]),
    "or_gemv_q6_K_q8_K": (None, [_P, _P, _P, _I, _I]),
    "or_gemv_qkv_q8_K": (None, [_P, _P, _P, _I, _P, _P, _P, _P, _I, _I, _I]),
    "or_gemv_gate_up_q4_K_q8_K": (None, [_P, _P, _P, _P, _P, _I, _I]),
    "or_gemv_f32": (None, [_P, _P, _P, _I, _I]),
    "or_gemv_q8_0": (None, [_P, _P, _P, _I, _I]),
    "or_gemv_q4_K_f32act": (None, [_P, _P, _P, _I, _I]),
    "or_gemv_q6_K_f32act": (None, [_P, _P, _P, _I, _I]),
    "or_matmul": (_I, [_I, _P, _P, _P, _I, _I]),
    "or_matmul_q8k": (_I, [_I, _P, _P, _P, _I, _I]),
    "or_rms_scale": (_F, [_P, _I, _F]),
    "or_rmsnorm": (None, [_P, _P, _P, _I, _F]),
    "or_rmsnorm_and_quantize_q8k": (None, [_P, _P, _P, _I, _F]),
    "or_swiglu": (None, [_P, _P, _P, _I]),
    "or_swiglu_and_quantize_q8k": (None, [_P, _P, _P, _I]),
    "or_apply_rope": (None, [_P, _I, _I, _I, _F]),
    "or_attention": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "or_get_embedding": (_I, [_P, _I, _P, _I, _I]),
    "or_argmax": (_I, [_P, _I]),
    "or_set_threads": (None, [_I]),
    "or_model_create": (_P, [C.POINTER(OrConfig), _P, _I, _P, _P, _I, C.POINTER(OrLayer)]),
    "or_model_init_kv": (_I, [_P, _I]),
    "or_model_forward": (_I, [_P, _I, _I, _P]),
    "or_model_forward_kv": (_I, [_P, _I, _I]),
    "or_model_hidden": (_P, [_P]),
    "or_model_read_kv": (_I, [_P, _I, _I, _I, _P, _P]),
    "or_model_free": (None, [_P]),
    "or_mt_seed": (None, [_P, C.c_uint32]),
    "or_mt_next": (C.c_uint32, [_P]),
    "or_mt_uniform01": (_F, [_P]),
    "or_sample": (_I, [_P, _I, _F, _F, _F]),
    "or_sample_blocked": (_I, [_P, _I, _F, _F, _F]),
}

_REF_SIGS = {
    "ref_set_threads": (None, [_I]),
    "ref_fp16_to_fp32": (_F, [C.c_uint16]),
    "ref_decode_q4k_scales_mins": (None, [_P, _P, _P]),
    "ref_get_scale_min_k4": (None, [_I, _P, _P, _P]),
    "ref_quantize_row_q8_K": (None, [_P, _I, _P]),
    "ref_quantize_row_q8_K_scalar": (None, [_P, _I, _P]),
    "ref_rmsnorm_and_quantize_q8k": (None, [_P, _P, _P, _I, _F]),
    "ref_swiglu_and_quantize_q8k": (None, [_P, _P, _P, _I]),
    "ref_rmsnorm": (None, [_P, _P, _P, _I, _F]),
    "ref_silu": (_F, [_F]),
    "ref_matmul": (None, [_I, _P, _P, _P, _I, _I]),
    "ref_matmul_q8k": (None, [_I, _P, _P, _P, _I, _I]),
    "ref_matmul_qkv_q8k": (None, [_P, _P, _P, _I, _P, _P, _P, _P, _I, _I, _I]),
    "ref_matmul_gate_up_q8k": (None, [_P, _P, _P, _P, _P, _I, _I]),
    "ref_gemv_q4_K_scalar": (None, [_P, _P, _P, _I, _I]),
    "ref_gemv_q6_K_scalar": (None, [_P, _P, _P, _I, _I]),
    "ref_gemv_q4_K_q8_K_scalar": (None, [_P, _P, _P, _I, _I]),
    "ref_gemv_q6_K_q8_K_scalar": (None, [_P, _P, _P, _I, _I]),
    "ref_gemv_f32": (None, [_P, _P, _P, _I, _I]),
    "ref_gemv_q8_0": (None, [_P, _P, _P, _I, _I]),
    "ref_apply_rope": (None, [_P, _I, _I, _I, _I, _F]),
    "ref_execute_attention": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "ref_get_embedding": (None, [_P, _I, _P, _I, _I, _I]),
    "ref_model_create": (_P, [C.POINTER(OrConfig), _P, _I, _P, _P, _I, C.POINTER(OrLayer)]),
    "ref_model_init_kv": (None, [_P, _I]),
    "ref_model_forward": (_I, [_P, _P, _I, _P]),
    "ref_model_hidden": (_P, [_P]),
    "ref_model_free": (None, [_P]),
}

_oracle = None
_ref = None


def _bind(path, sigs):
    lib = C.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def oracle():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            build(reference=False)
        _oracle = _bind(ORACLE_SO, _ORACLE_SIGS)
    return _oracle


def reference():
    """The reference's compiled ops, or None where oracle/_ref is not built."""
    global _ref
    if _ref is None and os.path.exists(REF_SO):
        _ref = _bind(REF_SO, _REF_SIGS)
    return _ref


def ptr(a):
    return None if a is None else a.ctypes.data


# ------------------------------------------------------------ GGUF reader

_SCALAR = {0: "<u1", 1: "<i1", 2: "<u2", 3: "<i2", 4: "<u4", 5: "<i4", 6: "<f4", 7: "<u1", 10: "<u8", 11: "<i8",
           12: "<f8"}


def tensor_nbytes(ggml_type, dims):
    cols = dims[0]
    rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
    if ggml_type == F32:
        return cols * rows * 4
    if ggml_type == Q8_0:
        return cols // 32 * 34 * rows
    if ggml_type == Q4_K:
        return cols // 256 * 144 * rows
    if ggml_type == Q6_K:
        return cols // 256 * 210 * rows
    raise ValueError(f"type {ggml_type}")


def read_gguf(image: np.ndarray):
    """Returns (kv dict, {name: (type, dims, uint8 view)}) of a GGUF v2/v3 image."""
    buf = memoryview(image)
    off = 0

    def take(fmt):
        nonlocal off
        v = struct.unpack_from(fmt, buf, off)
        off += struct.calcsize(fmt)
        return v[0]

    def string():
        nonlocal off
        n = take("<Q")
        s = bytes(buf[off:off + n]).decode()
        off += n
        return s

    assert take("<I") == 0x46554747, "bad magic"
    version = take("<I")
    assert version in (2, 3)
    n_t, n_kv = take("<Q"), take("<Q")
    kv = {}
    for _ in range(n_kv):
        k = string()
        t = take("<I")
        if t == 8:
            kv[k] = string()
        elif t == 9:
            at, n = take("<I"), take("<Q")
            if at == 8:
                kv[k] = [string() for _ in range(n)]
            else:
                dt = np.dtype(_SCALAR[at])
                kv[k] = np.frombuffer(buf, dt, n, off)
                off += dt.itemsize * n
        else:
            dt = np.dtype(_SCALAR[t])
            kv[k] = np.frombuffer(buf, dt, 1, off)[0].item()
            off += dt.itemsize
    infos = []
    for _ in range(n_t):
        name = string()
        nd = take("<I")
        dims = [take("<Q") for _ in range(nd)]
        t = take("<I")
        o = take("<Q")
        infos.append((name, t, dims, o))
    align = int(kv.get("general.alignment", 32))
    start = (off + align - 1) // align * align
    tensors = {}
    for name, t, dims, o in infos:
        nb = tensor_nbytes(t, dims)
        tensors[name] = (t, dims, image[start + o:start + o + nb])
    return kv, tensors


class OracleModel:
    """The oracle's forward() over a GGUF image (weights stay in `image`)."""

    def __init__(self, image: np.ndarray, use_reference_ops: bool = False):
        kv, T = read_gguf(image)
        self.image = image
        arch = kv.get("general.architecture", "llama")
        g = lambda k, d=None: kv.get(f"{arch}.{k}", d)
        te = T["token_embd.weight"]
        dim = int(g("embedding_length"))
        n_heads = int(g("attention.head_count"))
        ffn_pad = T["blk.0.ffn_down.weight"][1][0]
        self.cfg = OrConfig(int(g("block_count")), dim, n_heads, int(g("attention.head_count_kv", n_heads)),
                            int(g("attention.key_length", dim // n_heads)), int(g("feed_forward_length")), ffn_pad,
                            te[1][1], float(g("rope.freq_base", 10000.0)),
                            float(g("attention.layer_norm_rms_epsilon", 1e-6)))
        self.embd_type, self.embd = te[0], te[2]
        out = T.get("output.weight", te)
        self.T = T
        layers = (OrLayer * self.cfg.n_layers)()
        for l in range(self.cfg.n_layers):
            p = f"blk.{l}."
            t = lambda n: T[p + n]
            layers[l] = OrLayer(ptr(t("attn_norm.weight")[2]), ptr(t("attn_q.weight")[2]),
                                ptr(t("attn_k.weight")[2]), ptr(t("attn_v.weight")[2]), t("attn_v.weight")[0],
                                ptr(t("attn_output.weight")[2]), t("attn_output.weight")[0],
                                ptr(t("ffn_norm.weight")[2]), ptr(t("ffn_gate.weight")[2]),
                                ptr(t("ffn_up.weight")[2]), ptr(t("ffn_down.weight")[2]), t("ffn_down.weight")[0])
        self.layers = layers
        self.ref = use_reference_ops
        lib = reference() if use_reference_ops else oracle()
        if lib is None:
            raise FileNotFoundError("oracle/_ref/librefops.so is not built")
        self.lib = lib
        create = lib.ref_model_create if use_reference_ops else lib.or_model_create
        self.h = create(C.byref(self.cfg), ptr(self.embd), self.embd_type, ptr(T["output_norm.weight"][2]),
                        ptr(out[2]), out[0], layers)
        self._x = np.zeros(self.cfg.dim, np.float32)

    def init_kv(self, max_seq_len):
        if self.ref:
            self.lib.ref_model_init_kv(self.h, max_seq_len)
        else:
            assert self.lib.or_model_init_kv(self.h, max_seq_len) == 0

    def forward(self, token, pos, logits=None):
        if self.ref:
            # the reference's get_embedding is Q4_K-only; the row comes from the oracle
            oracle().or_get_embedding(ptr(self._x), self.embd_type, ptr(self.embd), self.cfg.dim, token)
            return self.lib.ref_model_forward(self.h, ptr(self._x), pos, ptr(logits))
        return self.lib.or_model_forward(self.h, token, pos, ptr(logits))

    def forward_kv(self, token, pos):
        """The layers of a token whose logits are not read (its K/V rows
        reach the cache), as the engine's batched prefill leaves them."""
        if self.ref:
            lg = np.empty(self.cfg.vocab, np.float32)
            return self.forward(token, pos, lg)
        return self.lib.or_model_forward_kv(self.h, token, pos)

    def hidden(self):
        f = self.lib.ref_model_hidden if self.ref else self.lib.or_model_hidden
        return np.ctypeslib.as_array(C.cast(f(self.h), C.POINTER(C.c_float)), shape=(self.cfg.dim,)).copy()

    def generate_greedy(self, prompt, n_gen, logits_cb=None):
        self.init_kv(len(prompt) + n_gen)
        lg = np.empty(self.cfg.vocab, np.float32)
        nxt = None
        for p, t in enumerate(prompt):
            nxt = self.forward(int(t), p, lg)
        out = [nxt]
        if logits_cb:
            logits_cb(0, lg)
        for i in range(1, n_gen):
            nxt = self.forward(out[-1], len(prompt) + i - 1, lg)
            out.append(nxt)
            if logits_cb:
                logits_cb(i, lg)
        return np.array(out, np.int32)

    def generate_sampled(self, prompt, n_gen, temperature, top_p, seed, max_seq=None, logits_cb=None):
        """The engine's sampled loop (mcpm_engine_generate_sampled): prompt
        tokens but the last only fill the cache, the last gives the first
        logits; each logits vector is sampled by or_sample_blocked (the device
        sampler's arithmetic, src/sampler.cpp:8-73 with blocked double sums)
        on one draw of std::uniform_real_distribution<float> over
        std::mt19937(seed) per generated token."""
        orc = oracle()
        V = self.cfg.vocab
        self.init_kv(max_seq or len(prompt) + n_gen)
        gen = np.zeros(625, np.uint32)  # or_mt19937 state
        orc.or_mt_seed(gen.ctypes.data, seed)
        lg = np.empty(V, np.float32)
        for p, t in enumerate(prompt[:-1]):
            self.forward_kv(int(t), p)
        self.forward(int(prompt[-1]), len(prompt) - 1, lg)
        out = []
        for i in range(n_gen):
            if logits_cb:
                logits_cb(i, lg)
            nxt = orc.or_sample_blocked(ptr(lg), V, temperature, top_p, orc.or_mt_uniform01(gen.ctypes.data))
            out.append(nxt)
            if i < n_gen - 1:
                self.forward(int(nxt), len(prompt) + i, lg)
        return np.array(out, np.int32)

    def kv_rows(self, layer, pos0, n):
        """K and V cache rows [pos0, pos0+n) of one layer (copies)."""
        kvd = self.cfg.n_kv_heads * self.cfg.head_dim
        k = np.empty(n * kvd, np.float32)
        v = np.empty(n * kvd, np.float32)
        assert self.lib.or_model_read_kv(self.h, layer, pos0, n, ptr(k), ptr(v)) == 0
        return k, v

    def close(self):
        if self.h:
            (self.lib.ref_model_free if self.ref else self.lib.or_model_free)(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
