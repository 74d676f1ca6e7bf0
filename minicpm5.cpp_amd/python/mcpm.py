"""ctypes binding of libmcpm_hip.so (include/mcpm_hip.h) for tests and benchmarks.

The library is the product: there is no fallback.  If it has not been built,
load_library() raises with the build command instead of silently running
something else.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.dirname(_HERE)
LIB_PATH = os.path.join(PKG_DIR, "libmcpm_hip.so")

TYPE_F32, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K = 0, 8, 12, 14
KC_QKV, KC_ATTN, KC_OPROJ, KC_GATE_UP, KC_DOWN, KC_LM_HEAD, KC_LAYERS = range(7)
# mcpm_engine_set_persistent's default mode
PERSIST_AUTO = 2
KC_NAMES = ["qkv", "attn", "oproj", "gate_up", "down", "lm_head", "layers"]
# include/mcpm_hip.h error codes
ERR_HIP, ERR_ARG, ERR_UNSUPPORTED, ERR_CONTEXT, ERR_IO, ERR_FORMAT, ERR_NOMEM = -1, -2, -3, -4, -5, -6, -7

# ggml block layouts (reference include/ops.h:33-65)
Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", 32)])
Q4_K = np.dtype([("d", "<u2"), ("dmin", "<u2"), ("scales", "u1", 12), ("qs", "u1", 128)])
Q6_K = np.dtype([("ql", "u1", 128), ("qh", "u1", 64), ("scales", "i1", 16), ("d", "<u2")])
Q8_K = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])
assert (Q8_0.itemsize, Q4_K.itemsize, Q6_K.itemsize, Q8_K.itemsize) == (34, 144, 210, 292)
BLOCK = {TYPE_Q8_0: (Q8_0, 32), TYPE_Q4_K: (Q4_K, 256), TYPE_Q6_K: (Q6_K, 256)}


class McpmError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"mcpm error {code}: {msg}")
        self.code = code


class ModelConfig(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int), ("dim", C.c_int), ("n_heads", C.c_int), ("n_kv_heads", C.c_int),
        ("head_dim", C.c_int), ("ffn", C.c_int), ("ffn_pad", C.c_int), ("vocab", C.c_int),
        ("rope_base", C.c_float), ("eps", C.c_float), ("tied_embeddings", C.c_int),
    ]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


def make_config(n_layers, dim, n_heads, n_kv_heads, head_dim, ffn, vocab, rope_base=10000.0, eps=1e-6, tied=1):
    return ModelConfig(n_layers, dim, n_heads, n_kv_heads, head_dim, ffn, (ffn + 255) // 256 * 256, vocab,
                       rope_base, eps, tied)


# MiniCPM5-2.4B-shaped decoder: 40 layers, hidden 2304, 32/8 heads of 64,
# FFN 5760, vocab 130560, tied Q6_K embedding, RoPE base 1e4.
def config_2p4b():
    return make_config(40, 2304, 32, 8, 64, 5760, 130560)


_lib = None
_P = C.c_void_p
_I = C.c_int
_I64 = C.c_int64
_F = C.c_float
_SZ = C.c_size_t

_SIGS = {
    "mcpm_init": (_I, [_I, C.POINTER(_P)]),
    "mcpm_destroy": (None, [_P]),
    "mcpm_last_error": (C.c_char_p, []),
    "mcpm_sync": (_I, [_P]),
    "mcpm_device_info": (_I, [_P, C.POINTER(_I), C.c_char_p, _SZ]),
    "mcpm_device_alloc": (_I, [_P, _SZ, C.POINTER(_P)]),
    "mcpm_stream_read": (_I, [_P, _P, _SZ, _I, _P]),
    "mcpm_device_free": (_I, [_P, _P]),
    "mcpm_copy_to_device": (_I, [_P, _P, _P, _SZ]),
    "mcpm_copy_to_host": (_I, [_P, _P, _P, _SZ]),
    "mcpm_copy_device": (_I, [_P, _P, _P, _SZ]),
    "mcpm_engine_prefill": (_I, [_P, C.POINTER(C.c_int), _I, _I]),
    "mcpm_engine_set_prefill": (_I, [_P, _I]),
    "mcpm_engine_uses_prefill": (_I, [_P]),
    "mcpm_engine_read_kv": (_I, [_P, _I, _I, _I, _P, _P]),
    "mcpm_fill_device": (_I, [_P, _P, _I, _SZ]),
    "mcpm_tensor_upload": (_I, [_P, _P, _SZ, _I, _I64, _I64, C.POINTER(_P)]),
    "mcpm_tensor_download": (_I, [_P, _P, _P, _SZ]),
    "mcpm_tensor_info": (_I, [_P, C.POINTER(_I), C.POINTER(_I64), C.POINTER(_I64)]),
    "mcpm_tensor_free": (None, [_P]),
    "mcpm_tensor_dequantize_rows": (_I, [_P, _P, _I64, _I64, _P]),
    "mcpm_quantize_row_q8_K": (_I, [_P, _P, _I, _P]),
    "mcpm_gemv_q4_K_q8_K": (_I, [_P, _P, _P, _P, _I, _I]),
    "mcpm_gemv_q6_K_q8_K": (_I, [_P, _P, _P, _P, _I, _I]),
    "mcpm_gemv_qkv_q8_K": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I]),
    "mcpm_gemv_gate_up_q4_K_q8_K": (_I, [_P, _P, _P, _P, _P, _P, _I, _I]),
    "mcpm_gemv_q4_K": (_I, [_P, _P, _P, _P, _I, _I]),
    "mcpm_gemv_q6_K": (_I, [_P, _P, _P, _P, _I, _I]),
    "mcpm_gemv_q8_0": (_I, [_P, _P, _P, _P, _I, _I]),
    "mcpm_gemv_f32": (_I, [_P, _P, _P, _P, _I, _I]),
    "mcpm_matmul": (_I, [_P, _P, _P, _P]),
    "mcpm_matmul_q8k": (_I, [_P, _P, _P, _I, _P]),
    "mcpm_rmsnorm": (_I, [_P, _P, _P, _P, _I, _F]),
    "mcpm_rmsnorm_and_quantize_q8k": (_I, [_P, _P, _P, _P, _I, _F]),
    "mcpm_swiglu_and_quantize_q8k": (_I, [_P, _P, _P, _P, _I]),
    "mcpm_apply_rope": (_I, [_P, _P, _I, _I, _I, _F]),
    "mcpm_execute_attention": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "mcpm_execute_attention_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "mcpm_get_embedding": (_I, [_P, _P, _P, _I]),
    "mcpm_argmax": (_I, [_P, _P, _I, _P]),
    "mcpm_sample_device": (_I, [_P, _P, _I, _F, _F, _F, _P]),
    "mcpm_engine_load_gguf": (_I, [_P, C.c_char_p, C.POINTER(_P)]),
    "mcpm_engine_load_gguf_memory": (_I, [_P, _P, _SZ, C.POINTER(_P)]),
    "mcpm_engine_free": (None, [_P]),
    "mcpm_engine_config": (_I, [_P, C.POINTER(ModelConfig)]),
    "mcpm_engine_weight_bytes_per_token": (_I64, [_P]),
    "mcpm_engine_init_kv_cache": (_I, [_P, _I]),
    "mcpm_engine_forward": (_I, [_P, _I, _I, _I, _P, C.POINTER(_I)]),
    "mcpm_engine_generate_greedy": (_I, [_P, _P, _I, _I, _P]),
    "mcpm_engine_decode_steps": (_I, [_P, _I]),
    "mcpm_engine_tokens": (_I, [_P, _P, _I]),
    "mcpm_engine_generate_sampled": (_I, [_P, _P, _I, _I, _F, _F, C.c_uint32, _P]),
    "mcpm_engine_decode_sampled": (_I, [_P, _I, _F, _F, C.c_uint32]),
    "mcpm_engine_generate_greedy_at": (_I, [_P, _P, _I, _I, _I, _P]),
    "mcpm_engine_generate_sampled_at": (_I, [_P, _P, _I, _I, _I, _F, _F, C.c_uint32, _P]),
    "mcpm_sample_logits": (_I, [_P, _I, _F, _F, _F]),
    "mcpm_engine_set_graph": (_I, [_P, _I]),
    "mcpm_engine_set_persistent": (_I, [_P, _I]),
    "mcpm_engine_uses_persistent": (_I, [_P]),
    "mcpm_engine_persistent_fixed_shape": (_I, [_P]),
    "mcpm_engine_persistent_xcd_local": (_I, [_P]),
    "mcpm_engine_set_spin_limit": (_I, [_P, C.c_uint]),
    "mcpm_set_op_timing": (_I, [_P, _I]),
    "mcpm_op_time": (_I, [_P, C.POINTER(C.c_double), C.POINTER(_I64)]),
    "mcpm_engine_set_kernel_timing": (_I, [_P, _I]),
    "mcpm_engine_kernel_time": (_I, [_P, C.POINTER(C.c_double), C.POINTER(_I64)]),
    "mcpm_engine_kernel_bytes": (_I64, [_P, _I]),
    "mcpm_synth_gguf": (_I, [C.POINTER(ModelConfig), C.c_uint64, _I, C.c_char_p, C.POINTER(_P), C.POINTER(_SZ)]),
    "mcpm_free_host": (None, [_P]),
    "mcpm_synth_normal": (None, [C.c_uint64, C.c_uint64, _F, _F, _P, _SZ]),
    "mcpm_quantize_rows": (_I, [_I, _P, _I64, _I64, _P]),
    "mcpm_type_row_bytes": (_SZ, [_I, _I64]),
}


def load_library(path: str = LIB_PATH) -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is not built; run `make -C {PKG_DIR}` (or __graft_entry__.build()) first")
    lib = C.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols():
    return list(_SIGS)


def check(rc: int):
    if rc < 0:
        raise McpmError(rc, load_library().mcpm_last_error().decode(errors="replace"))
    return rc


def ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ------------------------------------------------------------ host helpers

def synth_normal(seed: int, tensor_id: int, n: int, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    load_library().mcpm_synth_normal(seed, tensor_id, mean, std, ptr(out), n)
    return out


def quantize_rows(ggml_type: int, x: np.ndarray) -> np.ndarray:
    """Encode fp32 rows [rows, cols] into native ggml blocks (uint8 array)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    lib = load_library()
    rb = lib.mcpm_type_row_bytes(ggml_type, cols)
    out = np.zeros(rows * rb, np.uint8)
    check(lib.mcpm_quantize_rows(ggml_type, ptr(x), rows, cols, ptr(out)))
    return out


def synth_gguf(cfg: ModelConfig, seed: int, mix: int = 0, path: str | None = None):
    """Random-init model as a GGUF image; returns bytes (path None) or the path."""
    lib = load_library()
    img = _P()
    n = _SZ()
    check(lib.mcpm_synth_gguf(C.byref(cfg), seed, mix, path.encode() if path else None, C.byref(img), C.byref(n)))
    if path:
        return path
    try:
        return np.ctypeslib.as_array(C.cast(img, C.POINTER(C.c_uint8)), shape=(n.value,)).copy()
    finally:
        lib.mcpm_free_host(img)


def sample_logits(logits: np.ndarray, temperature: float, top_p: float, r: float) -> int:
    logits = np.ascontiguousarray(logits, np.float32)
    return check(load_library().mcpm_sample_logits(ptr(logits), logits.size, temperature, top_p, r))


# ------------------------------------------------------------ device side

class DeviceBuffer:
    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = nbytes
        p = _P()
        check(ctx.lib.mcpm_device_alloc(ctx.h, nbytes, C.byref(p)))
        self.ptr = p.value

    def free(self):
        if self.ptr:
            self.ctx.lib.mcpm_device_free(self.ctx.h, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Tensor:
    def __init__(self, ctx: "Context", native: np.ndarray, ggml_type: int, cols: int, rows: int):
        native = np.ascontiguousarray(native).view(np.uint8)
        self.ctx, self.type, self.cols, self.rows = ctx, ggml_type, cols, rows
        self.nbytes = native.nbytes
        h = _P()
        check(ctx.lib.mcpm_tensor_upload(ctx.h, ptr(native), native.nbytes, ggml_type, cols, rows, C.byref(h)))
        self.h = h.value

    def download(self) -> np.ndarray:
        out = np.zeros(self.nbytes, np.uint8)
        check(self.ctx.lib.mcpm_tensor_download(self.ctx.h, self.h, ptr(out), self.nbytes))
        return out

    def dequantize(self, row0=0, n_rows=None) -> np.ndarray:
        n_rows = self.rows - row0 if n_rows is None else n_rows
        buf = self.ctx.alloc(n_rows * self.cols * 4)
        check(self.ctx.lib.mcpm_tensor_dequantize_rows(self.ctx.h, self.h, row0, n_rows, buf.ptr))
        return self.ctx.download(buf, np.float32, (n_rows, self.cols))

    def free(self):
        if self.h:
            self.ctx.lib.mcpm_tensor_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = _P()
        check(self.lib.mcpm_init(device, C.byref(h)))
        self.h = h.value

    def info(self):
        n = _I()
        name = C.create_string_buffer(128)
        check(self.lib.mcpm_device_info(self.h, C.byref(n), name, 128))
        return n.value, name.value.decode()

    def sync(self):
        check(self.lib.mcpm_sync(self.h))

    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def upload(self, a: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(a)
        buf = DeviceBuffer(self, a.nbytes)
        check(self.lib.mcpm_copy_to_device(self.h, buf.ptr, ptr(a), a.nbytes))
        return buf

    def write(self, buf: DeviceBuffer, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= buf.nbytes
        check(self.lib.mcpm_copy_to_device(self.h, buf.ptr, ptr(a), a.nbytes))

    def download(self, buf: DeviceBuffer, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= buf.nbytes
        check(self.lib.mcpm_copy_to_host(self.h, ptr(out), buf.ptr, out.nbytes))
        return out

    def zeros(self, nbytes: int) -> DeviceBuffer:
        buf = DeviceBuffer(self, nbytes)
        check(self.lib.mcpm_fill_device(self.h, buf.ptr, 0, nbytes))
        return buf

    def tensor(self, native: np.ndarray, ggml_type: int, cols: int, rows: int) -> Tensor:
        return Tensor(self, native, ggml_type, cols, rows)

    def set_op_timing(self, enable: bool):
        check(self.lib.mcpm_set_op_timing(self.h, 1 if enable else 0))

    def op_time(self):
        """(summed kernel ms, timed launches) since the last call."""
        t = C.c_double()
        n = C.c_int64()
        check(self.lib.mcpm_op_time(self.h, C.byref(t), C.byref(n)))
        return t.value, n.value

    def close(self):
        if self.h:
            self.lib.mcpm_destroy(self.h)
            self.h = None


class Engine:
    def __init__(self, ctx: Context, gguf_path: str | None = None, image: np.ndarray | None = None):
        self.ctx, self.lib = ctx, ctx.lib
        h = _P()
        if gguf_path is not None:
            check(self.lib.mcpm_engine_load_gguf(ctx.h, gguf_path.encode(), C.byref(h)))
        else:
            image = np.ascontiguousarray(image, np.uint8)
            check(self.lib.mcpm_engine_load_gguf_memory(ctx.h, ptr(image), image.nbytes, C.byref(h)))
        self.h = h.value
        cfg = ModelConfig()
        check(self.lib.mcpm_engine_config(self.h, C.byref(cfg)))
        self.cfg = cfg

    def init_kv_cache(self, max_seq_len: int):
        check(self.lib.mcpm_engine_init_kv_cache(self.h, max_seq_len))
        self.max_seq_len = max_seq_len

    def forward(self, token: int, pos: int, max_seq_len: int | None = None, want_logits=True):
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        am = _I()
        check(self.lib.mcpm_engine_forward(self.h, token, pos, max_seq_len or self.max_seq_len,
                                           ptr(logits) if want_logits else None, C.byref(am)))
        return logits, am.value

    def generate_greedy(self, prompt, n_gen: int) -> np.ndarray:
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_gen, np.int32)
        check(self.lib.mcpm_engine_generate_greedy(self.h, ptr(prompt), prompt.size, n_gen, ptr(out)))
        return out

    def decode_steps(self, n: int):
        check(self.lib.mcpm_engine_decode_steps(self.h, n))

    def decode_sampled(self, n: int, temperature: float, top_p: float, seed: int):
        check(self.lib.mcpm_engine_decode_sampled(self.h, n, temperature, top_p, seed))

    def tokens(self, n: int) -> np.ndarray:
        out = np.empty(n, np.int32)
        check(self.lib.mcpm_engine_tokens(self.h, ptr(out), n))
        return out

    def sync(self):
        self.ctx.sync()

    def generate_greedy_at(self, tokens, pos0: int, n_gen: int) -> np.ndarray:
        """tokens at positions pos0.. after the cached rows below pos0, then n_gen greedy tokens."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(n_gen, np.int32)
        check(self.lib.mcpm_engine_generate_greedy_at(self.h, ptr(tokens), tokens.size, pos0, n_gen, ptr(out)))
        return out

    def generate_sampled_at(self, tokens, pos0: int, n_gen: int, temperature: float, top_p: float,
                            seed: int) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(n_gen, np.int32)
        check(self.lib.mcpm_engine_generate_sampled_at(self.h, ptr(tokens), tokens.size, pos0, n_gen, temperature,
                                                       top_p, seed, ptr(out)))
        return out

    def generate_sampled(self, prompt, n_gen: int, temperature: float, top_p: float, seed: int) -> np.ndarray:
        prompt = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_gen, np.int32)
        check(self.lib.mcpm_engine_generate_sampled(self.h, ptr(prompt), prompt.size, n_gen, temperature, top_p,
                                                    seed, ptr(out)))
        return out

    def set_graph(self, enable: bool):
        check(self.lib.mcpm_engine_set_graph(self.h, int(enable)))

    def set_persistent(self, mode):
        """False/0: five launches per layer; True/1: the persistent launch
        wherever the shape fits; PERSIST_AUTO (2, the default): only where it
        has an instance compiled for the shape."""
        check(self.lib.mcpm_engine_set_persistent(self.h, int(mode)))

    def uses_persistent(self) -> bool:
        return bool(self.lib.mcpm_engine_uses_persistent(self.h))

    def persistent_fixed_shape(self) -> bool:
        return bool(self.lib.mcpm_engine_persistent_fixed_shape(self.h))

    def persistent_xcd_local(self) -> bool:
        return bool(self.lib.mcpm_engine_persistent_xcd_local(self.h))

    def set_spin_limit(self, limit: int):
        check(self.lib.mcpm_engine_set_spin_limit(self.h, int(limit)))

    def set_prefill(self, enable: bool):
        check(self.lib.mcpm_engine_set_prefill(self.h, int(enable)))

    def uses_prefill(self) -> bool:
        return bool(self.lib.mcpm_engine_uses_prefill(self.h))

    def prefill(self, tokens, pos0: int = 0):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        check(self.lib.mcpm_engine_prefill(self.h, t.ctypes.data_as(C.POINTER(C.c_int)), t.size, pos0))

    def read_kv(self, layer: int, pos0: int, n: int):
        kvd = self.cfg.n_kv_heads * self.cfg.head_dim
        k = np.empty((n, kvd), np.float32)
        v = np.empty((n, kvd), np.float32)
        check(self.lib.mcpm_engine_read_kv(self.h, layer, pos0, n, k.ctypes.data, v.ctypes.data))
        return k, v

    def set_kernel_timing(self, kc: int):
        check(self.lib.mcpm_engine_set_kernel_timing(self.h, kc))

    def kernel_time(self):
        t = C.c_double()
        n = _I64()
        check(self.lib.mcpm_engine_kernel_time(self.h, C.byref(t), C.byref(n)))
        return t.value, n.value

    def kernel_bytes(self, kc: int) -> int:
        return self.lib.mcpm_engine_kernel_bytes(self.h, kc)

    def weight_bytes_per_token(self) -> int:
        return self.lib.mcpm_engine_weight_bytes_per_token(self.h)

    def free(self):
        if self.h:
            self.lib.mcpm_engine_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
