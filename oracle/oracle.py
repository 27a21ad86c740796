"""ctypes wrapper of liboracle.so -- the C restatement of flarellm's x86 decode
kernels (flare_oracle.c).  TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

OR_F32, OR_Q8_0, OR_Q4K, OR_Q6K = 0, 1, 2, 3
OR_KV_F32, OR_KV_F16, OR_KV_KIVI2, OR_KV_Q8, OR_KV_KIVI32 = 0, 1, 2, 3, 4


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    return LIB_PATH


class Config(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("hidden", "layers", "heads", "kv_heads", "head_dim", "inter", "vocab",
                                       "max_seq")] + [("eps", C.c_float), ("theta", C.c_float)] + \
               [(n, C.c_int) for n in ("layer_format", "embed_format", "output_format", "kv_mode")]


class Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down", "attn_norm",
                                          "ffn_norm")]


_lib = None
vp, sz, f32, i64 = C.c_void_p, C.c_size_t, C.c_float, C.c_int64


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        sig = {
            "or_set_threads": (None, [C.c_int]),
            "or_get_threads": (C.c_int, []),
            "or_set_order": (None, [C.c_int]),
            "or_f16_to_f32": (f32, [C.c_uint16]),
            "or_f32_to_f16_rne": (C.c_uint16, [f32]),
            "or_dequant_tensor": (C.c_int, [vp, C.c_int, sz, sz, vp]),
            "or_unpack_q4k_scales": (None, [vp, vp, vp]),
            "or_quantize_input_q8_0": (None, [vp, sz, vp, vp]),
            "or_rmsnorm_quantize_q8_0": (None, [vp, vp, sz, f32, vp, vp]),
            "or_rmsnorm": (None, [vp, vp, sz, f32, vp]),
            "or_block_dots_q8_0": (None, [vp, vp, sz, sz, vp]),
            "or_block_dots_q4k": (None, [vp, vp, sz, sz, vp]),
            "or_matvec_q8_0_preq": (None, [vp, vp, vp, sz, sz, vp]),
            "or_matvec_q4k_q8": (None, [vp, vp, vp, sz, sz, vp]),
            "or_matvec_argmax_q8_0_preq": (None, [vp, vp, vp, sz, sz, C.POINTER(i64), C.POINTER(f32)]),
            "or_matvec_argmax_q4k_q8_preq": (None, [vp, vp, vp, sz, sz, C.POINTER(i64), C.POINTER(f32)]),
            "or_matvec_argmax_f32": (None, [vp, vp, sz, sz, C.POINTER(i64), C.POINTER(f32)]),
            "or_matvec_f32": (None, [vp, vp, sz, sz, vp]),
            "or_rope_row": (None, [sz, sz, f32, vp, vp]),
            "or_apply_rope": (None, [vp, sz, sz, sz, f32]),
            "or_silu_mul": (None, [vp, vp, sz, vp]),
            "or_gqa_attention": (None, [vp, vp, vp, sz, sz, sz, sz, vp]),
            "or_kivi_quantize_to_packed": (None, [vp, sz, vp, C.POINTER(f32), C.POINTER(f32)]),
            "or_kivi32_qlen": (sz, [sz]),
            "or_kv_view": (None, [C.c_int, vp, vp, sz, sz, sz, vp, vp]),
            "or_model_create": (vp, [C.POINTER(Config), C.POINTER(Layer), vp, vp, vp]),
            "or_model_destroy": (None, [vp]),
            "or_model_reset": (None, [vp]),
            "or_forward_greedy": (i64, [vp, C.c_uint32, sz, C.POINTER(f32)]),
            "or_forward_logits": (None, [vp, C.c_uint32, sz, vp]),
            "or_model_final_normed": (C.POINTER(f32), [vp]),
            "or_generate_greedy": (None, [vp, vp, sz, sz, vp]),
            "or_sample": (i64, [vp, sz, f32, f32, C.c_int, f32, f32, vp, sz, f32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def set_threads(n: int | None = None) -> int:
    """Thread count of the oracle's row-parallel loops (None: this host's
    CPUs, at most 16).  Results do not depend on it."""
    if n is None:
        n = min(16, len(os.sched_getaffinity(0)))
    lib().or_set_threads(int(n))
    return int(lib().or_get_threads())


def set_order(order: int) -> None:
    """0: the reference's sequential sums (default); 1: pairwise sums (a
    measuring stick for order-dependent drift, not the reference)."""
    lib().or_set_order(int(order))


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---- kernels ---------------------------------------------------------------
def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.or_f16_to_f32(int(b)) for b in np.asarray(bits).ravel()], np.float32)


def f32_to_f16(vals: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.or_f32_to_f16_rne(float(v)) for v in np.asarray(vals, np.float32).ravel()], np.uint16)


def dequant(data: np.ndarray, fmt: int, rows: int, cols: int) -> np.ndarray:
    bpr = {OR_F32: cols, OR_Q8_0: cols // 32, OR_Q4K: cols // 256, OR_Q6K: cols // 256}[fmt]
    out = np.empty(rows * cols, np.float32)
    assert lib().or_dequant_tensor(_p(np.ascontiguousarray(data)), fmt, rows, bpr, _p(out)) == 0
    return out.reshape(rows, cols)


def unpack_q4k_scales(raw12: bytes):
    sc = (C.c_uint8 * 8)()
    mn = (C.c_uint8 * 8)()
    buf = (C.c_uint8 * 12)(*raw12)
    lib().or_unpack_q4k_scales(buf, sc, mn)
    return list(sc), list(mn)


def kivi32_qlen(T: int) -> int:
    return int(lib().or_kivi32_qlen(T))


def kv_view(kv_mode: int, K: np.ndarray, V: np.ndarray):
    """The K/V values a decode attention over all T rows of K, V ([T, nkv, D])
    reads in cache form kv_mode (OR_KV_F32 / F16 / Q8 / KIVI32)."""
    K = np.ascontiguousarray(K, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    T, nkv, D = K.shape
    Ko = np.empty_like(K)
    Vo = np.empty_like(V)
    lib().or_kv_view(kv_mode, _p(K), _p(V), T, nkv, D, _p(Ko), _p(Vo))
    return Ko, Vo


def quantize_q8(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    s = np.empty(x.size // 32, np.float32)
    q = np.empty(x.size, np.int8)
    lib().or_quantize_input_q8_0(_p(x), x.size, _p(s), _p(q))
    return q, s


def rmsnorm_quantize_q8(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    s = np.empty(x.size // 32, np.float32)
    q = np.empty(x.size, np.int8)
    lib().or_rmsnorm_quantize_q8_0(_p(x), _p(w), x.size, eps, _p(s), _p(q))
    return q, s


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().or_rmsnorm(_p(x), _p(w), x.size, eps, _p(out))
    return out


def block_dots(w: np.ndarray, fmt: int, rows: int, cols: int, q: np.ndarray) -> np.ndarray:
    L = lib()
    if fmt == OR_Q8_0:
        out = np.empty((rows, cols // 32), np.int32)
        L.or_block_dots_q8_0(_p(w), _p(q), rows, cols // 32, _p(out))
    else:
        out = np.empty((rows, cols // 256 * 8), np.int32)
        L.or_block_dots_q4k(_p(w), _p(q), rows, cols // 256, _p(out))
    return out


def matvec(w: np.ndarray, fmt: int, rows: int, cols: int, q: np.ndarray, s: np.ndarray) -> np.ndarray:
    out = np.empty(rows, np.float32)
    if fmt == OR_Q8_0:
        lib().or_matvec_q8_0_preq(_p(w), _p(s), _p(q), rows, cols // 32, _p(out))
    else:
        lib().or_matvec_q4k_q8(_p(w), _p(s), _p(q), rows, cols, _p(out))
    return out


def matvec_argmax(w, fmt, rows, cols, q, s):
    idx, val = C.c_int64(), C.c_float()
    if fmt == OR_Q8_0:
        lib().or_matvec_argmax_q8_0_preq(_p(w), _p(s), _p(q), rows, cols // 32, C.byref(idx), C.byref(val))
    else:
        lib().or_matvec_argmax_q4k_q8_preq(_p(w), _p(s), _p(q), rows, cols, C.byref(idx), C.byref(val))
    return idx.value, val.value


def matvec_argmax_f32(mat: np.ndarray, vec: np.ndarray):
    mat = np.ascontiguousarray(mat, np.float32)
    vec = np.ascontiguousarray(vec, np.float32)
    idx, val = C.c_int64(), C.c_float()
    lib().or_matvec_argmax_f32(_p(mat), _p(vec), mat.shape[0], mat.shape[1], C.byref(idx), C.byref(val))
    return idx.value, val.value


def matvec_f32(mat: np.ndarray, vec: np.ndarray) -> np.ndarray:
    mat = np.ascontiguousarray(mat, np.float32)
    vec = np.ascontiguousarray(vec, np.float32)
    out = np.empty(mat.shape[0], np.float32)
    lib().or_matvec_f32(_p(mat), _p(vec), mat.shape[0], mat.shape[1], _p(out))
    return out


def rope_row(head_dim: int, pos: int, theta: float):
    c = np.empty(head_dim // 2, np.float32)
    s = np.empty(head_dim // 2, np.float32)
    lib().or_rope_row(head_dim, pos, theta, _p(c), _p(s))
    return c, s


def apply_rope(data: np.ndarray, num_heads: int, head_dim: int, pos: int, theta: float) -> np.ndarray:
    d = np.array(data, np.float32, copy=True)
    lib().or_apply_rope(_p(d), num_heads, head_dim, pos, theta)
    return d


def silu_mul(g, u):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    lib().or_silu_mul(_p(g), _p(u), g.size, _p(out))
    return out


def gqa_attention(q, k_cache, v_cache, num_heads, num_kv_heads, head_dim, seq_len):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k_cache, np.float32)
    v = np.ascontiguousarray(v_cache, np.float32)
    out = np.empty(num_heads * head_dim, np.float32)
    lib().or_gqa_attention(_p(q), _p(k), _p(v), num_heads, num_kv_heads, head_dim, seq_len, _p(out))
    return out


def kivi_quantize_to_packed(v: np.ndarray):
    v = np.ascontiguousarray(v, np.float32)
    packed = np.zeros((v.size + 3) // 4, np.uint8)
    s, m = C.c_float(), C.c_float()
    lib().or_kivi_quantize_to_packed(_p(v), v.size, _p(packed), C.byref(s), C.byref(m))
    return packed, s.value, m.value


def sample(logits, temperature=0.7, top_p=0.9, top_k=40, repeat_penalty=1.1, min_p=0.0, prev=(), u=0.5) -> int:
    """Generator::step's penalty, temperature and sampler (generate.rs:210-230,
    sampling.rs); defaults are SamplingParams::default."""
    logits = np.ascontiguousarray(logits, np.float32)
    prev = np.ascontiguousarray(prev, np.uint32)
    return int(lib().or_sample(_p(logits), logits.size, temperature, top_p, int(top_k), repeat_penalty, min_p,
                               _p(prev) if prev.size else None, prev.size, u))


# ---- whole model -------------------------------------------------------------
class OracleModel:
    """Model::forward_greedy restated on the CPU over the same GGUF bytes."""

    def __init__(self, model, kv_mode: int = OR_KV_F32):
        spec = model.spec
        self.model = model  # keep the byte buffers alive
        cfg = Config(spec.hidden, spec.layers, spec.heads, spec.kv_heads, spec.head_dim, spec.inter, spec.vocab,
                     spec.max_seq, spec.eps, spec.theta, spec.layer_fmt, spec.embed_fmt,
                     -1 if spec.output_fmt is None else spec.output_fmt, kv_mode)
        layers = (Layer * spec.layers)()
        for i, ws in enumerate(model.layers):
            layers[i] = Layer(*[w.data.ctypes.data for w in ws], model.attn_norms[i].ctypes.data,
                              model.ffn_norms[i].ctypes.data)
        out = model.output.data.ctypes.data if model.output is not None else None
        self.h = lib().or_model_create(C.byref(cfg), layers, model.embedding.data.ctypes.data, out,
                                       model.output_norm.ctypes.data)
        self.spec = spec

    def close(self):
        if self.h:
            lib().or_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        lib().or_model_reset(self.h)

    def forward_greedy(self, token: int, pos: int):
        v = C.c_float()
        idx = lib().or_forward_greedy(self.h, token, pos, C.byref(v))
        return int(idx), v.value

    def forward_logits(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.spec.vocab, np.float32)
        lib().or_forward_logits(self.h, token, pos, _p(out))
        return out

    def final_normed(self) -> np.ndarray:
        p = lib().or_model_final_normed(self.h)
        return np.ctypeslib.as_array(p, shape=(self.spec.hidden,)).copy()

    def generate(self, prompt, n_gen: int) -> np.ndarray:
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(n_gen, np.uint32)
        lib().or_generate_greedy(self.h, _p(prompt), prompt.size, n_gen, _p(out))
        return out
