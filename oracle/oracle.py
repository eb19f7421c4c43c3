"""ctypes wrapper for the CPU oracle (oracle/oracle.c) -- TEST INFRASTRUCTURE.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this module, and only as the checker / CPU baseline.  The product
(``esolearn_amd``) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass, fields

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "liboracle.so")
_lib = None

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
u64p = np.ctypeslib.ndpointer(dtype=np.uint64, flags="C_CONTIGUOUS")
szp = np.ctypeslib.ndpointer(dtype=np.uintp, flags="C_CONTIGUOUS")


def build() -> str:
    subprocess.run(["bash", os.path.join(_HERE, "build.sh")], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = C.CDLL(_LIB_PATH)
    sz, i32, u64, f32, f64 = C.c_size_t, C.c_int, C.c_uint64, C.c_float, C.c_double
    vp = C.c_void_p
    sig = {
        "orc_rng_u64_at": (u64, [u64, u64]),
        "orc_rng_fill_u64": (None, [u64, u64, sz, u64p]),
        "orc_rng_fill_f64": (None, [u64, u64, sz, f64p]),
        "orc_normal_vec": (None, [u64, u64, sz, f32, f32, f32p]),
        "orc_normal_vec_par": (None, [u64, u64, sz, f32, f32, f32p]),
        "orc_quantize_symmetric": (None, [f32p, sz, i8p, C.POINTER(C.c_float)]),
        "orc_dequantize": (None, [i8p, sz, f32, f32p]),
        "orc_quantize_block32": (None, [f32p, i32, i32, i8p, f32p]),
        "orc_matmul_i8_f32_tiled": (None, [f32p, i8p, f32, i32, i32, i32, f32p]),
        "orc_matmul_i8_f32_par": (None, [f32p, i8p, f32, i32, i32, i32, f32p]),
        "orc_matmul_i8_f32_tb": (None, [f32p, i8p, f32, i32, i32, i32, f32p]),
        "orc_matmul_i8_f32_b32": (None, [f32p, i8p, f32p, i32, i32, i32, f32p]),
        "orc_matmul_i8_f32_bias": (None, [f32p, i8p, f32, f32p, i32, i32, i32, f32p]),
        "orc_gemv_f32": (None, [f32p, f32p, i32, i32, f32p]),
        "orc_gemv_trans_b": (None, [f32p, f32p, i32, i32, f32p]),
        "orc_gemv_into": (None, [f32p, f32p, i32, i32, f32p]),
        "orc_matmul_f32": (None, [f32p, f32p, i32, i32, i32, i32, i32, f32p]),
        "orc_f32_to_bf16_vec": (None, [f32p, sz, C.c_void_p]),
        "orc_matmul_bf16": (None, [f32p, f32p, i32, i32, i32, i32, i32, f32p]),
        "orc_matmul_bf16_par": (None, [f32p, f32p, i32, i32, i32, i32, f32p]),
        "orc_matmul_strided_batched": (None, [f32p, f32p, i32, i32, i32, i32, i32, i32, f32p]),
        "orc_rmsnorm": (None, [f32p, f32p, i32, i32, f32, f32p]),
        "orc_rope_with_freqs_preloaded": (None, [f32p, i32, i32, i32, i32, f32p, f32p]),
        "orc_scale": (None, [f32p, sz, f32, f32p]),
        "orc_softmax": (None, [f32p, i32, i32, f32p]),
        "orc_silu": (f32, [f32]),
        "orc_swiglu": (None, [f32p, f32p, sz, f32p]),
        "orc_add": (None, [f32p, f32p, sz, f32p]),
        "orc_embedding": (i32, [f32p, i64p, i32, i32, i32, f32p]),
        "orc_repeat_kv": (None, [f32p, i32, i32, i32, i32, f32p]),
        "orc_gather_reshape_repeat_kv": (None, [f32p, i32, i32, i32, i32, i32, f32p]),
        "orc_scatter_rows": (None, [f32p, f32p, i32, i32, i32, i32]),
        "orc_causal_mask_scale": (None, [f32p, i32, i32, f32, f32]),
        "orc_argmax": (C.c_int64, [f32p, C.c_int64]),
        "orc_compute_rope_freqs": (None, [i32, f32, i32, f64, f64, f64, C.c_int64, f64p]),
        "orc_llama_new": (vp, [vp, u64, i32, i32, i32]),
        "orc_llama_free": (None, [vp]),
        "orc_llama_new_empty": (vp, [vp]),
        "orc_llama_set_qtensor": (i32, [vp, i32, i32, i8p, f32]),
        "orc_llama_set_qtensor_b32": (C.c_int, [C.c_void_p, i32, i32, i8p, f32p]),
        "orc_llama_set_embed": (i32, [vp, f32p]),
        "orc_llama_set_norm": (i32, [vp, i32, i32, f32p, f32]),
        "orc_llama_rng_calls": (u64, [vp]),
        "orc_llama_tensor": (sz, [vp, i32, i32, vp]),
        "orc_llama_qtensor": (sz, [vp, i32, i32, vp, C.POINTER(C.c_float)]),
        "orc_llama_qscales_b32": (sz, [vp, i32, i32, vp]),
        "orc_cache_new": (vp, [vp, i32]),
        "orc_cache_free": (None, [vp]),
        "orc_cache_len": (i32, [vp, i32]),
        "orc_cache_layer": (None, [vp, i32, vp, vp]),
        "orc_llama_forward_with_cache": (i32, [vp, vp, C.c_int64, i32, i32, f32p]),
        "orc_llama_forward": (i32, [vp, i64p, i32, i32, f32p]),
        "orc_generate_greedy": (i32, [vp, i64p, i32, i32, i32, i64p, vp]),
        "orc_generate_greedy_fast": (i32, [vp, i64p, i32, i32, i64p, vp]),
        "orc_llama_forward_cache_seq": (i32, [vp, vp, i64p, i32, i32, i32, vp]),
        "orc_generate": (i32, [vp, i64p, i32, i32, f32, C.c_int64, f32, u64, i32, i64p, vp]),
        "orc_sample_token": (C.c_int64, [f32p, C.c_int64, f32, C.c_int64, f32, C.POINTER(u64)]),
        "orc_layernorm": (None, [f32p, f32p, f32p, i32, i32, f32, f32p, vp, vp]),
        "orc_gelu": (f32, [f32]),
        "orc_gelu_vec": (None, [f32p, sz, f32p]),
        "orc_sum": (f32, [f32p, sz]),
        "orc_mul": (None, [f32p, f32p, sz, f32p]),
        "orc_rope_rows": (None, [f32p, sz, i32, i32, i32, f32, f32p]),
        "orc_gather_columns": (None, [f32p, i32, i32, i32, i32, f32p]),
        "orc_scatter_columns": (None, [f32p, f32p, i32, i32, i32, i32]),
        "orc_add_broadcast": (None, [f32p, szp, i32, f32p, szp, i32, szp, i32, f32p]),
        "orc_scaled_softmax": (None, [f32p, i32, i32, f32, f32p]),
        "orc_split_qkv_reshape_heads": (None, [f32p, i32, i32, i32, f32p, f32p, f32p]),
        "orc_reshape_heads": (None, [f32p, i32, i32, i32, i32, i32, f32p]),
        "orc_set_threads": (None, [i32]),
        "orc_get_threads": (i32, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


# ---- fastrand / init ----
def rng_f64(seed: int, start: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float64)
    lib().orc_rng_fill_f64(seed, start, n, out)
    return out


def rng_u64(seed: int, start: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    lib().orc_rng_fill_u64(seed, start, n, out)
    return out


def normal_vec(seed: int, start: int, n: int, mean=0.0, std=0.02, par=False) -> np.ndarray:
    out = np.empty(n, np.float32)
    fn = lib().orc_normal_vec_par if par else lib().orc_normal_vec
    fn(seed, start, n, mean, std, out)
    return out


def prompt_ids(seed: int, n: int, vocab: int) -> np.ndarray:
    """Build-defined prompt: n draws of Rng::with_seed(seed).u64() % vocab."""
    return (rng_u64(seed, 0, n) % np.uint64(vocab)).astype(np.int64)


# ---- quantize ----
def quantize_symmetric(w):
    w = _f32(w).ravel()
    q = np.empty(w.size, np.int8)
    s = C.c_float()
    lib().orc_quantize_symmetric(w, w.size, q, C.byref(s))
    return q, np.float32(s.value)


def dequantize(q, scale):
    q = np.ascontiguousarray(q, np.int8).ravel()
    out = np.empty(q.size, np.float32)
    lib().orc_dequantize(q, q.size, float(scale), out)
    return out


def quantize_block32(w, k, n):
    w = _f32(w).ravel()
    q = np.empty(k * n, np.int8)
    s = np.empty(n * ((k + 31) // 32), np.float32)
    lib().orc_quantize_block32(w, k, n, q, s)
    return q, s


# ---- matmuls ----
def matmul_i8_f32(a, bq, scale, m, k, n, faithful=False):
    c = np.empty(m * n, np.float32)
    fn = lib().orc_matmul_i8_f32_tiled if faithful else lib().orc_matmul_i8_f32_par
    fn(_f32(a).ravel(), np.ascontiguousarray(bq, np.int8).ravel(), float(scale), m, k, n, c)
    return c.reshape(m, n)


def matmul_i8_f32_tb(a, bq_nk, scale, m, k, n):
    c = np.empty(m * n, np.float32)
    lib().orc_matmul_i8_f32_tb(_f32(a).ravel(), np.ascontiguousarray(bq_nk, np.int8).ravel(),
                               float(scale), m, k, n, c)
    return c.reshape(m, n)


def matmul_i8_f32_b32(a, bq, scales, m, k, n):
    c = np.empty(m * n, np.float32)
    lib().orc_matmul_i8_f32_b32(_f32(a).ravel(), np.ascontiguousarray(bq, np.int8).ravel(),
                                _f32(scales).ravel(), m, k, n, c)
    return c.reshape(m, n)


def matmul_i8_f32_bias(a, bq, scale, bias, m, k, n):
    c = np.empty(m * n, np.float32)
    lib().orc_matmul_i8_f32_bias(_f32(a).ravel(), np.ascontiguousarray(bq, np.int8).ravel(),
                                 float(scale), _f32(bias).ravel(), m, k, n, c)
    return c.reshape(m, n)


def matmul_f32(a, b, m, k, n, trans_a=False, trans_b=False):
    c = np.empty(m * n, np.float32)
    lib().orc_matmul_f32(_f32(a).ravel(), _f32(b).ravel(), m, k, n, int(trans_a), int(trans_b), c)
    return c.reshape(m, n)


def f32_to_bf16(x) -> np.ndarray:
    """kernels.rs:629-633 float_to_bf16 on every element (uint16 words)."""
    a = _f32(x).ravel()
    out = np.empty(a.size, np.uint16)
    lib().orc_f32_to_bf16_vec(a, a.size, out.ctypes.data)
    return out


def matmul_bf16(a, b, m, k, n, trans_a=False, trans_b=False):
    """bf16_ops::matmul_bf16 (cuda.rs:1226-1290): bf16 operands, exact
    products summed in f64 and rounded once."""
    c = np.empty(m * n, np.float32)
    lib().orc_matmul_bf16(_f32(a).ravel(), _f32(b).ravel(), m, k, n, int(trans_a), int(trans_b), c)
    return c.reshape(m, n)


def matmul_bf16_par(a, b, m, k, n, trans_b=False):
    """matmul_bf16 (trans_a = 0) on all cores: bit-identical."""
    c = np.empty(m * n, np.float32)
    lib().orc_matmul_bf16_par(_f32(a).ravel(), _f32(b).ravel(), m, k, n, int(trans_b), c)
    return c.reshape(m, n)


def gemv_f32(vec, mat, k, n):
    out = np.empty(n, np.float32)
    lib().orc_gemv_f32(_f32(vec), _f32(mat).ravel(), k, n, out)
    return out


def gemv_trans_b(vec, mat_t, k, n):
    out = np.empty(n, np.float32)
    lib().orc_gemv_trans_b(_f32(vec), _f32(mat_t).ravel(), k, n, out)
    return out


def gemv_into(vec, mat, k, n):
    out = np.empty(n, np.float32)
    lib().orc_gemv_into(_f32(vec), _f32(mat).ravel(), k, n, out)
    return out


def matmul_strided_batched(a, b, batch, m, k, n, trans_a=False, trans_b=False):
    c = np.empty(batch * m * n, np.float32)
    lib().orc_matmul_strided_batched(_f32(a).ravel(), _f32(b).ravel(), batch, m, k, n,
                                     int(trans_a), int(trans_b), c)
    return c


# ---- glue ----
def rmsnorm(x, w, rows, d, eps=1e-5):
    out = np.empty(rows * d, np.float32)
    lib().orc_rmsnorm(_f32(x).ravel(), _f32(w).ravel(), rows, d, eps, out)
    return out


def rope_with_freqs_preloaded(x, seq, n_heads, head_dim, start_pos, freqs):
    out = np.empty(seq * n_heads * head_dim, np.float32)
    lib().orc_rope_with_freqs_preloaded(_f32(x).ravel(), seq, n_heads, head_dim, start_pos,
                                        _f32(freqs), out)
    return out


def scale(x, s):
    x = _f32(x).ravel()
    out = np.empty_like(x)
    lib().orc_scale(x, x.size, s, out)
    return out


def softmax(x, rows, cols):
    out = np.empty(rows * cols, np.float32)
    lib().orc_softmax(_f32(x).ravel(), rows, cols, out)
    return out


def silu(x: float) -> float:
    return lib().orc_silu(x)


def swiglu(g, u):
    g = _f32(g).ravel()
    out = np.empty_like(g)
    lib().orc_swiglu(g, _f32(u).ravel(), g.size, out)
    return out


def add(a, b):
    a = _f32(a).ravel()
    out = np.empty_like(a)
    lib().orc_add(a, _f32(b).ravel(), a.size, out)
    return out


def embedding(weight, idx, vocab, dim):
    idx = np.ascontiguousarray(idx, np.int64)
    out = np.empty(idx.size * dim, np.float32)
    rc = lib().orc_embedding(_f32(weight).ravel(), idx, idx.size, vocab, dim, out)
    if rc != 0:
        raise IndexError("embedding index out of range")
    return out


def repeat_kv(x, n_kv, n_q, seq, d_head):
    out = np.empty(n_q * seq * d_head, np.float32)
    lib().orc_repeat_kv(_f32(x).ravel(), n_kv, n_q, seq, d_head, out)
    return out


def gather_reshape_repeat_kv(cache, max_seq, cached_len, n_kv, n_q, head_dim):
    out = np.empty(n_q * cached_len * head_dim, np.float32)
    lib().orc_gather_reshape_repeat_kv(_f32(cache).ravel(), max_seq, cached_len, n_kv, n_q,
                                       head_dim, out)
    return out


def causal_mask_scale(scores, n_mat, seq, scale_, mask_value):
    s = _f32(scores).ravel().copy()
    lib().orc_causal_mask_scale(s, n_mat, seq, scale_, mask_value)
    return s


def sample_token(logits, temperature, top_k, top_p, rng_state: int):
    """generate.rs:92-165; returns (token, the rng state after the call)."""
    st = C.c_uint64(rng_state)
    tok = lib().orc_sample_token(_f32(logits), len(logits), float(temperature), int(top_k),
                                 float(top_p), C.byref(st))
    return int(tok), int(st.value)


def argmax(logits) -> int:
    x = _f32(logits).ravel()
    return int(lib().orc_argmax(x, x.size))


def compute_rope_freqs(head_dim, theta, scaling=None):
    out = np.empty(head_dim // 2, np.float64)
    if scaling is None:
        lib().orc_compute_rope_freqs(head_dim, theta, 0, 0.0, 0.0, 0.0, 0, out)
    else:
        f, lo, hi, orig = scaling
        lib().orc_compute_rope_freqs(head_dim, theta, 1, f, lo, hi, orig, out)
    return out


# ---- the rest of the trait surface ----
def layernorm(x, gamma, beta, rows, d, eps=1e-5):
    """cpu.rs:416-475: (out [rows*d], mean [rows], rstd [rows])"""
    out = np.empty(rows * d, np.float32)
    mu = np.empty(rows, np.float32)
    rs = np.empty(rows, np.float32)
    lib().orc_layernorm(_f32(x).ravel(), _f32(gamma).ravel(), _f32(beta).ravel(), rows, d, eps, out,
                        mu.ctypes.data, rs.ctypes.data)
    return out, mu, rs


def gelu(x):
    x = _f32(x).ravel()
    out = np.empty_like(x)
    lib().orc_gelu_vec(x, x.size, out)
    return out


def sum_(x) -> float:
    x = _f32(x).ravel()
    return float(np.float32(lib().orc_sum(x, x.size)))


def mul_elementwise(a, b):
    a, b = _f32(a).ravel(), _f32(b).ravel()
    n = min(a.size, b.size)
    out = np.empty(n, np.float32)
    lib().orc_mul(a, b, n, out)
    return out


def rope(x, rows, last_dim, pos, head_dim, theta):
    out = np.empty(rows * last_dim, np.float32)
    lib().orc_rope_rows(_f32(x).ravel(), rows, last_dim, pos, head_dim, theta, out)
    return out


def gather_columns(x, rows, total, start, count):
    out = np.empty(rows * count, np.float32)
    lib().orc_gather_columns(_f32(x).ravel(), rows, total, start, count, out)
    return out


def scatter_columns(dst, src, rows, total, start, count):
    d = _f32(dst).ravel().copy()
    lib().orc_scatter_columns(d, _f32(src).ravel(), rows, total, start, count)
    return d


def add_broadcast(a, a_dims, b, b_dims, out_dims):
    ad, bd, od = (np.asarray(v, np.uintp) for v in (a_dims, b_dims, out_dims))
    out = np.empty(int(np.prod(od)), np.float32)
    lib().orc_add_broadcast(_f32(a).ravel(), ad, ad.size, _f32(b).ravel(), bd, bd.size, od, od.size, out)
    return out


def scaled_softmax(x, rows, cols, scale_):
    out = np.empty(rows * cols, np.float32)
    lib().orc_scaled_softmax(_f32(x).ravel(), rows, cols, scale_, out)
    return out


def split_qkv_reshape_heads(qkv, seq, n_heads, d_head):
    n = seq * n_heads * d_head
    q, k, v = (np.empty(n, np.float32) for _ in range(3))
    lib().orc_split_qkv_reshape_heads(_f32(qkv).ravel(), seq, n_heads, d_head, q, k, v)
    return q, k, v


def reshape_for_heads(x, batch, seq, n_heads, d_head):
    out = np.empty(batch * seq * n_heads * d_head, np.float32)
    lib().orc_reshape_heads(_f32(x).ravel(), batch, seq, n_heads, d_head, 0, out)
    return out


def reshape_from_heads(x, batch, seq, n_heads, d_head):
    out = np.empty(batch * seq * n_heads * d_head, np.float32)
    lib().orc_reshape_heads(_f32(x).ravel(), batch, seq, n_heads, d_head, 1, out)
    return out


# ---- model ----
class _Cfg(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_int32), ("hidden_size", C.c_int32),
        ("intermediate_size", C.c_int32), ("n_layers", C.c_int32), ("n_heads", C.c_int32),
        ("n_kv_heads", C.c_int32), ("max_seq_len", C.c_int32), ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_float), ("tie_word_embeddings", C.c_int32),
        ("has_rope_scaling", C.c_int32), ("rs_factor", C.c_double),
        ("rs_low_freq_factor", C.c_double), ("rs_high_freq_factor", C.c_double),
        ("rs_original_max_pos", C.c_int64),
    ]


@dataclass
class LlamaConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    max_seq_len: int = 2048
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    tie_word_embeddings: bool = True
    rope_scaling: tuple | None = None  # (factor, low, high, original_max_pos)

    def to_c(self) -> _Cfg:
        c = _Cfg()
        for f in fields(self):
            if f.name == "rope_scaling":
                continue
            setattr(c, f.name, getattr(self, f.name))
        if self.rope_scaling is not None:
            c.has_rope_scaling = 1
            (c.rs_factor, c.rs_low_freq_factor, c.rs_high_freq_factor,
             c.rs_original_max_pos) = self.rope_scaling
        return c

    @property
    def head_dim(self):
        return self.hidden_size // self.n_heads


T_EMBED, T_QKV, T_O, T_GATE, T_UP, T_DOWN, T_LM_HEAD, T_ROPE_FREQS = range(8)


class Llama:
    """Oracle Llama (llama.rs:593-680) with the int8 composition."""

    def __init__(self, cfg: LlamaConfig, seed: int | None, quantize=True, keep_f32=True,
                 block32=False):
        """seed None: an empty int8 model to be filled with set_qtensor/set_embed."""
        self.cfg = cfg
        self._c = cfg.to_c()
        if seed is None:
            self.h = lib().orc_llama_new_empty(C.byref(self._c))
        else:
            self.h = lib().orc_llama_new(C.byref(self._c), seed, int(quantize), int(keep_f32),
                                         int(block32))
        if not self.h:
            raise MemoryError("orc_llama_new failed")

    def set_qtensor(self, tid, layer, q, scale):
        q = np.ascontiguousarray(q, np.int8).ravel()
        if lib().orc_llama_set_qtensor(self.h, tid, layer, q, float(scale)) != 0:
            raise ValueError("set_qtensor: bad tensor")

    def set_qtensor_b32(self, tid, layer, q32, s32):
        """Block-32 weights (forward mode 2): q32 in the projection's layout."""
        q = np.ascontiguousarray(q32, np.int8).ravel()
        if lib().orc_llama_set_qtensor_b32(self.h, tid, layer, q, _f32(s32).ravel()) != 0:
            raise ValueError("set_qtensor_b32: bad tensor")

    def set_embed(self, w):
        lib().orc_llama_set_embed(self.h, _f32(w).ravel())

    def set_norm(self, which, layer, w, eps):
        """which: 0 input / 1 post-attention norm of `layer`, 2 the final norm."""
        if lib().orc_llama_set_norm(self.h, which, layer, _f32(w).ravel(), float(eps)) != 0:
            raise ValueError("set_norm: bad norm")

    def close(self):
        if self.h:
            lib().orc_llama_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def rng_calls(self) -> int:
        return int(lib().orc_llama_rng_calls(self.h))

    def tensor(self, tid, layer=0) -> np.ndarray:
        n = lib().orc_llama_tensor(self.h, tid, layer, None)
        out = np.empty(n, np.float32)
        lib().orc_llama_tensor(self.h, tid, layer, out.ctypes.data)
        return out

    def qtensor(self, tid, layer=0):
        n = lib().orc_llama_qtensor(self.h, tid, layer, None, None)
        out = np.empty(n, np.int8)
        s = C.c_float()
        lib().orc_llama_qtensor(self.h, tid, layer, out.ctypes.data, C.byref(s))
        return out, np.float32(s.value)

    def qscales_b32(self, tid, layer=0):
        n = lib().orc_llama_qscales_b32(self.h, tid, layer, None)
        out = np.empty(n, np.float32)
        lib().orc_llama_qscales_b32(self.h, tid, layer, out.ctypes.data)
        return out

    def new_cache(self, max_seq):
        return _Cache(self, max_seq)

    def forward_with_cache(self, cache, token, pos, mode=1):
        out = np.empty(self.cfg.vocab_size, np.float32)
        rc = lib().orc_llama_forward_with_cache(self.h, cache.h, int(token), int(pos), mode, out)
        if rc != 0:
            raise RuntimeError(f"oracle forward_with_cache failed: {rc}")
        return out

    def forward(self, tokens, mode=1):
        t = np.ascontiguousarray(tokens, np.int64)
        out = np.empty(t.size * self.cfg.vocab_size, np.float32)
        rc = lib().orc_llama_forward(self.h, t, t.size, mode, out)
        if rc != 0:
            raise RuntimeError(f"oracle forward failed: {rc}")
        return out.reshape(t.size, self.cfg.vocab_size)

    def generate(self, prompt, max_tokens, temperature, top_k, top_p, seed, mode=1,
                 want_logits=False):
        """generate() (generate.rs:51-89) with sample_token and Rng::with_seed(seed)."""
        p = np.ascontiguousarray(prompt, np.int64)
        nout = max(1, max_tokens)
        toks = np.empty(nout, np.int64)
        lg = np.empty(nout * self.cfg.vocab_size, np.float32) if want_logits else None
        rc = lib().orc_generate(self.h, p, p.size, max_tokens, float(temperature), int(top_k),
                                float(top_p), int(seed), mode, toks,
                                lg.ctypes.data if lg is not None else None)
        if rc < 0:
            raise RuntimeError(f"oracle generate failed: {rc}")
        if want_logits:
            return toks[:rc], lg.reshape(nout, -1)[:rc]
        return toks[:rc]

    def generate_greedy(self, prompt, max_tokens, mode=1, want_logits=False):
        p = np.ascontiguousarray(prompt, np.int64)
        nout = max(1, max_tokens)
        toks = np.empty(nout, np.int64)
        lg = np.empty(nout * self.cfg.vocab_size, np.float32) if want_logits else None
        rc = lib().orc_generate_greedy(self.h, p, p.size, max_tokens, mode, toks,
                                       lg.ctypes.data if lg is not None else None)
        if rc < 0:
            raise RuntimeError(f"oracle generate failed: {rc}")
        if want_logits:
            return toks[:rc], lg.reshape(nout, -1)[:rc]
        return toks[:rc]


    def generate_greedy_fast(self, prompt, max_tokens, want_logits=False):
        """generate_greedy(mode=1) evaluated layer-major (orc_generate_greedy_fast):
        the same tokens and bit-identical step logits, with each int8 weight read
        once for the whole prompt."""
        p = np.ascontiguousarray(prompt, np.int64)
        nout = max(1, max_tokens)
        toks = np.empty(nout, np.int64)
        lg = np.empty(nout * self.cfg.vocab_size, np.float32) if want_logits else None
        rc = lib().orc_generate_greedy_fast(self.h, p, p.size, max_tokens, toks,
                                            lg.ctypes.data if lg is not None else None)
        if rc < 0:
            raise RuntimeError(f"oracle generate_greedy_fast failed: {rc}")
        if want_logits:
            return toks[:rc], lg.reshape(nout, -1)[:rc]
        return toks[:rc]

    def forward_cache_seq(self, cache, tokens, pos0, n_logits=1):
        """n tokens through the cache path at positions pos0.. (layer-major,
        bit-identical to forward_with_cache per token); logits of the last
        n_logits rows."""
        t = np.ascontiguousarray(tokens, np.int64)
        lg = np.empty(max(1, n_logits) * self.cfg.vocab_size, np.float32)
        rc = lib().orc_llama_forward_cache_seq(self.h, cache.h, t, t.size, int(pos0), int(n_logits),
                                               lg.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"oracle forward_cache_seq failed: {rc}")
        return lg.reshape(max(1, n_logits), -1)[:n_logits]


class _Cache:
    def __init__(self, model: Llama, max_seq: int):
        self.model = model
        self.max_seq = max_seq
        self.h = lib().orc_cache_new(model.h, max_seq)

    def __del__(self):
        try:
            if self.h:
                lib().orc_cache_free(self.h)
                self.h = None
        except Exception:
            pass

    def seq_len(self, layer=0):
        return int(lib().orc_cache_len(self.h, layer))

    def layer(self, layer):
        n = self.max_seq * self.model.cfg.n_kv_heads * self.model.cfg.head_dim
        k = np.empty(n, np.float32)
        v = np.empty(n, np.float32)
        lib().orc_cache_layer(self.h, layer, k.ctypes.data, v.ctypes.data)
        return k, v


# BASELINE.json configs
TINY = LlamaConfig(vocab_size=32000, hidden_size=288, intermediate_size=768, n_layers=6,
                   n_heads=6, n_kv_heads=6, max_seq_len=256, rope_theta=10000.0,
                   tie_word_embeddings=True)
LLAMA2_7B = LlamaConfig(vocab_size=32000, hidden_size=4096, intermediate_size=11008,
                        n_layers=32, n_heads=32, n_kv_heads=32, max_seq_len=2048,
                        rope_theta=10000.0, tie_word_embeddings=False)
LLAMA3_8B = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336,
                        n_layers=32, n_heads=32, n_kv_heads=8, max_seq_len=2048,
                        rope_theta=500000.0, tie_word_embeddings=False)
