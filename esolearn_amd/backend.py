"""HipBackend: the MathBackend / DeviceBackend methods of the int8 Llama path
(crates/scry-llm/src/backend/mod.rs) over the scry_hip C ABI.

Names and argument meaning follow the reference trait: static methods, owned
storage returned by every op, errors raised (the reference panics).  Storage
lives on the GPU; ``to_vec`` copies back to numpy.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import call, load


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).ravel()


class Storage:
    """Device f32 storage (DeviceBackend::Storage)."""

    __slots__ = ("h", "n")

    def __init__(self, handle: int, n: int):
        self.h = handle
        self.n = n

    def to_vec(self) -> np.ndarray:
        out = np.empty(self.n, np.float32)
        call("scry_hip_to_vec", self.h, out.ctypes.data, self.n)
        return out

    def free(self) -> None:
        if self.h:
            load().scry_hip_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class I8Storage:
    """Device int8 weight storage (DeviceBackend::I8Storage)."""

    __slots__ = ("h", "n")

    def __init__(self, handle: int, n: int):
        self.h = handle
        self.n = n

    def to_vec(self) -> np.ndarray:
        out = np.empty(self.n, np.int8)
        call("scry_hip_i8_to_vec", self.h, out.ctypes.data, self.n)
        return out

    def free(self) -> None:
        if self.h:
            load().scry_hip_i8_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _out():
    return C.c_void_p()


def _st(h: C.c_void_p, n: int) -> Storage:
    return Storage(h.value, n)


class HipBackend:
    """Static-method backend, mirroring the reference trait surface."""

    # ---- runtime (cuda.rs:39-52 init_gpu, 1193-1197 synchronize)
    @staticmethod
    def init_gpu(device: int = 0) -> None:
        call("scry_hip_init", device)

    @staticmethod
    def synchronize() -> None:
        call("scry_hip_synchronize")

    @staticmethod
    def device_info() -> dict:
        name = C.create_string_buffer(256)
        arch = C.create_string_buffer(64)
        cu = C.c_int()
        call("scry_hip_device_info", name, 256, C.byref(cu), arch, 64)
        return {"name": name.value.decode(), "arch": arch.value.decode(), "cu_count": cu.value}

    # ---- DeviceBackend
    @staticmethod
    def zeros(n: int) -> Storage:
        o = _out()
        call("scry_hip_zeros", n, C.byref(o))
        return _st(o, n)

    @staticmethod
    def from_vec(data) -> Storage:
        a = _f32(data)
        o = _out()
        call("scry_hip_from_vec", a.ctypes.data, a.size, C.byref(o))
        return _st(o, a.size)

    @staticmethod
    def init_gpu_bf16(device: int = 0) -> None:
        """init_gpu_bf16 (cuda.rs:55-59): init, then bf16 mode."""
        call("scry_hip_init_bf16", device)

    @staticmethod
    def set_bf16_mode(on: bool) -> None:
        call("scry_hip_set_bf16_mode", int(bool(on)))

    @staticmethod
    def bf16_mode() -> bool:
        v = C.c_int()
        call("scry_hip_bf16_mode", C.byref(v))
        return bool(v.value)

    @staticmethod
    def from_vec_with_bf16(data, bf16_bytes) -> Storage:
        """DeviceBackend::from_vec_with_bf16 (mod.rs:28-32): bf16_bytes are the
        little-endian bf16 words of the same values (uint16 array or bytes)."""
        a = _f32(data)
        h = np.frombuffer(bytes(bf16_bytes), np.uint16) if isinstance(bf16_bytes, (bytes, bytearray)) \
            else np.ascontiguousarray(bf16_bytes, np.uint16).ravel()
        if h.size != a.size:
            raise ValueError("from_vec_with_bf16: bf16 data and f32 data differ in length")
        o = _out()
        call("scry_hip_from_vec_with_bf16", a.ctypes.data, h.ctypes.data, a.size, C.byref(o))
        return _st(o, a.size)

    @staticmethod
    def to_vec(s: Storage) -> np.ndarray:
        return s.to_vec()

    @staticmethod
    def clone_storage(s: Storage) -> Storage:
        o = _out()
        call("scry_hip_clone_storage", s.h, C.byref(o))
        return _st(o, s.n)

    @staticmethod
    def i8_from_vec(data) -> I8Storage:
        a = np.ascontiguousarray(data, dtype=np.int8).ravel()
        o = _out()
        call("scry_hip_i8_from_vec", a.ctypes.data, a.size, C.byref(o))
        return I8Storage(o.value, a.size)

    @staticmethod
    def i8_to_vec(s: I8Storage) -> np.ndarray:
        return s.to_vec()

    # ---- quantize.rs on the device
    @staticmethod
    def quantize_symmetric(w: Storage) -> tuple[I8Storage, float]:
        o = _out()
        s = C.c_float()
        call("scry_hip_quantize_symmetric", w.h, C.byref(o), C.byref(s))
        return I8Storage(o.value, w.n), np.float32(s.value)

    @staticmethod
    def dequantize(q: I8Storage, scale: float) -> Storage:
        o = _out()
        call("scry_hip_dequantize", q.h, float(scale), C.byref(o))
        return _st(o, q.n)

    @staticmethod
    def quantize_block32(w: Storage, k: int, n: int) -> tuple[I8Storage, Storage]:
        q, s = _out(), _out()
        call("scry_hip_quantize_block32", w.h, k, n, C.byref(q), C.byref(s))
        return I8Storage(q.value, w.n), _st(s, n * ((k + 31) // 32))

    # ---- MathBackend int8 (mod.rs:520-557)
    @staticmethod
    def matmul_i8_f32(a: Storage, b_q: I8Storage, scale: float, m: int, k: int, n: int) -> Storage:
        o = _out()
        call("scry_hip_matmul_i8_f32", a.h, b_q.h, float(scale), m, k, n, C.byref(o))
        return _st(o, m * n)

    @staticmethod
    def matmul_i8_f32_bias(a, b_q, scale, bias: Storage, m, k, n) -> Storage:
        o = _out()
        call("scry_hip_matmul_i8_f32_bias", a.h, b_q.h, float(scale), bias.h, m, k, n, C.byref(o))
        return _st(o, m * n)

    @staticmethod
    def matmul_i8_f32_block32(a, b_q, scales: Storage, m, k, n) -> Storage:
        o = _out()
        call("scry_hip_matmul_i8_f32_block32", a.h, b_q.h, scales.h, m, k, n, C.byref(o))
        return _st(o, m * n)

    # ---- MathBackend glue
    @staticmethod
    def matmul(a, b, m, k, n, trans_a=False, trans_b=False) -> Storage:
        o = _out()
        call("scry_hip_matmul", a.h, b.h, m, k, n, int(trans_a), int(trans_b), C.byref(o))
        return _st(o, m * n)

    @staticmethod
    def matmul_bias(a, b, bias, m, k, n, trans_a=False, trans_b=False) -> Storage:
        """C = A @ B + bias, the bias row [n] added to every row (mod.rs:62-86)."""
        o = _out()
        call("scry_hip_matmul_bias", a.h, b.h, bias.h, m, k, n, int(trans_a), int(trans_b),
             C.byref(o))
        return _st(o, m * n)

    @staticmethod
    def matmul_strided_batched(a, b, batch, m, k, n, trans_a=False, trans_b=False) -> Storage:
        o = _out()
        call("scry_hip_matmul_strided_batched", a.h, b.h, batch, m, k, n, int(trans_a),
             int(trans_b), C.byref(o))
        return _st(o, batch * m * n)

    @staticmethod
    def rmsnorm(x, w, rows, d, eps=1e-5) -> Storage:
        o = _out()
        call("scry_hip_rmsnorm", x.h, w.h, rows, d, float(eps), C.byref(o))
        return _st(o, rows * d)

    @staticmethod
    def rope_with_freqs_preloaded(x, seq, n_heads, head_dim, start_pos, freqs) -> Storage:
        o = _out()
        call("scry_hip_rope_with_freqs_preloaded", x.h, seq, n_heads, head_dim, start_pos,
             freqs.h, C.byref(o))
        return _st(o, x.n)

    @staticmethod
    def rope_with_freqs_scaled_preloaded(x, seq, n_heads, head_dim, start_pos, freqs,
                                         scale) -> Storage:
        o = _out()
        call("scry_hip_rope_with_freqs_scaled_preloaded", x.h, seq, n_heads, head_dim,
             start_pos, freqs.h, float(scale), C.byref(o))
        return _st(o, x.n)

    @staticmethod
    def scale(x, s) -> Storage:
        o = _out()
        call("scry_hip_scale", x.h, float(s), C.byref(o))
        return _st(o, x.n)

    @staticmethod
    def softmax(x, rows, cols) -> Storage:
        o = _out()
        call("scry_hip_softmax", x.h, rows, cols, C.byref(o))
        return _st(o, rows * cols)

    @staticmethod
    def swiglu(gate, up) -> Storage:
        o = _out()
        call("scry_hip_swiglu", gate.h, up.h, C.byref(o))
        return _st(o, gate.n)

    @staticmethod
    def add(a, b) -> Storage:
        o = _out()
        call("scry_hip_add", a.h, b.h, C.byref(o))
        return _st(o, a.n)

    @staticmethod
    def embedding(weight, ids, vocab, dim) -> Storage:
        idx = np.ascontiguousarray(ids, dtype=np.int64).ravel()
        o = _out()
        call("scry_hip_embedding", weight.h, idx.ctypes.data, idx.size, vocab, dim, C.byref(o))
        return _st(o, idx.size * dim)

    @staticmethod
    def gather_reshape_repeat_kv(cache, max_seq, cached_len, n_kv, n_q, head_dim) -> Storage:
        o = _out()
        call("scry_hip_gather_reshape_repeat_kv", cache.h, max_seq, cached_len, n_kv, n_q,
             head_dim, C.byref(o))
        return _st(o, n_q * cached_len * head_dim)

    @staticmethod
    def repeat_kv(x, n_kv, n_q, seq, d_head) -> Storage:
        o = _out()
        call("scry_hip_repeat_kv", x.h, n_kv, n_q, seq, d_head, C.byref(o))
        return _st(o, n_q * seq * d_head)

    @staticmethod
    def scatter_rows(dst, src, total_rows, cols, row_start, row_count) -> None:
        call("scry_hip_scatter_rows", dst.h, src.h, total_rows, cols, row_start, row_count)

    @staticmethod
    def argmax(logits: Storage) -> int:
        out = C.c_int64()
        call("scry_hip_argmax", logits.h, C.byref(out))
        return int(out.value)

    @staticmethod
    def sample_token(logits: Storage, config, rng) -> int:
        """sample_token (generate.rs:92-186) on the device: config is a
        SamplingConfig, rng an Rng whose state advances by the draw."""
        sc = _lib.SamplingConfigC(float(config.temperature), int(config.top_k),
                                  float(config.top_p), int(config.max_tokens))
        st = C.c_uint64(rng.state)
        out = C.c_int64()
        call("scry_hip_sample_token", logits.h, C.byref(sc), C.byref(st), C.byref(out))
        rng.state = int(st.value)
        return int(out.value)

    @staticmethod
    def sample_token_noalloc(logits: Storage, config, rng) -> int:
        """sample_token with no device allocation (a static scratch array per
        GPU, vocabularies up to 262144): same result and rng advance."""
        sc = _lib.SamplingConfigC(float(config.temperature), int(config.top_k),
                                  float(config.top_p), int(config.max_tokens))
        st = C.c_uint64(rng.state)
        out = C.c_int64()
        call("scry_hip_sample_token_noalloc", logits.h, C.byref(sc), C.byref(st), C.byref(out))
        rng.state = int(st.value)
        return int(out.value)

    # ---- the rest of the trait surface (mod.rs; CPU semantics cpu.rs)
    @staticmethod
    def ones(n: int) -> Storage:
        o = _out()
        call("scry_hip_ones", n, C.byref(o))
        return _st(o, n)

    @staticmethod
    def add_shapes(a, a_shape, b, b_shape, out_shape) -> Storage:
        """MathBackend::add with broadcasting (shapes as tuples)."""
        dims = [(C.c_size_t * len(d))(*d) for d in (a_shape, b_shape, out_shape)]
        o = _out()
        call("scry_hip_add_broadcast", a.h, dims[0], len(a_shape), b.h, dims[1], len(b_shape),
             dims[2], len(out_shape), C.byref(o))
        return _st(o, int(np.prod(out_shape)))

    @staticmethod
    def add_inplace(dst, src) -> None:
        call("scry_hip_add_inplace", dst.h, src.h)

    @staticmethod
    def scaled_softmax(x, scale, rows, cols) -> Storage:
        o = _out()
        call("scry_hip_scaled_softmax", x.h, scale, rows, cols, C.byref(o))
        return _st(o, x.n)

    @staticmethod
    def layernorm(x, gamma, beta, rows, d, eps=1e-5):
        """Returns (output, mean [rows], rstd [rows])."""
        o, mu, rs = _out(), _out(), _out()
        call("scry_hip_layernorm", x.h, gamma.h, beta.h, rows, d, eps, C.byref(o), C.byref(mu),
             C.byref(rs))
        return _st(o, x.n), _st(mu, rows), _st(rs, rows)

    @staticmethod
    def layernorm_inference(x, gamma, beta, rows, d, eps=1e-5) -> Storage:
        o = _out()
        call("scry_hip_layernorm_inference", x.h, gamma.h, beta.h, rows, d, eps, C.byref(o))
        return _st(o, x.n)

    @staticmethod
    def gelu(x) -> Storage:
        o = _out()
        call("scry_hip_gelu", x.h, C.byref(o))
        return _st(o, x.n)

    @staticmethod
    def sum(x) -> float:
        out = C.c_float()
        call("scry_hip_sum", x.h, C.byref(out))
        return float(np.float32(out.value))

    @staticmethod
    def mul_elementwise(a, b) -> Storage:
        o = _out()
        call("scry_hip_mul_elementwise", a.h, b.h, C.byref(o))
        return _st(o, min(a.n, b.n))

    @staticmethod
    def concat_rows(a, b, a_rows, b_rows, cols) -> Storage:
        o = _out()
        call("scry_hip_concat_rows", a.h, b.h, a_rows, b_rows, cols, C.byref(o))
        return _st(o, a.n + b.n)

    @staticmethod
    def rope(x, rows, last_dim, pos, head_dim, theta) -> Storage:
        """MathBackend::rope on rows of last_dim values (the shape's last axis)."""
        o = _out()
        call("scry_hip_rope", x.h, rows, last_dim, pos, head_dim, theta, C.byref(o))
        return _st(o, x.n)

    @staticmethod
    def gather_columns(x, rows, total_cols, col_start, col_count) -> Storage:
        o = _out()
        call("scry_hip_gather_columns", x.h, rows, total_cols, col_start, col_count, C.byref(o))
        return _st(o, rows * col_count)

    @staticmethod
    def scatter_columns(dst, src, rows, total_cols, col_start, col_count) -> None:
        call("scry_hip_scatter_columns", dst.h, src.h, rows, total_cols, col_start, col_count)

    @staticmethod
    def gather_rows(x, total_rows, cols, row_start, row_count) -> Storage:
        o = _out()
        call("scry_hip_gather_rows", x.h, total_rows, cols, row_start, row_count, C.byref(o))
        return _st(o, row_count * cols)

    @staticmethod
    def apply_causal_mask_and_scale(scores, seq, scale, mask_value) -> None:
        call("scry_hip_apply_causal_mask_and_scale", scores.h, seq, scale, mask_value)

    @staticmethod
    def apply_batched_causal_mask_and_scale(scores, num_matrices, seq, scale, mask_value) -> None:
        call("scry_hip_apply_batched_causal_mask_and_scale", scores.h, num_matrices, seq, scale,
             mask_value)

    @staticmethod
    def split_qkv_reshape_heads(qkv, seq, n_heads, d_head):
        q, k, v = _out(), _out(), _out()
        call("scry_hip_split_qkv_reshape_heads", qkv.h, seq, n_heads, d_head, C.byref(q),
             C.byref(k), C.byref(v))
        n = seq * n_heads * d_head
        return _st(q, n), _st(k, n), _st(v, n)

    @staticmethod
    def reshape_for_heads(x, batch, seq, n_heads, d_head) -> Storage:
        o = _out()
        call("scry_hip_reshape_for_heads", x.h, batch, seq, n_heads, d_head, C.byref(o))
        return _st(o, batch * seq * n_heads * d_head)

    @staticmethod
    def reshape_from_heads(x, batch, seq, n_heads, d_head) -> Storage:
        o = _out()
        call("scry_hip_reshape_from_heads", x.h, batch, seq, n_heads, d_head, C.byref(o))
        return _st(o, batch * seq * n_heads * d_head)


def init(device: int = 0) -> None:
    HipBackend.init_gpu(device)


__all__ = ["HipBackend", "Storage", "I8Storage", "init", "_lib"]
