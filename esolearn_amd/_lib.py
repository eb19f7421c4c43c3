"""ctypes binding of libscry_hip.so (the C ABI declared in include/scry_hip.h).

There is no fallback: if the library is missing or fails to load, every entry
point raises.  Non-zero status codes become ScryHipError, which is what the
reference's ops do when they fail (they panic).
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libscry_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "scry_hip.h")

SCRY_OK = 0
ERR_NAMES = {1: "INVALID", 2: "HIP", 3: "OOM", 4: "NOT_INIT", 5: "RANGE", 6: "UNSUPPORTED"}


class ScryHipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{ERR_NAMES.get(code, code)}] {msg}")
        self.code = code


class LlamaConfigC(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_int32), ("hidden_size", C.c_int32),
        ("intermediate_size", C.c_int32), ("n_layers", C.c_int32), ("n_heads", C.c_int32),
        ("n_kv_heads", C.c_int32), ("max_seq_len", C.c_int32), ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_float), ("tie_word_embeddings", C.c_int32),
        ("has_rope_scaling", C.c_int32), ("rs_factor", C.c_double),
        ("rs_low_freq_factor", C.c_double), ("rs_high_freq_factor", C.c_double),
        ("rs_original_max_pos", C.c_int64),
    ]


class SamplingConfigC(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float),
                ("max_tokens", C.c_int32)]


vp, sz, i32, i64, u64, f32, f64 = (C.c_void_p, C.c_size_t, C.c_int, C.c_int64, C.c_uint64,
                                   C.c_float, C.c_double)
P = C.POINTER

SIGNATURES = {
    "scry_hip_init": [i32],
    "scry_hip_shutdown": [],
    "scry_hip_last_error": [],
    "scry_hip_synchronize": [],
    "scry_hip_device_count": [P(i32)],
    "scry_hip_device_info": [C.c_char_p, sz, P(i32), C.c_char_p, sz],
    "scry_hip_zeros": [sz, P(vp)],
    "scry_hip_from_vec": [vp, sz, P(vp)],
    "scry_hip_to_vec": [vp, vp, sz],
    "scry_hip_clone_storage": [vp, P(vp)],
    "scry_hip_buf_len": [vp, P(sz)],
    "scry_hip_free": [vp],
    "scry_hip_i8_from_vec": [vp, sz, P(vp)],
    "scry_hip_i8_to_vec": [vp, vp, sz],
    "scry_hip_i8_len": [vp, P(sz)],
    "scry_hip_i8_free": [vp],
    "scry_hip_quantize_symmetric": [vp, P(vp), P(f32)],
    "scry_hip_dequantize": [vp, f32, P(vp)],
    "scry_hip_quantize_block32": [vp, i32, i32, P(vp), P(vp)],
    "scry_hip_matmul_i8_f32": [vp, vp, f32, i32, i32, i32, P(vp)],
    "scry_hip_matmul_i8_f32_bias": [vp, vp, f32, vp, i32, i32, i32, P(vp)],
    "scry_hip_matmul_i8_f32_block32": [vp, vp, vp, i32, i32, i32, P(vp)],
    "scry_hip_matmul": [vp, vp, i32, i32, i32, i32, i32, P(vp)],
    "scry_hip_matmul_bias": [vp, vp, vp, i32, i32, i32, i32, i32, P(vp)],
    "scry_hip_matmul_strided_batched": [vp, vp, i32, i32, i32, i32, i32, i32, P(vp)],
    "scry_hip_rmsnorm": [vp, vp, i32, i32, f32, P(vp)],
    "scry_hip_rope_with_freqs_preloaded": [vp, i32, i32, i32, i32, vp, P(vp)],
    "scry_hip_rope_with_freqs_scaled_preloaded": [vp, i32, i32, i32, i32, vp, f32, P(vp)],
    "scry_hip_scale": [vp, f32, P(vp)],
    "scry_hip_softmax": [vp, i32, i32, P(vp)],
    "scry_hip_swiglu": [vp, vp, P(vp)],
    "scry_hip_add": [vp, vp, P(vp)],
    "scry_hip_embedding": [vp, vp, i32, i32, i32, P(vp)],
    "scry_hip_gather_reshape_repeat_kv": [vp, i32, i32, i32, i32, i32, P(vp)],
    "scry_hip_repeat_kv": [vp, i32, i32, i32, i32, P(vp)],
    "scry_hip_scatter_rows": [vp, vp, i32, i32, i32, i32],
    "scry_hip_argmax": [vp, P(i64)],
    "scry_hip_sample_token": [vp, P(SamplingConfigC), P(u64), P(i64)],
    "scry_hip_sample_token_noalloc": [vp, P(SamplingConfigC), P(u64), P(i64)],
    "scry_hip_normal_vec": [P(u64), sz, f32, f32, P(vp)],
    "scry_hip_init_bf16": [i32],
    "scry_hip_set_bf16_mode": [i32],
    "scry_hip_bf16_mode": [P(i32)],
    "scry_hip_from_vec_with_bf16": [vp, vp, sz, P(vp)],
    "scry_hip_bench_qgemv_bias": [i32, i32, i32, i32, i32, i32, P(f64), P(f64)],
    "scry_hip_bench_gemv_bf16": [i32, i32, i32, i32, i32, i32, P(f64), P(f64)],
    "scry_hip_ones": [sz, P(vp)],
    "scry_hip_add_broadcast": [vp, P(sz), i32, vp, P(sz), i32, P(sz), i32, P(vp)],
    "scry_hip_add_inplace": [vp, vp],
    "scry_hip_scaled_softmax": [vp, f32, i32, i32, P(vp)],
    "scry_hip_layernorm": [vp, vp, vp, i32, i32, f32, P(vp), P(vp), P(vp)],
    "scry_hip_layernorm_inference": [vp, vp, vp, i32, i32, f32, P(vp)],
    "scry_hip_gelu": [vp, P(vp)],
    "scry_hip_sum": [vp, P(f32)],
    "scry_hip_mul_elementwise": [vp, vp, P(vp)],
    "scry_hip_concat_rows": [vp, vp, i32, i32, i32, P(vp)],
    "scry_hip_rope": [vp, sz, i32, i32, i32, f32, P(vp)],
    "scry_hip_gather_columns": [vp, i32, i32, i32, i32, P(vp)],
    "scry_hip_scatter_columns": [vp, vp, i32, i32, i32, i32],
    "scry_hip_gather_rows": [vp, i32, i32, i32, i32, P(vp)],
    "scry_hip_apply_causal_mask_and_scale": [vp, i32, f32, f32],
    "scry_hip_apply_batched_causal_mask_and_scale": [vp, i32, i32, f32, f32],
    "scry_hip_split_qkv_reshape_heads": [vp, i32, i32, i32, P(vp), P(vp), P(vp)],
    "scry_hip_reshape_for_heads": [vp, i32, i32, i32, i32, P(vp)],
    "scry_hip_reshape_from_heads": [vp, i32, i32, i32, i32, P(vp)],
    "scry_hip_llama_new_random": [P(LlamaConfigC), u64, i32, i32, P(vp)],
    "scry_hip_llama_from_safetensors": [P(LlamaConfigC), P(C.c_char_p), i32, i32, P(vp)],
    "scry_hip_llama_free": [vp],
    "scry_hip_llama_set_tensor": [vp, i32, i32, vp, sz],
    "scry_hip_llama_get_qtensor": [vp, i32, i32, vp, sz, P(f32)],
    "scry_hip_llama_get_embed": [vp, vp, sz],
    "scry_hip_llama_kv_cache_new": [vp, i32, P(vp)],
    "scry_hip_kv_cache_free": [vp],
    "scry_hip_kv_cache_seq_len": [vp, P(i32)],
    "scry_hip_kv_cache_layer_to_vec": [vp, i32, vp, vp, sz],
    "scry_hip_llama_forward_with_cache": [vp, vp, i64, i32, vp, P(i64)],
    "scry_hip_llama_generate_greedy": [vp, vp, i32, i32, vp, P(i32), vp],
    "scry_hip_llama_generate_greedy_prefill": [vp, vp, i32, i32, vp, P(i32), vp],
    "scry_hip_llama_generate": [vp, vp, i32, P(SamplingConfigC), P(u64), i32, vp, P(i32), vp],
    "scry_hip_llama_forward": [vp, vp, i32, vp],
    "scry_hip_llama_prefill": [vp, vp, i32, vp, i32, vp],
    "scry_hip_llama_decode_batch": [vp, vp, i32, vp, i32, vp, vp],
    "scry_hip_llama_bench_prefill": [vp, vp, i32, i32, i32, vp, P(f64), P(f64)],
    "scry_hip_llama_bench_prefill_batch": [vp, vp, i32, i32, i32, vp, P(f64), P(f64)],
    "scry_hip_graph_replay": [],
    "scry_hip_llama_profile_step": [vp, vp, i32, i32, i32, P(i32), vp, vp],
    "scry_hip_llama_bench_decode": [vp, vp, i32, i32, i32, vp, P(f64)],
    "scry_hip_llama_bench_decode_sampled": [vp, vp, i32, i32, i32, P(SamplingConfigC), u64, vp, P(f64)],
    "scry_hip_llama_time_projection": [vp, i32, i32, i32, P(f64), P(f64)],
    "scry_hip_llama_time_attention": [vp, i32, i32, P(f64), P(f64)],
    "scry_hip_bench_qgemv": [i32, i32, i32, i32, i32, i32, i32, P(f64), P(f64)],
    "scry_hip_bench_qgemv_dist": [i32, i32, i32, i32, i32, i32, i32, i32, i32, vp, P(f64), P(f64)],
}

_lib = None


def header_functions() -> list[str]:
    """Names of all functions declared in include/scry_hip.h."""
    text = open(HEADER).read()
    return re.findall(r"^\s*(?:int|const char \*)\s*(scry_hip_\w+)\s*\(", text, re.M)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run `python -m esolearn_amd.build`")
    L = C.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = C.c_char_p if name == "scry_hip_last_error" else C.c_int
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != SCRY_OK:
        msg = load().scry_hip_last_error()
        raise ScryHipError(rc, msg.decode() if msg else "")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))
