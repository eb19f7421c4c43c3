"""Llama with int8 projections on the GPU (crates/scry-llm/src/nn/llama.rs,
kv_cache.rs, generate.rs) over the scry_hip C ABI.

    model = LlamaModel.new_random(LlamaConfig(...), seed=0)   # LlamaModel::new + int8 layout
    cache = model.new_llama_kv_cache(max_seq)                 # llama.rs:712-719
    logits = model.forward_with_llama_cache(token, pos, cache)  # llama.rs:744-763
    tokens = generate(model, prompt, SamplingConfig(temperature=0, max_tokens=128))
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, fields

import numpy as np

from ._lib import LlamaConfigC, SamplingConfigC, call, load

QUANT_PER_TENSOR = 0
QUANT_BLOCK32 = 1
QUANT_BF16 = 2  # bf16 weights, bf16-rounded activations (the reference's bf16 feature)
T_EMBED, T_QKV, T_O, T_GATE, T_UP, T_DOWN, T_LM_HEAD = range(7)
@dataclass
class LlamaConfig:
    """LlamaConfig (llama.rs:20-34)."""

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
    rope_scaling: tuple | None = None  # (factor, low_freq_factor, high_freq_factor, orig_max_pos)

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.n_heads

    def to_c(self) -> LlamaConfigC:
        c = LlamaConfigC()
        for f in fields(self):
            if f.name != "rope_scaling":
                setattr(c, f.name, getattr(self, f.name))
        if self.rope_scaling is not None:
            c.has_rope_scaling = 1
            (c.rs_factor, c.rs_low_freq_factor, c.rs_high_freq_factor,
             c.rs_original_max_pos) = self.rope_scaling
        return c

    # BASELINE.json configurations
    @staticmethod
    def tiny() -> "LlamaConfig":  # stories15M-like: h288 L6 H6 ffn768 V32000
        return LlamaConfig(32000, 288, 768, 6, 6, 6, max_seq_len=256, rope_theta=10000.0,
                           tie_word_embeddings=True)

    @staticmethod
    def llama2_7b() -> "LlamaConfig":
        return LlamaConfig(32000, 4096, 11008, 32, 32, 32, max_seq_len=2048, rope_theta=10000.0,
                           tie_word_embeddings=False)

    @staticmethod
    def llama3_8b() -> "LlamaConfig":
        return LlamaConfig(128256, 4096, 14336, 32, 32, 8, max_seq_len=2048,
                           rope_theta=500000.0, tie_word_embeddings=False)


class LlamaKvCache:
    """Device KV cache (LlamaKvCache, kv_cache.rs:134-145)."""

    def __init__(self, model: "LlamaModel", max_seq: int):
        self.model = model
        self.max_seq = max_seq
        h = C.c_void_p()
        call("scry_hip_llama_kv_cache_new", model.h, max_seq, C.byref(h))
        self.h = h.value

    @property
    def seq_len(self) -> int:
        v = C.c_int()
        call("scry_hip_kv_cache_seq_len", self.h, C.byref(v))
        return v.value

    def layer(self, layer: int) -> tuple[np.ndarray, np.ndarray]:
        n = self.max_seq * self.model.cfg.n_kv_heads * self.model.cfg.head_dim
        k = np.empty(n, np.float32)
        v = np.empty(n, np.float32)
        call("scry_hip_kv_cache_layer_to_vec", self.h, layer, k.ctypes.data, v.ctypes.data, n)
        return k, v

    def free(self) -> None:
        if self.h:
            load().scry_hip_kv_cache_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class LlamaModel:
    """LlamaModel<HipBackend> with int8 projections."""

    def __init__(self, handle: int, cfg: LlamaConfig, quant_mode: int):
        self.h = handle
        self.cfg = cfg
        self.quant_mode = quant_mode
        self._caches: list = []

    @staticmethod
    def new_random(cfg: LlamaConfig, seed: int = 0, quant_mode: int = QUANT_PER_TENSOR,
                   init_on_device: bool = False):
        """LlamaModel::new(config, Rng::with_seed(seed)) then the int8 layout step."""
        c = cfg.to_c()
        h = C.c_void_p()
        call("scry_hip_llama_new_random", C.byref(c), int(seed), quant_mode, int(init_on_device),
             C.byref(h))
        return LlamaModel(h.value, cfg, quant_mode)

    @staticmethod
    def from_safetensors(cfg: LlamaConfig, paths, quant_mode: int = QUANT_PER_TENSOR):
        """LlamaModel::from_safetensors (llama.rs:765-958): HF safetensors shards
        (F32 / BF16 / F16), then the int8 layout step; the RMSNorms use the
        loaded weights and cfg.rms_norm_eps."""
        enc = [str(p).encode() for p in ([paths] if isinstance(paths, (str, bytes)) else paths)]
        arr = (C.c_char_p * len(enc))(*enc)
        c = cfg.to_c()
        h = C.c_void_p()
        call("scry_hip_llama_from_safetensors", C.byref(c), arr, len(enc), quant_mode, C.byref(h))
        return LlamaModel(h.value, cfg, quant_mode)

    def set_tensor(self, tensor_id: int, layer: int, data) -> None:
        a = np.ascontiguousarray(data, dtype=np.float32).ravel()
        call("scry_hip_llama_set_tensor", self.h, tensor_id, layer, a.ctypes.data, a.size)

    def qtensor(self, tensor_id: int, layer: int = 0) -> tuple[np.ndarray, np.float32]:
        cfg = self.cfg
        h, ffn, hd = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
        qd, kvd = cfg.n_heads * hd, cfg.n_kv_heads * hd
        n = {T_QKV: h * (qd + 2 * kvd), T_O: qd * h, T_GATE: h * ffn, T_UP: h * ffn,
             T_DOWN: ffn * h, T_LM_HEAD: cfg.vocab_size * h}[tensor_id]
        out = np.empty(n, np.int8)
        s = C.c_float()
        call("scry_hip_llama_get_qtensor", self.h, tensor_id, layer, out.ctypes.data, n,
             C.byref(s))
        return out, np.float32(s.value)

    def embed(self) -> np.ndarray:
        n = self.cfg.vocab_size * self.cfg.hidden_size
        out = np.empty(n, np.float32)
        call("scry_hip_llama_get_embed", self.h, out.ctypes.data, n)
        return out

    def new_llama_kv_cache(self, max_seq: int) -> LlamaKvCache:
        c = LlamaKvCache(self, max_seq)
        self._caches.append(c)
        return c

    def forward_with_llama_cache(self, token: int, pos: int, cache: LlamaKvCache,
                                 want_logits: bool = True):
        """Returns (logits [V] or None, device argmax)."""
        lg = np.empty(self.cfg.vocab_size, np.float32) if want_logits else None
        am = C.c_int64()
        call("scry_hip_llama_forward_with_cache", self.h, cache.h, int(token), int(pos),
             lg.ctypes.data if lg is not None else None, C.byref(am))
        return lg, int(am.value)

    def generate_greedy(self, prompt, max_tokens: int, want_logits: bool = False,
                        prefill: bool = False):
        """generate() at temperature 0; prefill=True runs the prompt (all but its
        last token) through one batched prefill instead of token by token."""
        p = np.ascontiguousarray(prompt, dtype=np.int64)
        nout = max(1, max_tokens)
        toks = np.empty(nout, np.int64)
        n = C.c_int()
        lg = np.empty(nout * self.cfg.vocab_size, np.float32) if want_logits else None
        fn = "scry_hip_llama_generate_greedy_prefill" if prefill else "scry_hip_llama_generate_greedy"
        call(fn, self.h, p.ctypes.data, p.size, max_tokens,
             toks.ctypes.data, C.byref(n), lg.ctypes.data if lg is not None else None)
        if want_logits:
            return toks[: n.value], lg.reshape(nout, -1)[: n.value]
        return toks[: n.value]

    def generate(self, prompt, config: "SamplingConfig", rng: "Rng", want_logits: bool = False,
                 prefill: bool = False):
        """generate() (generate.rs:51-89) with sample_token on the device;
        rng (fastrand::Rng state) advances by one draw per sampled token."""
        p = np.ascontiguousarray(prompt, dtype=np.int64)
        nout = max(1, config.max_tokens)
        toks = np.empty(nout, np.int64)
        n = C.c_int()
        lg = np.empty(nout * self.cfg.vocab_size, np.float32) if want_logits else None
        sc = SamplingConfigC(float(config.temperature), int(config.top_k), float(config.top_p),
                             int(config.max_tokens))
        st = C.c_uint64(rng.state)
        call("scry_hip_llama_generate", self.h, p.ctypes.data, p.size, C.byref(sc), C.byref(st),
             int(prefill), toks.ctypes.data, C.byref(n), lg.ctypes.data if lg is not None else None)
        rng.state = int(st.value)
        if want_logits:
            return toks[: n.value], lg.reshape(nout, -1)[: n.value]
        return toks[: n.value]

    def forward(self, tokens) -> np.ndarray:
        """LlamaModel::forward: logits [seq, V] for every position (no cache)."""
        t = np.ascontiguousarray(tokens, dtype=np.int64)
        lg = np.empty((t.size, self.cfg.vocab_size), np.float32)
        call("scry_hip_llama_forward", self.h, t.ctypes.data, t.size, lg.ctypes.data)
        return lg

    def prefill(self, caches, tokens, want_logits: bool = True):
        """Batched prefill of tokens [n_seq, seq] into the given caches (one per
        sequence); returns the last position's logits [n_seq, V] or None."""
        t = np.ascontiguousarray(np.atleast_2d(tokens), dtype=np.int64)
        n_seq, seq = t.shape
        if len(caches) != n_seq:
            raise ValueError("one cache per sequence")
        hs = (C.c_void_p * n_seq)(*[c.h for c in caches])
        lg = np.empty((n_seq, self.cfg.vocab_size), np.float32) if want_logits else None
        call("scry_hip_llama_prefill", self.h, hs, n_seq, t.ctypes.data, seq,
             lg.ctypes.data if lg is not None else None)
        return lg

    def decode_batch(self, caches, tokens, steps: int, want_logits: bool = False):
        """Greedy decode of several sequences at once: tokens[i] is the token at
        position caches[i].seq_len; returns the next tokens [n_seq, steps] (and
        the logits [steps, n_seq, V] with want_logits)."""
        t = np.ascontiguousarray(np.ravel(tokens), dtype=np.int64)
        n_seq = t.size
        if len(caches) != n_seq:
            raise ValueError("one cache per sequence")
        hs = (C.c_void_p * n_seq)(*[c.h for c in caches])
        toks = np.empty((n_seq, steps), np.int64)
        lg = np.empty((steps, n_seq, self.cfg.vocab_size), np.float32) if want_logits else None
        call("scry_hip_llama_decode_batch", self.h, hs, n_seq, t.ctypes.data, steps, toks.ctypes.data,
             lg.ctypes.data if lg is not None else None)
        return (toks, lg) if want_logits else toks

    def bench_prefill(self, prompts, decode_steps: int, batched: bool = False):
        """(prefill ms, decode ms, tokens [n_seq, decode_steps]) for prompts
        [n_seq, n_prompt]: batched prefill, then greedy decode per sequence in
        turn, or (batched) of all sequences per step."""
        p = np.ascontiguousarray(prompts, dtype=np.int64)
        n_seq, n_prompt = p.shape
        toks = np.empty((n_seq, decode_steps), np.int64)
        pm, dm = C.c_double(), C.c_double()
        fn = "scry_hip_llama_bench_prefill_batch" if batched else "scry_hip_llama_bench_prefill"
        call(fn, self.h, p.ctypes.data, n_seq, n_prompt, decode_steps, toks.ctypes.data, C.byref(pm),
             C.byref(dm))
        return pm.value, dm.value, toks

    def bench_decode(self, prompt, warmup: int, steps: int):
        p = np.ascontiguousarray(prompt, dtype=np.int64)
        toks = np.empty(steps, np.int64)
        ms = C.c_double()
        call("scry_hip_llama_bench_decode", self.h, p.ctypes.data, p.size, warmup, steps,
             toks.ctypes.data, C.byref(ms))
        return ms.value, toks

    def profile_step(self, prompt, steps: int):
        """Per-launch (start, end) in us from each step's first start, for
        `steps` replays of the stamped decode step after the prompt: two arrays
        [steps, 5 L + 2] (per layer qkv, attention, o, gate/up, down; then the
        LM head and the argmax finish)."""
        p = np.ascontiguousarray(prompt, dtype=np.int64)
        nl = 5 * self.cfg.n_layers + 2
        st = np.empty((steps, nl), np.float64)
        en = np.empty((steps, nl), np.float64)
        n = C.c_int()
        call("scry_hip_llama_profile_step", self.h, p.ctypes.data, p.size, steps, nl, C.byref(n),
             st.ctypes.data, en.ctypes.data)
        return st, en

    def bench_decode_sampled(self, prompt, warmup: int, steps: int, config: "SamplingConfig",
                             seed: int = 0):
        """bench_decode with the device sampler after every LM head."""
        p = np.ascontiguousarray(prompt, dtype=np.int64)
        toks = np.empty(steps, np.int64)
        ms = C.c_double()
        sc = SamplingConfigC(float(config.temperature), int(config.top_k), float(config.top_p),
                             int(config.max_tokens))
        call("scry_hip_llama_bench_decode_sampled", self.h, p.ctypes.data, p.size, warmup, steps,
             C.byref(sc), int(seed), toks.ctypes.data, C.byref(ms))
        return ms.value, toks

    def time_projection(self, tensor_id: int, iters: int = 64):
        us, b = C.c_double(), C.c_double()
        call("scry_hip_llama_time_projection", self.h, tensor_id, 0, iters, C.byref(us),
             C.byref(b))
        return us.value, b.value

    def time_attention(self, ctx_len: int, iters: int = 64):
        """Average device time of the decode attention kernel at ctx_len cached
        positions (rotating over the layers' caches) and its algorithmic bytes."""
        us, b = C.c_double(), C.c_double()
        call("scry_hip_llama_time_attention", self.h, int(ctx_len), int(iters), C.byref(us),
             C.byref(b))
        return us.value, b.value

    def free(self) -> None:
        if self.h:
            for c in self._caches:
                c.free()
            self._caches = []
            load().scry_hip_llama_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class SamplingConfig:
    """SamplingConfig (generate.rs:25-45)."""

    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    max_tokens: int = 128


class Rng:
    """fastrand::Rng (2.3.0, wyrand): the 64-bit state the device sampler
    advances.  Rng.with_seed(s) starts at s, as Rng::with_seed."""

    def __init__(self, state: int = 0):
        self.state = int(state) & 0xFFFFFFFFFFFFFFFF

    @classmethod
    def with_seed(cls, seed: int) -> "Rng":
        return cls(seed)


def generate(model: LlamaModel, prompt_tokens, config: SamplingConfig, rng: Rng | None = None) -> np.ndarray:
    """generate() (generate.rs:51-89) with sample_token (generate.rs:92-186):
    greedy below temperature 1e-8, else top-k / softmax / top-p / weighted draw
    by the device sampler; the token loop runs entirely on the device."""
    if len(prompt_tokens) == 0:
        raise ValueError("generate: prompt_tokens must not be empty")
    if config.temperature < 1e-8:
        return model.generate_greedy(prompt_tokens, config.max_tokens)
    if rng is None:
        raise ValueError("generate: sampling needs an rng (Rng.with_seed(seed))")
    return model.generate(prompt_tokens, config, rng)


def bench_qgemv(m: int, k: int, n: int, quant_mode: int = QUANT_PER_TENSOR, n_bufs: int = 32,
                warmup: int = 50, iters: int = 1000):
    us, b = C.c_double(), C.c_double()
    call("scry_hip_bench_qgemv", m, k, n, quant_mode, n_bufs, warmup, iters, C.byref(us),
         C.byref(b))
    return us.value, b.value


def bench_qgemv_dist(m: int, k: int, n: int, quant_mode: int = QUANT_PER_TENSOR, path: int = 0,
                     n_bufs: int = 32, warmup: int = 50, iters: int = 1000, group: int = 8):
    """(per-launch device times of each group of `group` launches [iters/group]
    in us, back-to-back average us, algorithmic bytes per launch) of
    matmul_i8_f32 at (m, k, n); path 0 = the automatic route, 1 = the GEMV,
    2 = the MFMA GEMM, 3 = the skinny MFMA kernel (up to 16 rows)."""
    per = np.empty(iters // group, np.float64)
    us, b = C.c_double(), C.c_double()
    call("scry_hip_bench_qgemv_dist", m, k, n, quant_mode, path, n_bufs, warmup, iters, group,
         per.ctypes.data, C.byref(us), C.byref(b))
    return per, us.value, b.value
