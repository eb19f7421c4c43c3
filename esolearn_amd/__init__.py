"""esolearn_amd: MI355X (gfx950) backend for scry-llm's int8 Llama forward path.

The compute lives in libscry_hip.so (hand-written HIP kernels + a C ABI,
include/scry_hip.h); this package is the host-side mirror of the reference
interface: ``HipBackend`` (backend trait methods), ``LlamaModel`` /
``LlamaKvCache`` / ``generate`` (llama.rs, kv_cache.rs, generate.rs).
"""
from .backend import HipBackend, I8Storage, Storage, init  # noqa: F401
from .linear import Linear, QuantState, normal_vec  # noqa: F401
from .llama import (QUANT_BF16, QUANT_BLOCK32, QUANT_PER_TENSOR, LlamaConfig, LlamaKvCache,  # noqa: F401
                    LlamaModel, Rng, SamplingConfig, bench_qgemv, generate)
from ._lib import ScryHipError  # noqa: F401
from . import synth  # noqa: F401
