"""Linear layer (crates/scry-llm/src/nn/linear.rs:1-101) on the HIP backend.

``output = input @ weight + bias`` with the weight stored ``[in_features,
out_features]`` (the HF ``Conv1D`` layout).  ``quantize_weights()`` switches
``forward()`` to ``matmul_i8_f32_bias`` (linear.rs:67-94): per-tensor int8
weights (the bit-exact ``quantize_symmetric``), the bias added in the store
epilogue of the dequant-fused GEMV (up to 16 rows) or of the MFMA GEMM (more
rows).  This is the quantized Linear of GPT-2's MLP and attention projections
and of scry-stt's Whisper layers (checkpoint/mod.rs:169-194).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np

from ._lib import call
from .backend import HipBackend, I8Storage, Storage, _out, _st
from .llama import Rng


@dataclass
class QuantState:
    """QuantState (linear.rs:9-13): int8 weight storage and its scale."""

    weight_q: I8Storage
    scale: np.float32


def normal_vec(rng: Rng, n: int, mean: float, std: float) -> Storage:
    """init::normal_vec (init.rs:12-14) into device storage; rng advances by
    two Rng::f64 calls per sample."""
    st = C.c_uint64(rng.state)
    o = _out()
    call("scry_hip_normal_vec", C.byref(st), n, float(mean), float(std), C.byref(o))
    rng.state = int(st.value)
    return _st(o, n)


class Linear:
    """Linear (linear.rs:16-25)."""

    def __init__(self, weight: Storage, bias: Storage, in_features: int, out_features: int):
        if weight.n != in_features * out_features or bias.n != out_features:
            raise ValueError("Linear: weight must be [in, out] and bias [out]")
        self.weight = weight
        self.bias = bias
        self.in_features = in_features
        self.out_features = out_features
        self.quant: QuantState | None = None

    @classmethod
    def new(cls, in_features: int, out_features: int, rng: Rng) -> "Linear":
        """Linear::new (linear.rs:28-39): N(0, 0.02) weights, zero bias."""
        w = normal_vec(rng, in_features * out_features, 0.0, 0.02)
        return cls(w, HipBackend.zeros(out_features), in_features, out_features)

    @classmethod
    def from_arrays(cls, weight, bias) -> "Linear":
        """A layer from host arrays: weight [in, out], bias [out]."""
        w = np.ascontiguousarray(weight, np.float32)
        b = np.ascontiguousarray(bias, np.float32).ravel()
        return cls(HipBackend.from_vec(w.ravel()), HipBackend.from_vec(b), w.shape[0], w.shape[1])

    def apply_residual_scaling(self, n_layer: int) -> None:
        """apply_residual_scaling (linear.rs:41-49): every weight times
        1/sqrt(2 n_layer) in f64, rounded once to f32 (a set-up step, on the
        host as in the reference)."""
        scale = 1.0 / math.sqrt(2.0 * n_layer)
        data = (self.weight.to_vec().astype(np.float64) * scale).astype(np.float32)
        old = self.weight
        self.weight = HipBackend.from_vec(data)
        old.free()

    def quantize_weights(self) -> None:
        """quantize_weights (linear.rs:51-65): symmetric per-tensor int8 on the
        device; forward() then takes the quantized path.  The f32 weights
        stay."""
        q, s = HipBackend.quantize_symmetric(self.weight)
        self.quant = QuantState(q, s)

    def forward(self, x: Storage, seq: int) -> Storage:
        """forward (linear.rs:67-94): x [seq, in_features] -> [seq, out_features]."""
        if x.n != seq * self.in_features:
            raise ValueError(f"Linear.forward: input holds {x.n} values, expected {seq}x{self.in_features}")
        if self.quant is not None:
            return HipBackend.matmul_i8_f32_bias(x, self.quant.weight_q, self.quant.scale, self.bias,
                                                 seq, self.in_features, self.out_features)
        # ops::matmul_bias: the product (bf16 operands in bf16 mode), then the
        # f32 bias row added to every output row on the device
        return HipBackend.matmul_bias(x, self.weight, self.bias, seq, self.in_features,
                                      self.out_features)

    def parameters(self) -> list[Storage]:
        """Module::parameters (linear.rs:97-101)."""
        return [self.weight, self.bias]

    def free(self) -> None:
        for t in (self.weight, self.bias):
            t.free()
        if self.quant is not None:
            self.quant.weight_q.free()
            self.quant = None


def bench_linear_bias(m: int, k: int, n: int, n_bufs: int = 64, warmup: int = 50, iters: int = 1000):
    """Average device time (us) and algorithmic bytes of one quantized
    Linear::forward GEMV launch (bias fused), over n_bufs weight copies."""
    us, b = C.c_double(), C.c_double()
    call("scry_hip_bench_qgemv_bias", m, k, n, n_bufs, warmup, iters, C.byref(us), C.byref(b))
    return us.value, b.value
