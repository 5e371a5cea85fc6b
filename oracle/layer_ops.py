"""Element-wise operations of realm_forward_layer restated in numpy --
TEST INFRASTRUCTURE ONLY.

  rms_norm   candle-nn 0.9.1 ops::rms_norm on the CPU, as
             CandleNeuralOpsBackend::rms_norm calls it
             (crates/realm-compute-cpu/src/candle_neural_ops_backend.rs:32-60):
             per row, sum2 = sum of x^2 in f32, m = sqrt(sum2 / dim + eps),
             y = x / m * weight.  candle-nn is a Cargo.lock dependency that is
             not in the reference tree; its published algorithm is restated.
  residual   CandleCpuBackend::add, element-wise x + r (memory64_host.rs:
             2318-2324, 2452-2458).
  swiglu     memory64_host.rs:2419-2425: sigmoid = 1 / (1 + exp(-g)),
             silu = g * sigmoid, out = silu * up, in f32.
"""
from __future__ import annotations

import numpy as np


def rms_norm(x, weight, eps: float, residual=None):
    x = np.asarray(x, np.float32)
    if residual is not None:
        x = (x + np.asarray(residual, np.float32)).astype(np.float32)
    w = np.asarray(weight, np.float32)
    dim = np.float32(x.shape[-1])
    sum2 = np.sum(x * x, axis=-1, dtype=np.float32, keepdims=True)
    m = np.sqrt(sum2 / dim + np.float32(eps)).astype(np.float32)
    return (x / m * w).astype(np.float32), x


def swiglu(gate, up):
    g = np.asarray(gate, np.float32)
    u = np.asarray(up, np.float32)
    with np.errstate(over="ignore"):
        sig = (np.float32(1.0) / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
    return ((g * sig).astype(np.float32) * u).astype(np.float32)
