"""TEST INFRASTRUCTURE ONLY: numpy restatement of Dense's bias + activation
epilogue and of weights.Store's f64 products.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
as the checker. It follows:
  * core.Activate (core/activate.go:6-37), in f64;
  * applyBiasAct (layers/dense/dense.go:145-167) for float32 activations:
    v = f64(pre) + bias[o] (bias f64; only when a bias is set), pre = f32(v),
    post = f32(Activate(f64(f32(v))));
  * matVecNativeF64 / matVecTNativeF64 (weights/native.go:1120-1158): f64 sums
    of f64(w) * x over the decoded weights, rows with gy == 0 skipped in the
    transposed product.
"""
from __future__ import annotations

import math

import numpy as np

# core.ActivationType (core/layer.go:88-99)
ACT = {"linear": -1, "relu": 0, "silu": 1, "gelu": 2, "tanh": 3, "sigmoid": 4, "leaky_relu": 5, "relu2": 6}


def activate(x: np.ndarray, act) -> np.ndarray:
    """core.Activate in f64 (core/activate.go:6-37)."""
    a = ACT[act] if isinstance(act, str) else int(act)
    x = np.asarray(x, np.float64)
    with np.errstate(over="ignore"):
        if a == 0:
            return np.where(x < 0, 0.0, x)
        if a == 6:
            return np.where(x < 0, 0.0, x * x)
        if a == 5:
            return np.where(x < 0, 0.01 * x, x)
        if a == 1:
            return x / (1.0 + np.exp(-x))
        if a == 2:
            return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x * x * x)))
        if a == 3:
            return np.tanh(x)
        if a == 4:
            return 1.0 / (1.0 + np.exp(-x))
    return x


def apply_bias_act(pre: np.ndarray, bias, act):
    """applyBiasAct for float32 tensors: returns (pre, post) as f32 arrays of pre's shape."""
    pre = np.asarray(pre, np.float32)
    rows = pre.shape[-1]
    if bias is not None and len(bias):
        b = np.zeros(rows, np.float64)
        n = min(rows, len(bias))  # o < len(bias)
        b[:n] = np.asarray(bias, np.float64)[:n]
        pre = (pre.astype(np.float64) + b).astype(np.float32)
    post = activate(pre.astype(np.float64), act).astype(np.float32)
    return pre, post


def store_matvec_f64(w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """matVecNativeF64 over decoded f32 weights w (rows*cols): exact sums rounded to f64."""
    w = np.asarray(w, np.float32).reshape(rows, cols).astype(np.float64)
    x = np.asarray(x, np.float64)[:cols]
    return np.array([math.fsum(w[r] * x) for r in range(rows)], np.float64)


def store_matvec_t_f64(w: np.ndarray, rows: int, cols: int, gy: np.ndarray, gx: np.ndarray) -> np.ndarray:
    """matVecTNativeF64: gx[c] + sum_r w[r, c] * gy[r] (rows with gy == 0 skipped), exact sums."""
    w = np.asarray(w, np.float32).reshape(rows, cols).astype(np.float64)
    gy = np.asarray(gy, np.float64)[:rows]
    keep = gy != 0
    prod = w[keep] * gy[keep, None]
    out = np.array(gx, np.float64, copy=True)
    for c in range(cols):
        out[c] = math.fsum(np.concatenate(([out[c]], prod[:, c])))
    return out
