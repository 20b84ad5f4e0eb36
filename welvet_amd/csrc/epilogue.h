// epilogue.h — Dense's bias + activation epilogue on the device.
//
// applyBiasAct (layers/dense/dense.go:145-167) for float32 activations:
//   v    = f64(pre) + bias[o]            (bias is f64; only when a bias is set)
//   pre  = f32(v)                        (only when a bias is set)
//   post = f32(Activate(f64(f32(v))))    (core/activate.go:6-37, f64 math)
// With a linear activation and no bias, post is a copy of pre.
#pragma once

#include <hip/hip_runtime.h>

#include "wv_internal.h"

namespace wv {

// core.Activate (core/activate.go:6-37) in f64.
__device__ __forceinline__ double activate_f64(double x, int act) {
    switch (act) {
    case ACT_RELU: return x < 0.0 ? 0.0 : x;
    case ACT_RELU2: return x < 0.0 ? 0.0 : x * x;
    case ACT_LEAKY_RELU: return x < 0.0 ? 0.01 * x : x;
    case ACT_SILU: return x / (1.0 + exp(-x));
    case ACT_GELU: return 0.5 * x * (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)));
    case ACT_TANH: return tanh(x);
    case ACT_SIGMOID: return 1.0 / (1.0 + exp(-x));
    default: return x;
    }
}

// Stores pre (biased when `bias` is set) to y[idx] and act(pre) to post[idx];
// returns the stored pre.
__device__ __forceinline__ float store_bias_act(float* y, float* post, int64_t idx, float s, const double* bias,
                                                int64_t row, int act) {
    if (bias) s = float(double(s) + bias[row]);
    y[idx] = s;
    post[idx] = act == ACT_LINEAR ? s : float(activate_f64(double(s), act));
    return s;
}

}  // namespace wv
