// Activation functions in f32, shared by the elementwise kernels and the
// GEMM epilogue so that both give the same bits.
// Reference: modules/nn.mojo:576-647 (activation, _gelu_tanh),
// gpu/linear.mojo:662-684 (gelu_tanh_bias).
#pragma once
#include "t2h_device.h"

namespace t2h {
namespace {

// GELU-tanh: 0.5*v*(1+tanh(z)) == v * sigmoid(2z) == v / (1 + exp(-2z)), with
// z = 0.7978845608028654*(v + 0.044715*v^3). exp via v_exp_f32 (exp2) and the
// reciprocal via v_rcp_f32: a few ulp, no cancellation near z = 0 (unlike
// (1-e)/(1+e)), and saturates cleanly (exp overflow -> 0, underflow -> v).
__device__ __forceinline__ float gelu_tanh_f(float v) {
    constexpr float k0 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;  // -2*sqrt(2/pi)*log2(e)
    constexpr float k1 = k0 * 0.044715f;
    const float v2 = v * v;
    const float arg = v * __builtin_fmaf(k1, v2, k0);   // -2z * log2(e)
    const float e = __builtin_amdgcn_exp2f(arg);
    return v * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float silu_f(float v) {
    const float e = __builtin_amdgcn_exp2f(-v * 1.4426950408889634f);
    return v * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float gelu_erf_f(float v) {
    return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
}

template <int KIND> __device__ __forceinline__ float act_f(float v) {
    if constexpr (KIND == T2H_ACT_RELU) return v > 0.0f ? v : 0.0f;
    else if constexpr (KIND == T2H_ACT_SILU) return silu_f(v);
    else if constexpr (KIND == T2H_ACT_GELU) return gelu_erf_f(v);
    else return gelu_tanh_f(v);
}

// x + b as fma(x, 1, b): one rounding of the exact sum, i.e. the same bits as
// the reference's `acc += b`, in a form that fuses with the f16 -> f32 convert.
__device__ __forceinline__ float bias_add(float x, float b) { return __builtin_fmaf(x, 1.0f, b); }

}  // namespace
}  // namespace t2h
