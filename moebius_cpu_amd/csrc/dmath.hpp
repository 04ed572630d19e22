// Device math shared by the kernels: the reference's own exp/SiLU
// (src/engine/math.rs:17-36, a Cephes range reduction with a degree-6
// polynomial), evaluated with the same f32 operations so the GPU's SiLU
// matches the CPU engine bit for bit. IEEE fused multiply-add and the correctly
// rounded f32 division (hipcc's default) make every step deterministic; the
// library builds with -ffp-contract=off so no multiply-add is fused implicitly.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mh {

__device__ __forceinline__ float ref_exp(float x) {
    constexpr float LOG2_E = 1.44269504088896340736f;
    constexpr float LN2_HI = 0.693359375f;
    constexpr float LN2_LO = -2.12194440e-4f;
    // clamp that keeps NaN, as f32::clamp
    x = x < -87.33655f ? -87.33655f : (x > 88.0f ? 88.0f : x);
    const float n = roundf(x * LOG2_E);  // half away from zero, as f32::round
    const float r = __builtin_fmaf(n, -LN2_LO, __builtin_fmaf(n, -LN2_HI, x));
    float p = 1.9875691e-4f;
    p = __builtin_fmaf(p, r, 1.3981999e-3f);
    p = __builtin_fmaf(p, r, 8.333452e-3f);
    p = __builtin_fmaf(p, r, 4.1665796e-2f);
    p = __builtin_fmaf(p, r, 1.6666665e-1f);
    p = __builtin_fmaf(p, r, 5e-1f);
    const float poly = __builtin_fmaf(p * r, r, r) + 1.0f;
    const uint32_t bits = uint32_t(int32_t(n) + 127) << 23;
    return poly * __uint_as_float(bits);
}

__device__ __forceinline__ float ref_silu(float x) { return x / (1.0f + ref_exp(-x)); }

// FAST precision's SiLU: x . 1 / (1 + 2^(-x log2 e)) from the hardware base-2
// exponential and reciprocal (v_exp_f32, v_rcp_f32, about 1 ulp each), within a
// few ulp of ref_silu at a fraction of its cost (no polynomial, no IEEE
// division). At the ends it saturates as ref_silu does: for x below about -88
// the exponential overflows and the result is -0 (ref_silu: a value of order
// 1e-37), above about 88 it is x. NaN stays NaN.
__device__ __forceinline__ float fast_silu(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.44269504088896340736f));
}

// The SiLU of a kernel instantiated for FAST precision (FM) or for the
// reference's arithmetic.
template <bool FM>
__device__ __forceinline__ float silu_of(float x) {
    if constexpr (FM) return fast_silu(x);
    else return ref_silu(x);
}

// Rust f32::max(v, 0.0): 0 for NaN.
__device__ __forceinline__ float relu_ref(float v) { return v > 0.0f ? v : 0.0f; }

}  // namespace mh
