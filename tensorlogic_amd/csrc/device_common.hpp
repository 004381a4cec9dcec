// device_common.hpp -- device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tlhip {

typedef _Float16 h16;
typedef h16 h2 __attribute__((ext_vector_type(2)));
typedef h16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(h16, b); }
// v_cvt_f16_f32: round-to-nearest-even, f16 denormals preserved.
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (h16)f); }
__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// Pair (lo half of a, lo half of b) and (hi half of a, hi half of b).
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

__device__ __forceinline__ float fdot2(h2 a, h2 b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
}

template <int W>
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = W / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// sigmoid as the reference CPU path computes it (activations.rs:252-266):
// f32 1 / (1 + exp(-x)), then stored f16.
__device__ __forceinline__ uint16_t sigmoid_h(uint16_t x) {
    float v = h2f(x);
    return f2h(1.0f / (1.0f + expf(-v)));
}
// TL silu(g) * u: three f16 stores (sigmoid, x*sigmoid, *u).
__device__ __forceinline__ uint16_t swiglu_h(uint16_t g, uint16_t u) {
    uint16_t s = sigmoid_h(g);
    uint16_t a = f2h(h2f(g) * h2f(s));
    return f2h(h2f(a) * h2f(u));
}
__device__ __forceinline__ uint16_t add_h(uint16_t a, uint16_t b) { return f2h(h2f(a) + h2f(b)); }

// gelu_f16 (unified.metal:837-848), tanh form, evaluated in f32 with each
// product and sum rounded separately:
// 0.5*x*(1 + tanh(sqrt(2/pi) * (x + 0.044715*x^3))).
__device__ __forceinline__ uint16_t gelu_h(uint16_t a) {
    const float v = h2f(a);
    const float x3 = __fmul_rn(__fmul_rn(v, v), v);
    const float inner = __fmul_rn(0.7978845608f, __fadd_rn(v, __fmul_rn(0.044715f, x3)));
    return f2h(__fmul_rn(__fmul_rn(0.5f, v), __fadd_rn(1.0f, tanhf(inner))));
}

// Shared epilogue of the GEMV kernels with the bias / residual element
// already in registers (see GemvEpi).
__device__ __forceinline__ uint16_t epilogue_v(int epi, float acc, uint16_t b, uint16_t r) {
    uint16_t y = f2h(acc);
    switch (epi) {
        case 1: y = add_h(y, b); break;
        case 2: y = add_h(r, y); break;
        case 4: y = add_h(r, add_h(y, b)); break;
        case 5: y = gelu_h(add_h(y, b)); break;
        default: break;
    }
    return y;
}

// Shared epilogue of the GEMM kernel (see GemvEpi).
__device__ __forceinline__ uint16_t epilogue_h(int epi, float acc, const uint16_t* bias,
                                               const uint16_t* resid, size_t ri, int n) {
    uint16_t r = f2h(acc);
    switch (epi) {
        case 1: r = add_h(r, bias[n]); break;
        case 2: r = add_h(resid[ri], r); break;
        case 4: r = add_h(resid[ri], add_h(r, bias[n])); break;
        case 5: r = gelu_h(add_h(r, bias[n])); break;
        default: break;
    }
    return r;
}

}  // namespace tlhip
