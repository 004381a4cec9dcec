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

// GGUF payload -> f16 pairs.  A byte b placed under the high byte 0x64 is
// the f16 1024 + b, so (1024 + q) - 1032 = q - 8 (Q4_0) and, after the xor
// that offsets int8 by 128, (1024 + q + 128) - 1152 = q (Q8_0), both exact;
// the multiply by the block scale d is then the one correctly rounded
// product RNE_f16((q - 8) * d) / RNE_f16(q * d) of the reference's
// dequantisation.  perm(X, Y, sel) takes byte i from sel byte i: 0-3 = Y's
// bytes, 4-7 = X's.
// Q4_0: bytes j..j+3 of the 16 payload bytes hold elements j..j+3 in their
// low nibbles and j+16..j+19 in their high nibbles; out = (e0,e2) (e1,e3)
// (e16,e18) (e17,e19) relative to j.
// (a & m) | o as the one instruction v_and_or_b32.  Written out because
// the compiler splits it into v_and + v_or when m and o are constants (a
// three-operand instruction takes no literal here); the mask comes in a
// scalar register, the or-value in a vector register, both set once.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
    return r;
}

__device__ __forceinline__ void q4_unpack(uint32_t w, h2 dd, h2 out[4]) {
    // A low nibble q under the exponent bits 0x6400 is the f16 1024 + q; a
    // high nibble left in place (bits 4..7, q << 4) under 0x5400 is 64 + q
    // (mantissa step 1/16 at 64).  Both are exact, so subtracting 1032 / 72
    // gives q - 8 exactly, and one mask-or per pair (a shift per two pairs)
    // replaces the masks, shift and byte permutes.
    const h2 blo = {(h16)-1032.0f, (h16)-1032.0f}, bhi = {(h16)-72.0f, (h16)-72.0f};
    const uint32_t s = w >> 8;
    out[0] = (as_h2(and_or(w, 0x000F000Fu, 0x64006400u)) + blo) * dd;
    out[1] = (as_h2(and_or(s, 0x000F000Fu, 0x64006400u)) + blo) * dd;
    out[2] = (as_h2(and_or(w, 0x00F000F0u, 0x54005400u)) + bhi) * dd;
    out[3] = (as_h2(and_or(s, 0x00F000F0u, 0x54005400u)) + bhi) * dd;
}

// Q8_0: four int8 (e0..e3) -> (e0,e2) (e1,e3).
__device__ __forceinline__ void q8_unpack(uint32_t w, h2 dd, h2 out[2]) {
    const h2 bias = {(h16)-1152.0f, (h16)-1152.0f};
    const uint32_t k = 0x64646464u;
    const uint32_t v = w ^ 0x80808080u;
    out[0] = (as_h2(__builtin_amdgcn_perm(k, v, 0x04020400u)) + bias) * dd;
    out[1] = (as_h2(__builtin_amdgcn_perm(k, v, 0x04030401u)) + bias) * dd;
}

__device__ __forceinline__ float fdot2(h2 a, h2 b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations (lgkmcnt) and meets the other waves, without the vmcnt(0) a
// full __syncthreads() fence adds -- global loads issued before it (a
// GEMV's weight rows) stay in flight.  The "memory" clobber keeps the
// compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Cross-lane data movement within rows of 16 lanes by DPP (no LDS round
// trip): quad_perm xor 1 (0xB1), quad_perm xor 2 (0x4E), row_half_mirror
// (0x141: lane i <-> 7 - i of each 8), row_mirror (0x140: i <-> 15 - i).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of 8 lanes, left in every lane of the group.
// Every step adds a symmetric pair, so all lanes hold the same value.
__device__ __forceinline__ float group8_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    return v;
}

// Sum over the lanes of a wave that share (lane & 7): lanes l, l+8, ...,
// l+56, the same value in all eight (row_ror:8 within each row of 16, then
// the rows by two xor shuffles).
__device__ __forceinline__ float stride8_sum(float v) {
    v += dpp_f<0x128>(v);   // row_ror:8
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// Sum over the 64-lane wave, the same value in every lane (fixed order:
// quads, 8s and 16s by DPP, then the rows by two xor shuffles).
template <int W>
__device__ __forceinline__ float wave_sum(float v) {
    static_assert(W == 64, "wave64 reduction");
    v = group8_sum(v);
    v += dpp_f<0x140>(v);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// Single-barrier workgroup max / sum: the caller must not write `red` again
// before another barrier (use one array per reduction).  The barrier also
// publishes every LDS write made before the call.
template <int NWV>
__device__ __forceinline__ float block_max1(float v, float* red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int k = 1; k < NWV; k++) t = fmaxf(t, red[k]);
    return t;
}
template <int NWV>
__device__ __forceinline__ float block_sum1(float v, float* red) {
    v = wave_sum<64>(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int k = 1; k < NWV; k++) t += red[k];
    return t;
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

// ---------------------------------------------------------------------------
// Buffer loads (out-of-range offsets read zeros without a memory access) and
// buffer loads straight into LDS.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void* gl_lds_t;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// Buffer load to LDS at wave-uniform LDS byte address lds (+ 16 or 4 bytes
// per lane), written as assembly: the compiler then neither tracks these
// LDS writes (it would wait for every one of them before any LDS read) nor
// counts them, and the kernel waits for them itself with sk_wait_vm.  M0
// holds the LDS address (one wait state between its write and the load);
// the compiler uses M0 for nothing else in the kernels that call this.
template <int SZ>
__device__ __forceinline__ void sk_dma(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t off) {
    lds = __builtin_amdgcn_readfirstlane(lds);   // an SGPR for the "s" operand however the caller computed it
    if constexpr (SZ == 16)
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds), "v"(off), "s"(r)
                     : "memory");
    else
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(lds), "v"(off), "s"(r)
                     : "memory");
}
template <int N>
__device__ __forceinline__ void sk_wait_vm() {   // a compiler barrier for memory, unlike the builtin
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

}  // namespace tlhip
