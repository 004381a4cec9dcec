// gemv_device.hpp -- device code of the fused dequant-GEMV (parameter
// block, activation staging, weight loads, block dot products, epilogues and
// the GEMV kernel templates), shared by the sources that instantiate them:
// kernels_gemv.hip (repack / dequantisation, the generic GEMV launches) and
// kernels_gemv_norm.hip (normalised GEMVs specialised on their epilogue).
//
// y[m, n] = sum_k x[m, k] * W[n, k], W stored packed (Q4_0 / Q8_0) or f16.
// The arithmetic is the reference's: every weight is first rounded to f16
// exactly as dequantize_q4_0 / dequantize_q8_0 produce it (gguf.rs:22-112:
// RNE_f16((q - 8) * d) and RNE_f16(q * d)), here with one packed f16
// multiply (v_pk_mul_f16, correctly rounded), then multiplied by the f16
// activation and accumulated in fp32 (v_dot2_f32_f16), as
// matmul_transposed_b_tiled_32x32_f16 accumulates (unified.metal:4291-4348).
//
// Work mapping: one wavefront owns RI consecutive output rows.  Lane l reads
// block l, l+64, ... of each row with one 16-byte load per block (Q4_0: the
// 16 nibble bytes; Q8_0: 2 loads; f16: 4 loads), so a wave's loads for one
// row are one contiguous stretch of the row.  All loads for the RI rows are
// issued before any arithmetic (bytes in flight per lane = RI*NB*16).  The
// activation chunk a lane needs is the same for every row, so it is loaded
// once and kept in registers, pre-permuted into the pair order the nibble
// unpacking produces.  Partial sums are reduced across the wave with xor
// shuffles; lane 0 applies the epilogue.
#pragma once
#include "device_common.hpp"
#include "internal.hpp"

namespace tlhip {

// Q6_K group -> 16 f16 pairs in element order.  The six-bit codes u are
// rebuilt four at a time as bytes (low nibbles from q4, bits 4-5 from q2),
// placed under the f16 exponent byte 0x64 (1024 + u) and shifted by -1056
// to u - 32, exactly; d * sc * (u - 32) needs at most 23 significant bits,
// so one f32 product and one f16 rounding give the reference's value.
// Pair order: out[2t], out[2t+1] = elements (4t, 4t+2), (4t+1, 4t+3) for
// t < 4 (low nibbles), the same for elements 16.. in out[8..15].
__device__ __forceinline__ void q6k_unpack(const u4& q4, uint32_t q2lo, uint32_t q2hi, float ds0, float ds1,
                                           h2 (&out)[16]) {
    const h2 bias = {(h16)-1056.0f, (h16)-1056.0f};
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t lo = (q4[t] & 0x0F0F0F0Fu) | (((q2lo >> (2 * t)) << 4) & 0x30303030u);
        const uint32_t hi = ((q4[t] >> 4) & 0x0F0F0F0Fu) | (((q2hi >> (2 * t)) << 4) & 0x30303030u);
        const h2 a0 = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04020400u)) + bias;
        const h2 a1 = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04030401u)) + bias;
        const h2 b0 = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04020400u)) + bias;
        const h2 b1 = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04030401u)) + bias;
        out[2 * t] = h2{(h16)(ds0 * (float)a0[0]), (h16)(ds0 * (float)a0[1])};
        out[2 * t + 1] = h2{(h16)(ds0 * (float)a1[0]), (h16)(ds0 * (float)a1[1])};
        out[8 + 2 * t] = h2{(h16)(ds1 * (float)b0[0]), (h16)(ds1 * (float)b0[1])};
        out[8 + 2 * t + 1] = h2{(h16)(ds1 * (float)b1[0]), (h16)(ds1 * (float)b1[1])};
    }
}

// ---------------------------------------------------------------------------
// GEMV
// ---------------------------------------------------------------------------
struct GemvParams {
    const uint16_t* x;
    const uint8_t* wq;
    const uint16_t* wd;
    const uint16_t* bias;
    const uint16_t* resid;
    uint16_t* y;
    int M, N, K, ldy, epi;
    // fused normalisation prologue (M = 1)
    const uint16_t* norm_w;
    const uint16_t* norm_b;
    float eps;
    // EPI_QKV_ROPE
    int nq, nk, head_dim, rot, layout, pos0;
    const float* rope_tab;
    const int32_t* d_pos;
    uint16_t* q_out;
    uint16_t* kc;
    uint16_t* vc;
    // normalised GEMV: x row = embd[*d_token] (written to x_out by workgroup 0)
    const uint16_t* embd;
    const int32_t* d_token;
    uint16_t* x_out;
    // normalised GEMV (QKV epilogue): the f16 normalised row, written by
    // workgroup 0 for a later GEMV of the same normalisation
    uint16_t* xn_out;
    // EPI_ARGMAX: per-workgroup (value, index) keys
    unsigned long long* amax_slots;
    // LayerNorm prologue (QKV and greedy-key epilogues): the row is
    // f16(x + x_add) -- the residual stream's last addition, made here --
    // and workgroup 0 writes that sum to x_out
    const uint16_t* x_add;
};

// Fourth word of a raw buffer resource descriptor on gfx9-family GPUs
// (gfx950 included): 32-bit data format, no swizzle, no stride; with it a
// buffer load range-checks its offset against the descriptor's byte count
// and returns zeros past it.
constexpr int BUF_RSRC_WORD3 = 0x00020000;

// Cache-policy bits of a load: the instruction's nt (non-temporal) bit on
// gfx950.
constexpr int CP_STREAM = 2;

// 0 in a VGPR the compiler cannot see through: indexing a uniform address
// with it makes the load a vector load (in-order completion) instead of a
// scalar one.
__device__ __forceinline__ int opaque_zero() {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return z;
}

// Every field of the parameter block in SGPRs before anything else runs.
// Left alone, the compiler requests kernel-argument words lazily, next to
// their first use, and a wait for one scalar load is a wait for all of them
// (they return out of order), so the fields used behind a branch or after
// the first loads cost a further round trip each before the weight loads
// go out.  An empty asm that takes them all as SGPR operands makes the
// compiler issue every kernel-argument load at once and wait once.
__device__ __forceinline__ void kernarg_fence(const GemvParams& p) {
    asm volatile("" ::"s"(p.x), "s"(p.wq), "s"(p.wd), "s"(p.bias), "s"(p.resid), "s"(p.y), "s"(p.M), "s"(p.N),
                 "s"(p.K), "s"(p.ldy), "s"(p.epi), "s"(p.norm_w), "s"(p.norm_b), "s"(p.eps), "s"(p.nq), "s"(p.nk),
                 "s"(p.head_dim), "s"(p.rot), "s"(p.layout), "s"(p.pos0), "s"(p.rope_tab), "s"(p.d_pos),
                 "s"(p.q_out), "s"(p.kc), "s"(p.vc), "s"(p.embd), "s"(p.d_token), "s"(p.x_out), "s"(p.xn_out), "s"(p.amax_slots),
                 "s"(p.x_add));
    __builtin_amdgcn_sched_barrier(0);   // nothing that uses them moves above
}

// Activation pair order of a weight type: Q6_K unpacks in the Q4_0 order.
template <int WT>
constexpr bool xo_nibble() { return WT == TLHIP_Q4_0 || WT == TLHIP_Q6_K; }

// 32 consecutive f16 activations as 16 natural pairs xw[i] = (x2i, x2i+1).
__device__ __forceinline__ void load_x32(const uint16_t* __restrict__ xb, uint32_t xw[16]) {
    const u4* p = (const u4*)xb;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        u4 t = p[v];
        xw[4 * v + 0] = t[0]; xw[4 * v + 1] = t[1]; xw[4 * v + 2] = t[2]; xw[4 * v + 3] = t[3];
    }
}

// Per-block activation chunk in the pair order of the unpacking:
//   Q4_0 (16 pairs): [4t+0]=(x4t,x4t+2) [4t+1]=(x4t+1,x4t+3)
//                    [4t+2]=(x16+4t,x16+4t+2) [4t+3]=(x16+4t+1,x16+4t+3)
//   Q8_0 (16 pairs): [2t+0]=(x4t,x4t+2) [2t+1]=(x4t+1,x4t+3), t < 8
//   F16  (16 pairs): natural pairs (x2i, x2i+1)
template <int WT>
__device__ __forceinline__ void order_x(const uint32_t xw[16], uint32_t xc[16]) {
    if (xo_nibble<WT>()) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            xc[4 * t + 0] = pack_lo(xw[2 * t], xw[2 * t + 1]);
            xc[4 * t + 1] = pack_hi(xw[2 * t], xw[2 * t + 1]);
            xc[4 * t + 2] = pack_lo(xw[8 + 2 * t], xw[8 + 2 * t + 1]);
            xc[4 * t + 3] = pack_hi(xw[8 + 2 * t], xw[8 + 2 * t + 1]);
        }
    } else if (WT == TLHIP_Q8_0) {
#pragma unroll
        for (int t = 0; t < 8; t++) {
            xc[2 * t + 0] = pack_lo(xw[2 * t], xw[2 * t + 1]);
            xc[2 * t + 1] = pack_hi(xw[2 * t], xw[2 * t + 1]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) xc[i] = xw[i];
    }
}

template <int WT>
__device__ __forceinline__ void load_xchunk(const uint16_t* __restrict__ xb, uint32_t xc[16]) {
    uint32_t xw[16];
    load_x32(xb, xw);
    order_x<WT>(xw, xc);
}

// Quad v (8 activations) of block b as four f16 pairs, for the plain GEMV's
// LDS staging (xs[v][b] = 16 bytes in the pair order of the unpacking):
// elements {4v..4v+3, 16+4v..16+4v+3} for Q4_0 / Q6_K, {8v..8v+7} otherwise.
template <int WT>
__device__ __forceinline__ void load_quad_words(const uint16_t* __restrict__ src, int b, int v, uint32_t w[4]) {
    if (xo_nibble<WT>()) {
        const uint2 lo = *(const uint2*)(src + (size_t)b * 32 + 4 * v);
        const uint2 hi = *(const uint2*)(src + (size_t)b * 32 + 16 + 4 * v);
        w[0] = lo.x; w[1] = lo.y; w[2] = hi.x; w[3] = hi.y;
    } else {
        const u4 t = *(const u4*)(src + (size_t)b * 32 + 8 * v);
        w[0] = t[0]; w[1] = t[1]; w[2] = t[2]; w[3] = t[3];
    }
}

// Sum over the workgroup's WPB waves in a fixed order, with ONE barrier:
// the caller must not write `red` again before another barrier.
template <int WPB>
__device__ __forceinline__ float wg_sum1(float v, float* red) {
    v = wave_sum<64>(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    float t = red[0];
#pragma unroll
    for (int k = 1; k < WPB; k++) t += red[k];
    return t;
}

// Activation staging for the normalised GEMV (M = 1).  The workgroup loads
// the row once, forms the row statistics, normalises with exactly the
// formulas and f16 store of rms_norm_kernel / layer_norm_kernel
//   RMS: y = f16((x * (1 / sqrt(mean(x^2) + eps))) * w)
//   LN:  y = f16(((x - mean) * (1 / sqrt(var + eps))) * w + b)
// and leaves it in LDS already in the pair order of the unpacking.  LDS is
// quad-major, xs[v][b] = 16 bytes (pairs 4v..4v+3 of block b's chunk), so
// lane l's reads of block l are consecutive 16-byte words (no conflicts).
// Quad v of a block holds elements {4v..4v+3, 16+4v..16+4v+3} for Q4_0 /
// Q6_K and {8v..8v+7} for Q8_0 / f16; thread t holds quads t, t + NT, ...
// (8 activations each, so the loads and the statistics spread over four
// waves of a K = 2048 row).  The loads go through range-checked buffer
// descriptors: a quad past the row reads zeros with no memory request, so
// there is neither a branch (whose join would make the compiler wait for
// the loads before the weight rows go out) nor a duplicate read.  They are
// issued before the weight rows (vector loads retire in order), so the
// statistics start while the weights are still in flight.
template <int WT>
__device__ __forceinline__ int quad_elem(int v, int e) {
    return xo_nibble<WT>() ? (e < 4 ? 4 * v + e : 12 + 4 * v + e) : 8 * v + e;
}

template <int WT>
__device__ __forceinline__ u4 pack_quad(const float f[8]) {
    uint32_t w[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        h2 h;
        h[0] = (h16)f[2 * t];
        h[1] = (h16)f[2 * t + 1];
        w[t] = as_u32(h);
    }
    if (WT == TLHIP_F16) return u4{w[0], w[1], w[2], w[3]};
    return u4{pack_lo(w[0], w[1]), pack_hi(w[0], w[1]), pack_lo(w[2], w[3]), pack_hi(w[2], w[3])};
}

// Q8_0 in the one-row GEMVs (load_rows_buf, load_flat and their dots): a
// lane's two 16-byte words are halves of two blocks, so that each load
// instruction reads 1 KB of consecutive bytes -- whole 128-byte lines -- and
// can be non-temporal.  Word l of pass i holds half (lane & 1) of block
// 64 i + 32 l + (lane >> 1) of the lane's row (or flat task stream), i.e.
// bytes 16 * (128 i + 64 l + lane) of it; each word has its own scale.
// (With both halves of block lane + 64 i in one lane, each instruction
// covers every other 16 bytes and the second relies on the line the first
// brought into L2, which a non-temporal load does not keep.)
template <int WT>
constexpr bool half_slots() { return WT == TLHIP_Q8_0; }
template <int WT>
constexpr int ds_per() { return half_slots<WT>() ? 2 : 1; }
// Block of word l of pass i (half_slots) in a lane's row or task stream.
__device__ __forceinline__ int half_block(int i, int l, int lane) { return 64 * i + 32 * l + (lane >> 1); }

// Index into the activation staging (u4 xs[4][NB * 64], taken flat) of quad v
// of block b: quad-major (xs[v][b]; lane l's reads of block l are
// consecutive 16-byte words) or, for half_slots, block-major (lane pairs
// read the two halves of one block: consecutive 32-byte pieces).
template <int WT, int NB>
__device__ __forceinline__ int xs_at(int b, int v) { return half_slots<WT>() ? b * 4 + v : v * (NB * 64) + b; }

// The staged activation chunks of a block (16 pairs in the pair order of
// WT's unpacking) or of half of one (pairs 8h .. 8h + 7).
template <int WT, int NB>
struct XsChunk {
    const u4* xs;
    __device__ __forceinline__ void operator()(int b, uint32_t (&xc)[16]) const {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const u4 t = xs[xs_at<WT, NB>(b, v)];
            xc[4 * v] = t[0]; xc[4 * v + 1] = t[1]; xc[4 * v + 2] = t[2]; xc[4 * v + 3] = t[3];
        }
    }
    __device__ __forceinline__ void half(int b, int h, uint32_t (&xc)[8]) const {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const u4 t = xs[xs_at<WT, NB>(b, 2 * h + j)];
            xc[4 * j] = t[0]; xc[4 * j + 1] = t[1]; xc[4 * j + 2] = t[2]; xc[4 * j + 3] = t[3];
        }
    }
};

template <int WT, int NB, int WPB, int PRO>
struct NormStage {
    static constexpr int NT = WPB * 64;
    static constexpr int IPT = (NB * 256 + NT - 1) / NT;
    uint32_t xw[IPT][4], ww[IPT][4], bw[IPT][4];   // raw f16 pairs until finish()
    uint32_t aw[IPT][4];   // LayerNorm with x_add: the added row
    uint32_t xn[IPT][4];   // the normalised quads in natural element order (for xn_out)

    __device__ __forceinline__ static void load_buf(const uint16_t* __restrict__ src, int K, int it, uint32_t w[4]) {
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, K * 2, BUF_RSRC_WORD3);
        const int b = it >> 2, v = it & 3;
        if (xo_nibble<WT>()) {
            const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (b * 32 + 4 * v) * 2, 0, 0));
            const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (b * 32 + 16 + 4 * v) * 2, 0, 0));
            w[0] = lo.x; w[1] = lo.y; w[2] = hi.x; w[3] = hi.y;
        } else {
            const u4 t = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, (b * 32 + 8 * v) * 2, 0, 0));
            w[0] = t[0]; w[1] = t[1]; w[2] = t[2]; w[3] = t[3];
        }
    }

    __device__ __forceinline__ static void to_float(const uint32_t w[4], float f[8]) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const h2 h = as_h2(w[t]);
            f[2 * t] = (float)h[0];
            f[2 * t + 1] = (float)h[1];
        }
    }

    __device__ __forceinline__ void load(const GemvParams& p, const uint16_t* __restrict__ xsrc) {
#pragma unroll
        for (int k = 0; k < IPT; k++) {
            const int it = threadIdx.x + k * NT;
            load_buf(xsrc, p.K, it, xw[k]);
            load_buf(p.norm_w, p.K, it, ww[k]);
            if (PRO == PRO_LN) load_buf(p.norm_b, p.K, it, bw[k]);
            if (PRO == PRO_LN && p.x_add) load_buf(p.x_add, p.K, it, aw[k]);
        }
    }

    // Workgroup 0 writes the normalised row to xn_out, after its own work:
    // stores issued before the dot products would sit in the same in-order
    // counter as the weight loads the products wait for.  Natural element
    // order: one 16-byte store per quad (Q4_0's quad halves: two 8-byte ones).
    __device__ __forceinline__ void store_xn(const GemvParams& p) const {
        if (!p.xn_out || blockIdx.x != 0) return;
        const int items = (p.K >> 5) * 4;
#pragma unroll
        for (int k = 0; k < IPT; k++) {
            const int it = threadIdx.x + k * NT;
            if (it >= items) continue;
            const int b = it >> 2, v = it & 3;
            uint16_t* dst = p.xn_out + (size_t)b * 32;
            if (xo_nibble<WT>()) {
                *(uint2*)(dst + 4 * v) = uint2{xn[k][0], xn[k][1]};
                *(uint2*)(dst + 16 + 4 * v) = uint2{xn[k][2], xn[k][3]};
            } else {
                *(u4*)(dst + 8 * v) = u4{xn[k][0], xn[k][1], xn[k][2], xn[k][3]};
            }
        }
    }

    __device__ __forceinline__ void finish(const GemvParams& p, u4 (*xs)[NB * 64], float (*red)[WPB]) {
        const int items = (p.K >> 5) * 4;
        float f[IPT][8];
#pragma unroll
        for (int k = 0; k < IPT; k++) to_float(xw[k], f[k]);   // (quads past the row read zeros)
        if (PRO == PRO_LN && p.x_add)
#pragma unroll
            for (int k = 0; k < IPT; k++) {
                float g[8];
                to_float(aw[k], g);
#pragma unroll
                for (int e = 0; e < 8; e++) f[k][e] = h2f(f2h(f[k][e] + g[e]));   // the residual's f16 add
            }
        if (p.x_out && blockIdx.x == 0)   // the residual copy of an embedded or summed row
#pragma unroll
            for (int k = 0; k < IPT; k++) {
                const int it = threadIdx.x + k * NT;
                if (it < items) {
                    const int b = it >> 2, v = it & 3;
#pragma unroll
                    for (int e = 0; e < 8; e++) p.x_out[(size_t)b * 32 + quad_elem<WT>(v, e)] = f2h(f[k][e]);
                }
            }
        float mean = 0.0f, inv;
        if (PRO == PRO_RMS) {
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < IPT; k++)
#pragma unroll
                for (int e = 0; e < 8; e++) ss += f[k][e] * f[k][e];
            inv = 1.0f / sqrtf(wg_sum1<WPB>(ss, red[0]) / (float)p.K + p.eps);
        } else {
            float sm = 0.0f;
#pragma unroll
            for (int k = 0; k < IPT; k++)
#pragma unroll
                for (int e = 0; e < 8; e++) sm += f[k][e];
            mean = wg_sum1<WPB>(sm, red[0]) / (float)p.K;
            float q = 0.0f;
#pragma unroll
            for (int k = 0; k < IPT; k++) {
                if ((int)threadIdx.x + k * NT >= items) continue;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float d = f[k][e] - mean;
                    q += d * d;
                }
            }
            inv = 1.0f / sqrtf(wg_sum1<WPB>(q, red[1]) / (float)p.K + p.eps);
        }
#pragma unroll
        for (int k = 0; k < IPT; k++) {
            const int it = threadIdx.x + k * NT;
            if (it >= items) continue;
            const int b = it >> 2, v = it & 3;
            float w[8], bb[8];
            to_float(ww[k], w);
            if (PRO == PRO_LN) to_float(bw[k], bb);
#pragma unroll
            for (int e = 0; e < 8; e++)
                f[k][e] = PRO == PRO_RMS ? (f[k][e] * inv) * w[e] : (((f[k][e] - mean) * inv) * w[e]) + bb[e];
            (&xs[0][0])[xs_at<WT, NB>(b, v)] = pack_quad<WT>(f[k]);
            if (p.xn_out)   // (the same f16 values the dot products read)
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    h2 h;
                    h[0] = (h16)f[k][2 * t];
                    h[1] = (h16)f[k][2 * t + 1];
                    xn[k][t] = as_u32(h);
                }
        }
        lds_barrier();
    }

};

// Weight payload of one 32-element block: Q4_0 1 x 16 B, Q8_0 2 x 16 B, F16 4 x 16 B.
// 16-byte words a lane holds per 32-element block: Q4_0 the 16 nibble bytes;
// Q8_0 the 32 int8; f16 the 32 values; Q6_K the 16 q4 bytes, then
// {q2 word 0, q2 word 1, sc pair | d << 16, 0}.
template <int WT> struct BlkLoads {
    static constexpr int n = WT == TLHIP_Q4_0 ? 1 : (WT == TLHIP_Q8_0 || WT == TLHIP_Q6_K ? 2 : 4);
};

// Cache policy of the one-row GEMVs' weight loads.  Q4_0 and Q8_0 rows are
// read non-temporally: each is read once per pass, and every load
// instruction covers whole 128-byte lines (16 bytes per lane, consecutive
// lanes; Q8_0 through half_slots).  Measured on MI355X (A/B of library
// builds on one box, same tokens): config-4 decode under graph replay
// 1985 -> 2181 tok/s; under the profiler's serialised launches the GEMV
// durations are unchanged and the decode attention 5.05 -> 4.60 us per
// layer, so most of the gain is at the kernel boundaries; the Q4_0
// [5632 x 2048] GEMV alone over 48 rotating weight copies is unchanged
// (3.52 vs 3.51 us).  Phi-2 (Q8_0) decode 1065 -> 1114 tok/s with
// half_slots; with Q8_0's earlier layout (both words of a block in one
// lane, each instruction covering every other 16 bytes) non-temporal loads
// lost 1050 -> 1002 tok/s.  Q6_K's planes are read the same way (16, 8
// and 2 bytes per lane, consecutive lanes).  f16 rows (64 bytes per lane)
// keep plain loads.
template <int WT>
constexpr int weight_cp() { return WT == TLHIP_F16 ? 0 : CP_STREAM; }

template <int WT>
__device__ __forceinline__ float block_dot(const u4* q, uint32_t dbits, const uint32_t xc[16], float acc) {
    if (WT == TLHIP_Q4_0) {
        h16 dh = __builtin_bit_cast(h16, (uint16_t)dbits);
        h2 dd = {dh, dh};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            h2 r[4];
            q4_unpack(q[0][t], dd, r);
#pragma unroll
            for (int j = 0; j < 4; j++) acc = fdot2(r[j], as_h2(xc[4 * t + j]), acc);
        }
    } else if (WT == TLHIP_Q6_K) {
        const uint32_t sw = q[1][2];
        const float dv = h2f((uint16_t)(sw >> 16));
        h2 r[16];
        q6k_unpack(q[0], q[1][0], q[1][1], dv * (float)(int8_t)(sw & 0xff), dv * (float)(int8_t)((sw >> 8) & 0xff), r);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            acc = fdot2(r[2 * t], as_h2(xc[4 * t + 0]), acc);
            acc = fdot2(r[2 * t + 1], as_h2(xc[4 * t + 1]), acc);
            acc = fdot2(r[8 + 2 * t], as_h2(xc[4 * t + 2]), acc);
            acc = fdot2(r[8 + 2 * t + 1], as_h2(xc[4 * t + 3]), acc);
        }
    } else if (WT == TLHIP_Q8_0) {
        h16 dh = __builtin_bit_cast(h16, (uint16_t)dbits);
        h2 dd = {dh, dh};
#pragma unroll
        for (int v = 0; v < 2; v++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                h2 r[2];
                q8_unpack(q[v][t], dd, r);
                acc = fdot2(r[0], as_h2(xc[8 * v + 2 * t + 0]), acc);
                acc = fdot2(r[1], as_h2(xc[8 * v + 2 * t + 1]), acc);
            }
    } else {
#pragma unroll
        for (int v = 0; v < 4; v++)
#pragma unroll
            for (int t = 0; t < 4; t++) acc = fdot2(as_h2(q[v][t]), as_h2(xc[4 * v + t]), acc);
    }
    return acc;
}

// Q8_0 half block: 16 int8 (one 16-byte word) against pairs 8h .. 8h + 7 of
// the block's activation chunk -- block_dot's arithmetic for one of its two
// words.
__device__ __forceinline__ float q8_half_dot(const u4& q, uint32_t dbits, const uint32_t xc[8], float acc) {
    h16 dh = __builtin_bit_cast(h16, (uint16_t)dbits);
    h2 dd = {dh, dh};
#pragma unroll
    for (int t = 0; t < 4; t++) {
        h2 r[2];
        q8_unpack(q[t], dd, r);
        acc = fdot2(r[0], as_h2(xc[2 * t + 0]), acc);
        acc = fdot2(r[1], as_h2(xc[2 * t + 1]), acc);
    }
    return acc;
}


// Fused projection epilogue for rows (row, row + 1) of the stacked
// [q | k | v] weight (M = 1, decode or one prefill row): the linear's f16
// store (+ bias), then RoPE on q and k at position pos (rope_kernel's
// arithmetic) written to q_out and the K cache, V copied to the V cache --
// linear + rope + Cache::update of the reference's program in one store.
// Rows of a head are in pair order: pair i is (row 2i, row 2i + 1), which is
// the natural order for the interleaved layout and a load-time permutation
// of the rows for the half-rotation (NeoX) layout; dims >= rot pass through.
// The bias pair, the position and the pair's (cos, sin) were loaded at the
// start of the kernel (QkvPre), so the tail makes no dependent loads.
struct QkvPre {
    int pos;
    uint32_t b01;   // f16 bits of bias[row] (low half) and bias[row + 1]
    float c, sn;
};

__device__ __forceinline__ void qkv_rope_pre(const GemvParams& p, int row, int pos, QkvPre& q) {
    q.pos = pos;
    // one 4-byte load (row is even), split only at the store, so no wait here
    q.b01 = p.bias ? *(const uint32_t*)(p.bias + row) : 0u;
    q.c = 1.0f;
    q.sn = 0.0f;
    const int D = p.head_dim;
    int e = -1;
    if (row < p.nq) e = row % D;
    else if (row < p.nq + p.nk) e = (row - p.nq) % D;
    if (e >= 0 && e < p.rot) {
        const int half = p.rot >> 1, i = e >> 1;
        q.c = p.rope_tab[2 * ((size_t)pos * half + i)];
        q.sn = p.rope_tab[2 * ((size_t)pos * half + i) + 1];
    }
}

__device__ __forceinline__ void qkv_rope_store(const GemvParams& p, int row, float a0, float a1, const QkvPre& q) {
    uint16_t r0 = f2h(a0), r1 = f2h(a1);
    if (p.bias) {
        r0 = add_h(r0, (uint16_t)(q.b01 & 0xffffu));
        r1 = add_h(r1, (uint16_t)(q.b01 >> 16));
    }
    const int pos = q.pos;
    const int D = p.head_dim;
    uint16_t* dst;
    int e;
    if (row < p.nq) {
        dst = p.q_out + (size_t)(row / D) * D;
        e = row % D;
    } else if (row < p.nq + p.nk) {
        const int c = row - p.nq;
        dst = p.kc + (size_t)pos * p.nk + (size_t)(c / D) * D;
        e = c % D;
    } else {
        const int c = row - p.nq - p.nk;
        p.vc[(size_t)pos * p.nk + c] = r0;
        p.vc[(size_t)pos * p.nk + c + 1] = r1;
        return;
    }
    if (e < p.rot) {
        const int half = p.rot >> 1, i = e >> 1;
        const float x0 = h2f(r0), x1 = h2f(r1);
        const float o0 = __fsub_rn(__fmul_rn(x0, q.c), __fmul_rn(x1, q.sn));
        const float o1 = __fadd_rn(__fmul_rn(x0, q.sn), __fmul_rn(x1, q.c));
        const int i0 = p.layout ? i : 2 * i, i1 = p.layout ? i + half : 2 * i + 1;
        dst[i0] = f2h(o0);
        dst[i1] = f2h(o1);
    } else {
        dst[e] = r0;
        dst[e + 1] = r1;
    }
}

// Loads of RI rows x NB blocks of the wave, all issued before any use.
template <int WT, int NB, int RI>
__device__ __forceinline__ void load_rows(const GemvParams& p, int row0, int lane, u4 (&q)[RI][NB][BlkLoads<WT>::n],
                                          uint32_t (&ds)[RI][NB]) {
    constexpr int NL = BlkLoads<WT>::n;
    const int nbr = p.K >> 5;
    if (WT == TLHIP_Q6_K) {
        const uint8_t* q2 = p.wq + q6k_q2_offset(p.N, p.K);
        const uint8_t* sc = p.wq + q6k_sc_offset(p.N, p.K);
#pragma unroll
        for (int ri = 0; ri < RI; ri++) {
            const int row = min(row0 + ri, p.N - 1);
#pragma unroll
            for (int i = 0; i < NB; i++) {
                const int b = min(lane + 64 * i, nbr - 1);
                q[ri][i][0] = *(const u4*)(p.wq + (size_t)row * (p.K / 2) + (size_t)b * 16);
                const uint2 h = *(const uint2*)(q2 + (size_t)row * (p.K / 4) + (size_t)b * 8);
                const uint32_t s2 = *(const uint16_t*)(sc + (size_t)row * (p.K / 16) + (size_t)b * 2);
                const uint32_t dv = p.wd[(size_t)row * (p.K / 256) + b / 8];
                q[ri][i][1] = u4{h.x, h.y, s2 | (dv << 16), 0u};
                ds[ri][i] = 0u;
            }
        }
        return;
    }
    const size_t row_bytes = WT == TLHIP_Q4_0 ? (size_t)p.K / 2 : (WT == TLHIP_Q8_0 ? (size_t)p.K : (size_t)p.K * 2);
#pragma unroll
    for (int ri = 0; ri < RI; ri++) {
        const int row = min(row0 + ri, p.N - 1);
        const uint8_t* wr = p.wq + (size_t)row * row_bytes;
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int b = min(lane + 64 * i, nbr - 1);
#pragma unroll
            for (int l = 0; l < NL; l++) q[ri][i][l] = *(const u4*)(wr + (size_t)b * (16 * NL) + 16 * l);
            ds[ri][i] = WT == TLHIP_F16 ? 0u : (uint32_t)p.wd[(size_t)row * nbr + b];
        }
    }
}

// load_rows through range-checked buffer loads.  row0 must be wave-uniform:
// every row base is then a scalar address (one descriptor per row and
// stream, built by the scalar unit), each lane's offset is a 32-bit
// multiple of its block index, and a block past the row (lane + 64 i >=
// K / 32) reads zero bytes and a zero scale -- a zero weight -- with no
// memory request and no clamp.  Rows past N are clamped to the last row.
// What this saves is the per-lane 64-bit address arithmetic load_rows
// issues before its first weight load; on MI355X that delay, repeated for
// every wave a SIMD holds, cost 0.2-0.3 us of a 4 us GEMV.
// AUX: the loads' cache-policy bits (weight_cp).
template <int WT, int NB, int RI, int AUX>
__device__ __forceinline__ void load_rows_buf_cp(const uint8_t* wq, const uint16_t* wd, int N, int K, int row0, int lane,
                                                 u4 (&q)[RI][NB][BlkLoads<WT>::n], uint32_t (&ds)[RI][NB * ds_per<WT>()]) {
    constexpr int NL = BlkLoads<WT>::n;
    const int nbr = K >> 5;
    if (WT == TLHIP_Q6_K) {
        const uint8_t* q2 = wq + q6k_q2_offset(N, K);
        const uint8_t* sc = wq + q6k_sc_offset(N, K);
#pragma unroll
        for (int ri = 0; ri < RI; ri++) {
            const size_t row = (size_t)min(row0 + ri, N - 1);
            const __amdgpu_buffer_rsrc_t r4 = __builtin_amdgcn_make_buffer_rsrc((void*)(wq + row * (K / 2)), (short)0, K / 2, BUF_RSRC_WORD3);
            const __amdgpu_buffer_rsrc_t r2 = __builtin_amdgcn_make_buffer_rsrc((void*)(q2 + row * (K / 4)), (short)0, K / 4, BUF_RSRC_WORD3);
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)(sc + row * (K / 16)), (short)0, K / 16, BUF_RSRC_WORD3);
            const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc((void*)(wd + row * (K / 256)), (short)0, K / 128, BUF_RSRC_WORD3);
#pragma unroll
            for (int i = 0; i < NB; i++) {
                const int b = lane + 64 * i;
                q[ri][i][0] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r4, b * 16, 0, AUX));
                const uint2 h = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r2, b * 8, 0, AUX));
                const uint32_t s2 = __builtin_amdgcn_raw_buffer_load_b16(rs, b * 2, 0, AUX);
                const uint32_t dv = __builtin_amdgcn_raw_buffer_load_b16(rd, (b >> 3) * 2, 0, AUX);
                q[ri][i][1] = u4{h.x, h.y, s2 | (dv << 16), 0u};
                ds[ri][i] = 0u;
            }
        }
        return;
    }
    const int row_bytes = WT == TLHIP_Q4_0 ? K / 2 : (WT == TLHIP_Q8_0 ? K : K * 2);
#pragma unroll
    for (int ri = 0; ri < RI; ri++) {
        const size_t row = (size_t)min(row0 + ri, N - 1);
        const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)(wq + row * row_bytes), (short)0, row_bytes, BUF_RSRC_WORD3);
        const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc((void*)(wd + row * nbr), (short)0,
                                                                            WT == TLHIP_F16 ? 0 : nbr * 2, BUF_RSRC_WORD3);
#pragma unroll
        for (int i = 0; i < NB; i++) {
            if constexpr (half_slots<WT>()) {
#pragma unroll
                for (int l = 0; l < 2; l++) {
                    q[ri][i][l] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rq, 16 * (128 * i + 64 * l + lane), 0, AUX));
                    ds[ri][2 * i + l] = __builtin_amdgcn_raw_buffer_load_b16(rd, half_block(i, l, lane) * 2, 0, AUX);
                }
                continue;
            }
            const int b = lane + 64 * i;
#pragma unroll
            for (int l = 0; l < NL; l++)
                q[ri][i][l] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rq, b * (16 * NL) + 16 * l, 0, AUX));
            ds[ri][i] = WT == TLHIP_F16 ? 0u : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rd, b * 2, 0, AUX);
        }
    }
}

template <int WT, int NB, int RI>
__device__ __forceinline__ void load_rows_buf(const uint8_t* wq, const uint16_t* wd, int N, int K, int row0, int lane,
                                              u4 (&q)[RI][NB][BlkLoads<WT>::n], uint32_t (&ds)[RI][NB * ds_per<WT>()]) {
    load_rows_buf_cp<WT, NB, RI, weight_cp<WT>()>(wq, wd, N, K, row0, lane, q, ds);
}

// Lane 0's bias / residual elements of the wave's rows, loaded right after
// the weights so the epilogue makes no dependent loads.
template <int RI, int MX>
struct EpiPre {   // zero-extended f16 bits (kept unpacked until the epilogue)
    uint32_t b[RI];
    uint32_t r[RI][MX];
};

template <int RI, int MX>
__device__ __forceinline__ void epi_preload(const GemvParams& p, int row0, EpiPre<RI, MX>& e) {
#pragma unroll
    for (int ri = 0; ri < RI; ri++) {
        const int row = min(row0 + ri, p.N - 1);
        e.b[ri] = p.bias ? (uint32_t)p.bias[row] : 0u;
#pragma unroll
        for (int m = 0; m < MX; m++) e.r[ri][m] = (p.resid && m < p.M) ? (uint32_t)p.resid[(size_t)m * p.N + row] : 0u;
    }
}

// Lane 0's stores of the wave's RI reduced rows (m = activation row).
template <int RI, int MX>
__device__ __forceinline__ void store_rows(const GemvParams& p, int row0, const float (&acc)[RI][MX],
                                           const EpiPre<RI, MX>& e) {
    if (p.epi == EPI_SWIGLU_PAIR) {
        // row pairs (2i, 2i+1) = (gate_i, up_i); RI is even and row0 even
#pragma unroll
        for (int ri = 0; ri < RI; ri += 2) {
            const int row = row0 + ri;
            if (row + 1 < p.N)
#pragma unroll
                for (int m = 0; m < MX; m++)
                    if (m < p.M) p.y[(size_t)m * p.ldy + row / 2] = swiglu_h(f2h(acc[ri][m]), f2h(acc[ri + 1][m]));
        }
    } else {
#pragma unroll
        for (int ri = 0; ri < RI; ri++) {
            const int row = row0 + ri;
            if (row < p.N)
#pragma unroll
                for (int m = 0; m < MX; m++)
                    if (m < p.M) p.y[(size_t)m * p.ldy + row] = epilogue_v(p.epi, acc[ri][m], (uint16_t)e.b[ri], (uint16_t)e.r[ri][m]);
        }
    }
}

// Greedy argmax key of an f16 logit: order-preserving 16-bit image in the
// high half (NaN lowest, -0 as +0), index in the low half, so the largest
// key is the largest value and, among equal values, the largest index --
// the last maximum, as temperature_sample's max_by keeps it.
__device__ __forceinline__ unsigned long long amax_key(uint16_t h, int idx) {
    uint32_t k;
    if ((h & 0x7fffu) > 0x7c00u) k = 0u;                       // NaN
    else {
        if (h == 0x8000u) h = 0;                                // -0 == +0
        k = (h & 0x8000u) ? (~(uint32_t)h & 0xffffu) : ((uint32_t)h | 0x8000u);
    }
    return ((unsigned long long)k << 32) | (uint32_t)idx;
}

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }

// NB: blocks per lane (ceil(K/32/64)); RI: rows per wave; MX: max activation
// rows.  M = 1: the workgroup stages the activation row once in LDS, in the
// pair order of the unpacking (the layout of gemv_norm_kernel's staging,
// without the normalisation), from loads issued before the weight rows --
// vector loads retire in order, so the staging completes while the weights
// are still in flight, and the row crosses the L2 -> CU path once per
// workgroup instead of once per wave.  (Each lane loading its own blocks'
// chunks from L2 instead, with no LDS and no barrier, was measured on
// MI355X: equal or slower back to back -- 5632 x 2048 3.88-3.99 vs
// 3.82-3.88 us, 2048 x 5632 4.31-4.44 vs 3.98-4.09 us.)  M > 1: every wave
// loads its activation chunks from global memory (L2).
template <int WT, int NB, int RI, int MX>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
    __shared__ u4 xs[4][MX == 1 ? NB * 64 : 1];
    kernarg_fence(p);
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int row0 = wave * RI;
    const bool active = row0 < p.N;   // (only the last workgroup has idle waves)
    const int nbr = p.K >> 5;
    constexpr int NL = BlkLoads<WT>::n;
    uint32_t xw[MX == 1 ? NB : 1][4];
    if constexpr (MX == 1) {
        const int items = nbr * 4;
#pragma unroll
        for (int k = 0; k < NB; k++) {   // (clamped, unconditional: see load_rows below)
            const int it = min((int)threadIdx.x + 256 * k, items - 1);
            load_quad_words<WT>(p.x, it >> 2, it & 3, xw[k]);
        }
        __builtin_amdgcn_sched_barrier(0);   // keep them ahead of the weight loads
    } else if (!active) {
        return;
    }
    // (unconditional: load_rows clamps rows into the matrix, and a load under
    // a branch would make the staging below wait for every load)
    u4 q[RI][NB][NL];
    uint32_t ds[RI][NB];   // scales zero-extended: no packing that would force an early wait
    load_rows<WT, NB, RI>(p, row0, lane, q, ds);
    EpiPre<RI, MX> pre;
    if constexpr (MX != 1) {
        if (lane == 0) epi_preload<RI, MX>(p, row0, pre);
    } else {
        const int items = nbr * 4;
#pragma unroll
        for (int k = 0; k < NB; k++) {
            const int it = threadIdx.x + 256 * k;
            if (it < items) {
                const uint32_t* w = xw[k];
                xs[it & 3][it >> 2] = WT == TLHIP_F16 ? u4{w[0], w[1], w[2], w[3]}
                                                      : u4{pack_lo(w[0], w[1]), pack_hi(w[0], w[1]),
                                                           pack_lo(w[2], w[3]), pack_hi(w[2], w[3])};
            }
        }
        if (lane == 0 && active) epi_preload<RI, MX>(p, row0, pre);
        lds_barrier();
        if (!active) return;
    }

    float acc[RI][MX];
#pragma unroll
    for (int ri = 0; ri < RI; ri++)
#pragma unroll
        for (int m = 0; m < MX; m++) acc[ri][m] = 0.0f;
#pragma unroll
    for (int i = 0; i < NB; i++) {
        const int b = lane + 64 * i;
        if (b < nbr) {
#pragma unroll
            for (int m = 0; m < MX; m++) {
                if (m < p.M) {
                    uint32_t xc[16];
                    if constexpr (MX == 1) {
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            const u4 t = xs[v][b];
                            xc[4 * v] = t[0]; xc[4 * v + 1] = t[1]; xc[4 * v + 2] = t[2]; xc[4 * v + 3] = t[3];
                        }
                    } else {
                        load_xchunk<WT>(p.x + (size_t)m * p.K + (size_t)b * 32, xc);
                    }
#pragma unroll
                    for (int ri = 0; ri < RI; ri++) acc[ri][m] = block_dot<WT>(q[ri][i], ds[ri][i], xc, acc[ri][m]);
                }
            }
        }
    }
#pragma unroll
    for (int ri = 0; ri < RI; ri++)
#pragma unroll
        for (int m = 0; m < MX; m++) acc[ri][m] = wave_sum<64>(acc[ri][m]);
    if (lane == 0) store_rows<RI, MX>(p, row0, acc, pre);
}

// Activation quad `it` (block it / 4, quad it % 4) of a row through a
// range-checked buffer descriptor of the row: a quad past the row reads
// zeros with no memory request.  Pair order of gemv_kernel's staging.
template <int WT>
__device__ __forceinline__ void load_quad_buf(__amdgpu_buffer_rsrc_t r, int it, uint32_t w[4]) {
    const int b = it >> 2, v = it & 3;
    if (xo_nibble<WT>()) {
        const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (b * 32 + 4 * v) * 2, 0, 0));
        const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (b * 32 + 16 + 4 * v) * 2, 0, 0));
        w[0] = lo.x; w[1] = lo.y; w[2] = hi.x; w[3] = hi.y;
    } else {
        const u4 t = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, (b * 32 + 8 * v) * 2, 0, 0));
        w[0] = t[0]; w[1] = t[1]; w[2] = t[2]; w[3] = t[3];
    }
}

// Flat task layout (FN > 0 in the M = 1 kernels): the wave's RI consecutive
// rows taken as one contiguous stream of RI * FN blocks -- rows are
// contiguous in the packed layout, so the stream is one stretch of memory --
// and task t = lane + 64 i is block t % FN of row t / FN.  With FN blocks per
// row not a multiple of 64 the lane-per-block layout leaves lanes idle in
// the last pass (K = 2560: 80 blocks in 2 x 64 slots, 3 of 8 slots
// computing on zeros); here RI * FN / 64 tasks per lane keep every lane busy
// (4 rows of 80 blocks: 5 tasks each).  A task slot spans at most two rows
// (FN >= 64): lanes below the row boundary add into the lower row's sum, the
// others into the upper's.
template <int FN, int RI>
struct Flat {
    static_assert(FN >= 64, "a task slot spans at most two rows");
    static constexpr int IT = (RI * FN + 63) / 64;
};

// Loads of the wave's flat task stream, all issued before any use, through
// range-checked buffer loads over the rows that exist (a task past them, or
// every task of a wave past N, reads a zero weight with no memory request).
template <int WT, int FN, int RI, int AUX>
__device__ __forceinline__ void load_flat_cp(const uint8_t* wq, const uint16_t* wd, int N, int K, int row0, int lane,
                                             u4 (&q)[Flat<FN, RI>::IT][BlkLoads<WT>::n],
                                             uint32_t (&ds)[Flat<FN, RI>::IT * ds_per<WT>()]) {
    constexpr int NL = BlkLoads<WT>::n, IT = Flat<FN, RI>::IT;
    const int row_bytes = WT == TLHIP_Q4_0 ? K / 2 : (WT == TLHIP_Q8_0 ? K : K * 2);
    const int rows = row0 < N ? min(RI, N - row0) : 0;
    const size_t r0 = (size_t)min(row0, N - 1);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)(wq + r0 * row_bytes), (short)0,
                                                                        rows * row_bytes, BUF_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc((void*)(wd + r0 * FN), (short)0,
                                                                        WT == TLHIP_F16 ? 0 : rows * FN * 2, BUF_RSRC_WORD3);
#pragma unroll
    for (int i = 0; i < IT; i++) {
        if constexpr (half_slots<WT>()) {
#pragma unroll
            for (int l = 0; l < 2; l++) {
                q[i][l] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rq, 16 * (128 * i + 64 * l + lane), 0, AUX));
                ds[2 * i + l] = __builtin_amdgcn_raw_buffer_load_b16(rd, half_block(i, l, lane) * 2, 0, AUX);
            }
            continue;
        }
        const int gb = lane + 64 * i;
#pragma unroll
        for (int l = 0; l < NL; l++)
            q[i][l] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rq, gb * (16 * NL) + 16 * l, 0, AUX));
        ds[i] = WT == TLHIP_F16 ? 0u : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rd, gb * 2, 0, AUX);
    }
}

template <int WT, int FN, int RI>
__device__ __forceinline__ void load_flat(const uint8_t* wq, const uint16_t* wd, int N, int K, int row0, int lane,
                                          u4 (&q)[Flat<FN, RI>::IT][BlkLoads<WT>::n],
                                          uint32_t (&ds)[Flat<FN, RI>::IT * ds_per<WT>()]) {
    load_flat_cp<WT, FN, RI, weight_cp<WT>()>(wq, wd, N, K, row0, lane, q, ds);
}

// Half-block words (half_slots) of pass I, word L, into the row sums.
template <int WT, int FN, int RI, int I, int L, typename CH>
__device__ __forceinline__ void dot_flat_half(const u4& q, uint32_t d, const CH& chunk, int lane, float (&acc)[RI]) {
    const int gb = half_block(I, L, lane);
    const int r = gb / FN;
    uint32_t xc[8];
    chunk.half(gb - r * FN, lane & 1, xc);
    constexpr int rlo = (64 * I + 32 * L) / FN;
    constexpr int rhi = (64 * I + 32 * L + 31) / FN < RI ? (64 * I + 32 * L + 31) / FN : RI - 1;
    if constexpr (rlo >= RI) {
        return;   // (every block of the word is past the stream: zero weights)
    } else if constexpr (rlo == rhi) {
        acc[rlo] = q8_half_dot(q, d, xc, acc[rlo]);
    } else {
        const bool lo = gb < (rlo + 1) * FN;
        float c = lo ? acc[rlo] : acc[rhi];
        c = q8_half_dot(q, d, xc, c);
        acc[rlo] = lo ? c : acc[rlo];
        acc[rhi] = lo ? acc[rhi] : c;
    }
}

// The block dots of the flat task stream into the RI row sums; CH(b, xc)
// fetches block b's activation chunk in the pair order of WT's unpacking
// (CH.half(b, h, xc): its pairs 8h .. 8h + 7, for half_slots).
template <int WT, int FN, int RI, int I = 0, typename CH>
__device__ __forceinline__ void dot_flat(const u4 (&q)[Flat<FN, RI>::IT][BlkLoads<WT>::n],
                                         const uint32_t (&ds)[Flat<FN, RI>::IT * ds_per<WT>()], const CH& chunk,
                                         int lane, float (&acc)[RI]) {
    if constexpr (I < Flat<FN, RI>::IT && half_slots<WT>()) {
        dot_flat_half<WT, FN, RI, I, 0>(q[I][0], ds[2 * I], chunk, lane, acc);
        dot_flat_half<WT, FN, RI, I, 1>(q[I][1], ds[2 * I + 1], chunk, lane, acc);
        dot_flat<WT, FN, RI, I + 1>(q, ds, chunk, lane, acc);
    } else if constexpr (I < Flat<FN, RI>::IT) {
        const int gb = lane + 64 * I;
        const int r = gb / FN;
        uint32_t xc[16];
        chunk(gb - r * FN, xc);
        constexpr int rlo = (64 * I) / FN;
        constexpr int rhi = (64 * I + 63) / FN < RI ? (64 * I + 63) / FN : RI - 1;
        if constexpr (rlo == rhi) {
            acc[rlo] = block_dot<WT>(q[I], ds[I], xc, acc[rlo]);
        } else {
            const bool lo = gb < (rlo + 1) * FN;
            float c = lo ? acc[rlo] : acc[rhi];
            c = block_dot<WT>(q[I], ds[I], xc, c);
            acc[rlo] = lo ? c : acc[rlo];
            acc[rhi] = lo ? acc[rhi] : c;
        }
        dot_flat<WT, FN, RI, I + 1>(q, ds, chunk, lane, acc);
    }
}

// Plain GEMV of one activation row (M = 1) with the single-row epilogues
// (STORE, BIAS, RESID, BIAS_RESID, BIAS_GELU): the decoder's output and
// down projections and linear() on one row.  The per-block arithmetic is
// gemv_kernel's (the same dequantised weights and products, fp32 sums, the
// same wave reduction); the lane partial sums are gemv_kernel's for the
// row-per-wave layout of Q4_0, Q6_K and f16, and in another order for the
// flat layout and Q8_0's half-block words (the same values up to fp32
// summation order).  What differs besides is how the loads are addressed.  Its
// parameter block holds only what these epilogues read, fetched as the
// code first needs it; the wave's rows are scalar (the wave index is read
// through readfirstlane), and every load is a range-checked buffer load
// (load_rows_buf, load_quad_buf): the weight loads go out after a handful
// of scalar instructions instead of gemv_kernel's per-lane 64-bit address
// arithmetic, and blocks or quads past the row read zeros (zero weights,
// zero activations) so the dot needs no bounds branch.
struct Gemv1Params {
    const uint16_t* x;
    const uint8_t* wq;
    const uint16_t* wd;
    const uint16_t* bias;
    const uint16_t* resid;
    uint16_t* y;
    int N, K, epi;
};

// EPI >= 0: the epilogue as a template argument (the bias / residual loads
// and the epilogue's branches resolved at compile time; measured on MI355X
// under graph replay: Q4_0 [2048 x 2048] + residual 2.87 -> 2.60 us,
// [2048 x 5632] + residual 4.10 -> 3.99 us, [5632 x 2048] 3.81 -> 3.71 us,
// bit-identical outputs); EPI < 0: chosen at run time from p.epi and the
// pointers present.
// The body takes its workgroup index as bx, so that a launch of another
// kernel can run it on some of its workgroups (WPB * 64 threads each).
template <int WT, int NB, int RI, int EPI = -1, int FN = 0, int WPB = 4>
__device__ __forceinline__ void gemv_m1_body(const Gemv1Params& p, int bx) {
    constexpr int NT = WPB * 64, NSX = (NB * 256 + NT - 1) / NT;   // activation quads per thread
    __shared__ u4 xs[4][NB * 64];
    const bool has_bias = EPI < 0 ? p.bias != nullptr : (EPI == EPI_BIAS || EPI == EPI_BIAS_RESID || EPI == EPI_BIAS_GELU);
    const bool has_resid = EPI < 0 ? p.resid != nullptr : (EPI == EPI_RESID || EPI == EPI_BIAS_RESID);
    const int epi = EPI < 0 ? p.epi : EPI;
    constexpr int NL = BlkLoads<WT>::n;
    const int lane = threadIdx.x & 63;
    const int row0 = (bx * WPB + __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6)) * RI;
    uint32_t xw[NSX][4];
    {
        const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)p.x, (short)0, p.K * 2, BUF_RSRC_WORD3);
#pragma unroll
        for (int k = 0; k < NSX; k++) load_quad_buf<WT>(rx, (int)threadIdx.x + NT * k, xw[k]);
    }
    __builtin_amdgcn_sched_barrier(0);   // the activation loads go out first
    constexpr int FIT = FN > 0 ? Flat<(FN > 0 ? FN : 64), RI>::IT : 1;
    u4 q[RI][NB][NL];
    uint32_t ds[RI][NB * ds_per<WT>()];
    u4 qf[FIT][NL];
    uint32_t dsf[FIT * ds_per<WT>()];
    if constexpr (FN > 0) load_flat<WT, FN, RI>(p.wq, p.wd, p.N, p.K, row0, lane, qf, dsf);
    else load_rows_buf<WT, NB, RI>(p.wq, p.wd, p.N, p.K, row0, lane, q, ds);
    // the epilogue's f16 operands: one per row, the same address in every
    // lane; an absent operand is never loaded (the branch is uniform)
    // From 4 rows per wave lane ri finishes row row0 + ri (see the stores
    // below) and loads its own operands; with fewer rows lane 0 finishes them
    // all from operands loaded at one scalar offset each (measured on MI355X:
    // the per-lane form cost config-4 decode 0.45 % at 2 rows per wave, and
    // gained Phi-2 decode 1.8 % at 4).  Range-checked loads: rows past N
    // read zero.
    constexpr bool LANE_EPI = RI >= 4;
    uint32_t eb[RI], er[RI];
#pragma unroll
    for (int ri = 0; ri < RI; ri++) eb[ri] = er[ri] = 0u;
    const int erow = row0 + (lane < RI ? lane : 0);
    if (has_bias) {
        const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)p.bias, (short)0, p.N * 2, BUF_RSRC_WORD3);
        if constexpr (LANE_EPI) eb[0] = __builtin_amdgcn_raw_buffer_load_b16(rb, erow * 2, 0, 0);
        else
#pragma unroll
            for (int ri = 0; ri < RI; ri++) eb[ri] = __builtin_amdgcn_raw_buffer_load_b16(rb, 0, (row0 + ri) * 2, 0);
    }
    if (has_resid) {
        const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc((void*)p.resid, (short)0, p.N * 2, BUF_RSRC_WORD3);
        if constexpr (LANE_EPI) er[0] = __builtin_amdgcn_raw_buffer_load_b16(rr, erow * 2, 0, 0);
        else
#pragma unroll
            for (int ri = 0; ri < RI; ri++) er[ri] = __builtin_amdgcn_raw_buffer_load_b16(rr, 0, (row0 + ri) * 2, 0);
    }
#pragma unroll
    for (int k = 0; k < NSX; k++) {
        const int it = threadIdx.x + NT * k;
        const uint32_t* w = xw[k];
        if (NT * NSX == NB * 256 || it < NB * 256)   // (the staging row holds NB * 256 quads)
            (&xs[0][0])[xs_at<WT, NB>(it >> 2, it & 3)] =
                WT == TLHIP_F16 ? u4{w[0], w[1], w[2], w[3]}
                                : u4{pack_lo(w[0], w[1]), pack_hi(w[0], w[1]), pack_lo(w[2], w[3]), pack_hi(w[2], w[3])};
    }
    lds_barrier();
    if (row0 >= p.N) return;   // (uniform: only the last workgroup has idle waves)
    float acc[RI];
#pragma unroll
    for (int ri = 0; ri < RI; ri++) acc[ri] = 0.0f;
    const XsChunk<WT, NB> chunk{&xs[0][0]};
    if constexpr (FN > 0) {
        dot_flat<WT, FN, RI>(qf, dsf, chunk, lane, acc);
    } else if constexpr (half_slots<WT>()) {
#pragma unroll
        for (int i = 0; i < NB; i++)
#pragma unroll
            for (int l = 0; l < 2; l++) {
                uint32_t xc[8];
                chunk.half(half_block(i, l, lane), lane & 1, xc);
#pragma unroll
                for (int ri = 0; ri < RI; ri++) acc[ri] = q8_half_dot(q[ri][i][l], ds[ri][2 * i + l], xc, acc[ri]);
            }
    } else {
#pragma unroll
        for (int i = 0; i < NB; i++) {
            uint32_t xc[16];
            chunk(lane + 64 * i, xc);
#pragma unroll
            for (int ri = 0; ri < RI; ri++) acc[ri] = block_dot<WT>(q[ri][i], ds[ri][i], xc, acc[ri]);
        }
    }
#pragma unroll
    for (int ri = 0; ri < RI; ri++) acc[ri] = wave_sum<64>(acc[ri]);
    if constexpr (LANE_EPI) {
        // every lane holds the RI row sums: lane ri stores row row0 + ri (the
        // epilogues side by side instead of one after another in lane 0)
        float a = acc[0];
#pragma unroll
        for (int ri = 1; ri < RI; ri++) a = lane == ri ? acc[ri] : a;
        if (lane < RI && row0 + lane < p.N) p.y[row0 + lane] = epilogue_v(epi, a, (uint16_t)eb[0], (uint16_t)er[0]);
    } else if (lane == 0) {
#pragma unroll
        for (int ri = 0; ri < RI; ri++)
            if (row0 + ri < p.N) p.y[row0 + ri] = epilogue_v(epi, acc[ri], (uint16_t)eb[ri], (uint16_t)er[ri]);
    }
}

template <int WT, int NB, int RI, int EPI = -1, int FN = 0, int WPB = 4>
__global__ __launch_bounds__(WPB * 64) void gemv_m1_kernel(Gemv1Params p) {
    gemv_m1_body<WT, NB, RI, EPI, FN, WPB>(p, (int)blockIdx.x);
}

// Normalised GEMV (M = 1): norm(x) staged once per workgroup in LDS (the
// weight loads are issued first, so they are in flight during it), then
// the same block dots.  EPI_ARGMAX additionally reduces the workgroup's
// stored logits to one (value, index) key in amax_slots[blockIdx.x].
// The parameter block as a kernel specialised on its epilogue sees it: EPI
// (and M = 1) as constants, and the fields that epilogue never reads as
// null / zero constants, so the compiler drops their loads and every branch
// on them (measured on MI355X at [2560 x 2048] and [11264 x 2048] Q4_0:
// 0.3 us less per launch, bit-identical outputs).  EPI < 0: the block as
// passed, epilogue chosen at run time.
template <int PRO, int EPI>
__device__ __forceinline__ GemvParams norm_view(const GemvParams& k) {
    if (EPI < 0) return k;
    GemvParams p = {};
    p.x = k.x;
    p.wq = k.wq;
    p.wd = k.wd;
    p.y = k.y;
    p.M = 1;
    p.N = k.N;
    p.K = k.K;
    p.ldy = k.ldy;
    p.epi = EPI;
    p.norm_w = k.norm_w;
    p.eps = k.eps;
    if (PRO == PRO_LN) p.norm_b = k.norm_b;
    if (EPI == EPI_BIAS || EPI == EPI_BIAS_RESID || EPI == EPI_BIAS_GELU || EPI == EPI_QKV_ROPE || EPI == EPI_ARGMAX)
        p.bias = k.bias;
    if (EPI == EPI_RESID || EPI == EPI_BIAS_RESID) p.resid = k.resid;
    if (EPI == EPI_QKV_ROPE) {
        p.nq = k.nq;
        p.nk = k.nk;
        p.head_dim = k.head_dim;
        p.rot = k.rot;
        p.layout = k.layout;
        p.pos0 = k.pos0;
        p.rope_tab = k.rope_tab;
        p.d_pos = k.d_pos;
        p.q_out = k.q_out;
        p.kc = k.kc;
        p.vc = k.vc;
        // (the embedding-row prologue only ever precedes layer 0's QKV)
        p.embd = k.embd;
        p.d_token = k.d_token;
        p.x_out = k.x_out;
        p.xn_out = k.xn_out;
        if (PRO == PRO_LN) p.x_add = k.x_add;
    }
    if (EPI == EPI_ARGMAX) {
        p.amax_slots = k.amax_slots;
        if (PRO == PRO_LN) p.x_add = k.x_add;
    }
    return p;
}

template <int WT, int NB, int RI, int WPB, int PRO, int EPI = -1, int FN = 0>
__global__ __launch_bounds__(WPB * 64) void gemv_norm_kernel(GemvParams pk) {
    __shared__ u4 xs[4][NB * 64];
    __shared__ float red[2][WPB];
    __shared__ unsigned long long wkey[WPB];
    const GemvParams p = norm_view<PRO, EPI>(pk);
    kernarg_fence(p);
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int row0 = (blockIdx.x * WPB + w) * RI;   // wave-uniform (load_rows_buf)
    const int nbr = p.K >> 5;
    constexpr int NL = BlkLoads<WT>::n;
    u4 q[RI][NB][NL];
    uint32_t ds[RI][NB * ds_per<WT>()];   // scales zero-extended: no packing that would force an early wait
    // The decode position (only lane 0's RoPE table loads depend on it) is
    // read first, as a vector load: those retire in order, so waiting for it
    // later does not wait for the activation and weight loads issued after
    // it.  As a scalar load (what a uniform address gets) any wait for it
    // would be a wait for every scalar load, and it held back all the
    // activation and weight loads by one memory round trip.  The load is
    // unconditional, so no branch join forces the wait right here: without
    // a device position it reads the first word of the norm weight, which
    // launch_gemv requires for every normalised GEMV (the scale array is
    // absent for F16 weights).
    const bool dev_pos = p.epi == EPI_QKV_ROPE && p.d_pos;
    const int pos_raw = (dev_pos ? p.d_pos : (const int32_t*)p.norm_w)[opaque_zero()];
    // (the token is uniform: read through readfirstlane, the row address
    // stays scalar and the staging loads take one buffer descriptor instead
    // of a loop over the lanes' distinct descriptors)
    const uint16_t* xsrc = p.embd ? p.embd + (size_t)__builtin_amdgcn_readfirstlane(*p.d_token) * p.K : p.x;
    NormStage<WT, NB, WPB, PRO> st;
    st.load(p, xsrc);
    // (unconditional: rows are clamped into the matrix, and loads under a
    // branch leave the compiler's wait counts imprecise after it)
    constexpr int FIT = FN > 0 ? Flat<(FN > 0 ? FN : 64), RI>::IT : 1;
    u4 qf[FIT][NL];
    uint32_t dsf[FIT * ds_per<WT>()];
    if constexpr (FN > 0) load_flat<WT, FN, RI>(p.wq, p.wd, p.N, p.K, row0, lane, qf, dsf);
    else load_rows_buf<WT, NB, RI>(p.wq, p.wd, p.N, p.K, row0, lane, q, ds);
    EpiPre<RI, 1> pre;
    QkvPre qp[RI / 2 > 0 ? RI / 2 : 1];
    if (lane == 0 && row0 < p.N && p.epi == EPI_QKV_ROPE) {
        const int pos = p.pos0 + (dev_pos ? pos_raw : 0);
#pragma unroll
        for (int ri = 0; ri + 1 < RI; ri += 2)
            if (row0 + ri + 1 < p.N) qkv_rope_pre(p, row0 + ri, pos, qp[ri / 2]);
    }
    // single-row epilogues and greedy keys: lane ri finishes row row0 + ri,
    // so its bias / residual element is loaded by that lane, here
    uint32_t eb1 = 0u, er1 = 0u;
    if (lane < RI && row0 + lane < p.N && p.epi != EPI_QKV_ROPE && p.epi != EPI_SWIGLU_PAIR) {
        if (p.bias) eb1 = p.bias[row0 + lane];
        if (p.resid) er1 = p.resid[row0 + lane];
    }
    st.finish(p, xs, red);
    const XsChunk<WT, NB> chunk{&xs[0][0]};

    float acc[RI][1];
#pragma unroll
    for (int ri = 0; ri < RI; ri++) acc[ri][0] = 0.0f;
    if (row0 < p.N) {
        if constexpr (FN > 0) {
            float af[RI];
#pragma unroll
            for (int ri = 0; ri < RI; ri++) af[ri] = 0.0f;
            dot_flat<WT, FN, RI>(qf, dsf, chunk, lane, af);
#pragma unroll
            for (int ri = 0; ri < RI; ri++) acc[ri][0] = af[ri];
        } else if constexpr (half_slots<WT>()) {
#pragma unroll
            for (int i = 0; i < NB; i++)
#pragma unroll
                for (int l = 0; l < 2; l++) {
                    const int b = half_block(i, l, lane);
                    if (b < nbr) {
                        uint32_t xc[8];
                        chunk.half(b, lane & 1, xc);
#pragma unroll
                        for (int ri = 0; ri < RI; ri++) acc[ri][0] = q8_half_dot(q[ri][i][l], ds[ri][2 * i + l], xc, acc[ri][0]);
                    }
                }
        } else {
#pragma unroll
            for (int i = 0; i < NB; i++) {
                const int b = lane + 64 * i;
                if (b < nbr) {
                    uint32_t xc[16];
                    chunk(b, xc);
#pragma unroll
                    for (int ri = 0; ri < RI; ri++) acc[ri][0] = block_dot<WT>(q[ri][i], ds[ri][i], xc, acc[ri][0]);
                }
            }
        }
#pragma unroll
        for (int ri = 0; ri < RI; ri++) acc[ri][0] = wave_sum<64>(acc[ri][0]);
    }
    if (p.epi == EPI_QKV_ROPE) {
        if (lane == 0 && row0 < p.N)
#pragma unroll
            for (int ri = 0; ri + 1 < RI; ri += 2)
                if (row0 + ri + 1 < p.N) qkv_rope_store(p, row0 + ri, acc[ri][0], acc[ri + 1][0], qp[ri / 2]);
        st.store_xn(p);
        return;
    }
    if (p.epi == EPI_SWIGLU_PAIR) {
        if (lane == 0 && row0 < p.N) store_rows<RI, 1>(p, row0, acc, pre);
        return;
    }
    // every lane holds the RI row sums: lane ri finishes row row0 + ri (the
    // RI epilogues run side by side instead of one after another in lane 0)
    float a = acc[0][0];
#pragma unroll
    for (int ri = 1; ri < RI; ri++) a = lane == ri ? acc[ri][0] : a;
    const int row = row0 + lane;
    const bool mine = lane < RI && row < p.N;
    if (p.epi != EPI_ARGMAX) {
        if (mine) p.y[row] = epilogue_v(p.epi, a, (uint16_t)eb1, (uint16_t)er1);
        return;
    }
    unsigned long long best = 0ull;
    if (mine) {
        uint16_t r = f2h(a);
        if (p.bias) r = add_h(r, (uint16_t)eb1);
        p.y[row] = r;
        best = amax_key(r, row);
    }
    // the RI lanes' keys to lane 0 (lanes past RI hold 0), then the waves
#pragma unroll
    for (int o = 1; o < RI; o <<= 1) best = umax64(best, __shfl_xor(best, o, 64));
    if (lane == 0) wkey[w] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = wkey[0];
#pragma unroll
        for (int k = 1; k < WPB; k++) b = umax64(b, wkey[k]);
        p.amax_slots[blockIdx.x] = b;
    }
}


// Launch shapes of the normalised GEMV (M = 1) by row count: 8 waves x 4
// rows from 16384 rows (not for the paired epilogues), 8 waves x 2 rows from
// 8192, else 4 waves x 2 rows; the epilogue-specialised paired kernels take
// 4 waves x 2 rows, the SwiGLU pair 4 waves x 4 rows from 8192 (measured at
// [11264 x 2048] Q4_0 under graph replay: 6.27-6.29 vs 6.32-6.36 us with 8
// waves x 2 rows).  gemv_norm_slots
// gives the workgroup count of the greedy-key epilogue's shapes.
template <int WT, int NB, int PRO, int EPI = -1>
static void launch_norm_shape(hipStream_t s, const GemvParams& p) {
    constexpr bool paired = EPI == EPI_QKV_ROPE || EPI == EPI_SWIGLU_PAIR;
    if constexpr (NB == 2 && WT != TLHIP_Q6_K) {
        if (p.K == 80 * 32) {
            // 80 blocks per row (K = 2560): the flat task layout with the same
            // rows per workgroup as the shapes below -- 4 rows per wave (5
            // tasks per lane, none idle) from 8192 rows, 2 rows per wave (3
            // tasks, 1 in 6 idle) below, where 4 would leave too few waves
            // (measured on MI355X, Q8_0 Phi-2 decode: [10240 x 2560] + GELU
            // 10.78 -> 9.55 us with 4 rows; [7680 x 2560] QKV 8.23 -> 9.54 us
            // with 4 rows in 2-wave workgroups)
            const bool pair = paired || p.epi == EPI_QKV_ROPE || p.epi == EPI_SWIGLU_PAIR;
            // (8 waves x 4 rows from 8192 rows too unless the greedy keys fix
            // 16 rows per workgroup: one quad of the 2560-element row per
            // staging thread instead of two for a quarter of them)
            if (!pair && p.N >= 16384)
                hipLaunchKernelGGL((gemv_norm_kernel<WT, NB, 4, 8, PRO, EPI, 80>), dim3((p.N + 31) / 32), dim3(512), 0, s, p);
            else if (!pair && p.N >= 8192)
                hipLaunchKernelGGL((gemv_norm_kernel<WT, NB, 4, 4, PRO, EPI, 80>), dim3((p.N + 15) / 16), dim3(256), 0, s, p);
            else
                hipLaunchKernelGGL((gemv_norm_kernel<WT, NB, 2, 4, PRO, EPI, 80>), dim3((p.N + 7) / 8), dim3(256), 0, s, p);
            return;
        }
    }
    if (!paired && p.N >= 16384 && p.epi != EPI_QKV_ROPE && p.epi != EPI_SWIGLU_PAIR) {
        const int wgs = (p.N + 31) / 32;   // 8 waves x 4 rows
        if constexpr (!paired) hipLaunchKernelGGL((gemv_norm_kernel<WT, NB, 4, 8, PRO, EPI>), dim3(wgs), dim3(512), 0, s, p);
    } else if (p.N >= 8192 && !paired) {
        const int wgs = (p.N + 15) / 16;   // 8 waves x 2 rows
        hipLaunchKernelGGL((gemv_norm_kernel<WT, NB, 2, 8, PRO, EPI>), dim3(wgs), dim3(512), 0, s, p);
    } else if (EPI == EPI_SWIGLU_PAIR && p.N >= 8192) {
        // 4 waves x 4 rows (measured on MI355X, config-4 decode with its
        // [11264 x 2048] Q4_0 gate/up + SwiGLU: 2202 -> 2219 tok/s against 2
        // rows per wave, same tokens)
        hipLaunchKernelGGL((gemv_norm_kernel<WT, NB, 4, 4, PRO, EPI>), dim3((p.N + 15) / 16), dim3(256), 0, s, p);
    } else {
        const int wgs = (p.N + 7) / 8;     // 4 waves x 2 rows
        hipLaunchKernelGGL((gemv_norm_kernel<WT, NB, 2, 4, PRO, EPI>), dim3(wgs), dim3(256), 0, s, p);
    }
}

// The single-row GEMV from 1024 rows (two rows per wave up to K = 4096, one
// beyond), specialised on its epilogue (kernels_gemv_m1.hip): plain store,
// bias, residual, bias + residual, each only when the pointers it reads are
// present.  false: not specialised.
bool launch_m1_epi(hipStream_t s, tlhip_dtype wt, const Gemv1Params& p, int nb, int ri);

// The normalised GEMV of a decode step, specialised on its epilogue
// (kernels_gemv_norm.hip): RMSNorm with the SwiGLU pair, QKV + RoPE + cache
// or greedy-key epilogue; LayerNorm with the QKV, bias + GELU or greedy-key
// epilogue.  false: no specialisation for this combination (or NB > 2).
bool launch_norm_epi(hipStream_t s, tlhip_dtype wt, const GemvParams& p, int nb, int pro);

}  // namespace tlhip
