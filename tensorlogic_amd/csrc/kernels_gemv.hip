// kernels_gemv.hip -- fused dequant-GEMV for decode (M <= 4), GGUF repack
// and dequantisation kernels, gfx950 / wave64.
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
#include "device_common.hpp"
#include "internal.hpp"

namespace tlhip {

// ---------------------------------------------------------------------------
// repack: GGUF blocks <-> structure-of-arrays (qs rows + scale array)
// ---------------------------------------------------------------------------
// Block b of the GGUF stream is block (b % bpr) of source row r = b / bpr;
// it lands in destination row dst_row0 + r * dst_step (step 1 = plain
// upload, step 2 interleaves two matrices row by row).
template <int BB, int QB>   // block bytes, payload bytes per block
__global__ void repack_kernel(const uint8_t* __restrict__ blocks, uint8_t* __restrict__ qs,
                              uint16_t* __restrict__ d, int64_t nblocks, int64_t bpr,
                              int64_t dst_row0, int64_t dst_step, int to_gguf) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const int64_t r = b / bpr, c = b % bpr;
    const int64_t db = (dst_row0 + r * dst_step) * bpr + c;
    const uint8_t* src = blocks + b * BB;
    uint8_t* q = qs + db * QB;
    if (!to_gguf) {
        d[db] = (uint16_t)(src[0] | (src[1] << 8));
#pragma unroll
        for (int i = 0; i < QB; i++) q[i] = src[2 + i];
    } else {
        uint8_t* dst = (uint8_t*)blocks + b * BB;
        uint16_t s = d[db];
        dst[0] = (uint8_t)(s & 0xff);
        dst[1] = (uint8_t)(s >> 8);
#pragma unroll
        for (int i = 0; i < QB; i++) dst[2 + i] = q[i];
    }
}

tlhip_status launch_repack_rows(hipStream_t s, tlhip_dtype wt, const uint8_t* blocks, void* qs,
                                uint16_t* d, int64_t nblocks, int64_t bpr, int64_t dst_row0,
                                int64_t dst_step, int to_gguf) {
    if (nblocks <= 0) return TLHIP_OK;
    dim3 grid((unsigned)((nblocks + 255) / 256));
    if (wt == TLHIP_Q4_0)
        hipLaunchKernelGGL((repack_kernel<18, 16>), grid, dim3(256), 0, s, blocks, (uint8_t*)qs, d,
                           nblocks, bpr, dst_row0, dst_step, to_gguf);
    else
        hipLaunchKernelGGL((repack_kernel<34, 32>), grid, dim3(256), 0, s, blocks, (uint8_t*)qs, d,
                           nblocks, bpr, dst_row0, dst_step, to_gguf);
    return TLHIP_OK;
}

tlhip_status launch_repack(hipStream_t s, tlhip_dtype wt, const uint8_t* blocks, void* qs,
                           uint16_t* d, int64_t nblocks, int64_t bpr, int to_gguf) {
    return launch_repack_rows(s, wt, blocks, qs, d, nblocks, bpr, 0, 1, to_gguf);
}

// ---------------------------------------------------------------------------
// dequantisation to f16 (bit-exact with gguf.rs dequantize_q4_0 / q8_0)
// one thread per block; 32 outputs written as 4 x 16 bytes
// ---------------------------------------------------------------------------
__device__ __forceinline__ void q4_unpack(uint32_t w, h2 dd, h2 out[4]) {
    const h2 bias = {(h16)-1032.0f, (h16)-1032.0f};
    out[0] = (as_h2((w & 0x000F000Fu) | 0x64006400u) + bias) * dd;          // e0, e2
    out[1] = (as_h2(((w >> 8) & 0x000F000Fu) | 0x64006400u) + bias) * dd;   // e1, e3
    out[2] = (as_h2(((w >> 4) & 0x000F000Fu) | 0x64006400u) + bias) * dd;   // e16, e18
    out[3] = (as_h2(((w >> 12) & 0x000F000Fu) | 0x64006400u) + bias) * dd;  // e17, e19
}

__device__ __forceinline__ void q8_unpack(uint32_t w, h2 dd, h2 out[2]) {
    const h2 bias = {(h16)-1152.0f, (h16)-1152.0f};
    uint32_t v = w ^ 0x80808080u;
    out[0] = (as_h2((v & 0x00FF00FFu) | 0x64006400u) + bias) * dd;          // e0, e2
    out[1] = (as_h2(((v >> 8) & 0x00FF00FFu) | 0x64006400u) + bias) * dd;   // e1, e3
}

__global__ void dequant_q4_0_kernel(const uint8_t* __restrict__ qs, const uint16_t* __restrict__ d,
                                    uint16_t* __restrict__ out, int64_t nblocks) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    u4 q = *(const u4*)(qs + b * 16);
    h16 dh = __builtin_bit_cast(h16, d[b]);
    h2 dd = {dh, dh};
    uint32_t lo[8], hi[8];   // elements 0..15 and 16..31 as 8 pairs each
#pragma unroll
    for (int t = 0; t < 4; t++) {
        h2 r[4];
        q4_unpack(q[t], dd, r);
        // r[0] = (e4t, e4t+2), r[1] = (e4t+1, e4t+3) -> natural pairs
        lo[2 * t + 0] = pack_lo(as_u32(r[0]), as_u32(r[1]));   // (e4t, e4t+1)
        lo[2 * t + 1] = pack_hi(as_u32(r[0]), as_u32(r[1]));   // (e4t+2, e4t+3)
        hi[2 * t + 0] = pack_lo(as_u32(r[2]), as_u32(r[3]));
        hi[2 * t + 1] = pack_hi(as_u32(r[2]), as_u32(r[3]));
    }
    u4* o = (u4*)(out + b * 32);
    o[0] = u4{lo[0], lo[1], lo[2], lo[3]};
    o[1] = u4{lo[4], lo[5], lo[6], lo[7]};
    o[2] = u4{hi[0], hi[1], hi[2], hi[3]};
    o[3] = u4{hi[4], hi[5], hi[6], hi[7]};
}

__global__ void dequant_q8_0_kernel(const uint8_t* __restrict__ qs, const uint16_t* __restrict__ d,
                                    uint16_t* __restrict__ out, int64_t nblocks) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const u4* qp = (const u4*)(qs + b * 32);
    h16 dh = __builtin_bit_cast(h16, d[b]);
    h2 dd = {dh, dh};
    uint32_t o32[16];
#pragma unroll
    for (int v = 0; v < 2; v++) {
        u4 q = qp[v];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            h2 r[2];
            q8_unpack(q[t], dd, r);
            o32[8 * v + 2 * t + 0] = pack_lo(as_u32(r[0]), as_u32(r[1]));
            o32[8 * v + 2 * t + 1] = pack_hi(as_u32(r[0]), as_u32(r[1]));
        }
    }
    u4* o = (u4*)(out + b * 32);
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = u4{o32[4 * i], o32[4 * i + 1], o32[4 * i + 2], o32[4 * i + 3]};
}

tlhip_status launch_dequant(hipStream_t s, tlhip_dtype wt, const void* qs, const uint16_t* d,
                            uint16_t* out, int64_t N, int64_t K) {
    int64_t nb = N * K / 32;
    if (nb <= 0) return TLHIP_OK;
    dim3 grid((unsigned)((nb + 255) / 256));
    if (wt == TLHIP_Q4_0)
        hipLaunchKernelGGL(dequant_q4_0_kernel, grid, dim3(256), 0, s, (const uint8_t*)qs, d, out, nb);
    else
        hipLaunchKernelGGL(dequant_q8_0_kernel, grid, dim3(256), 0, s, (const uint8_t*)qs, d, out, nb);
    return TLHIP_OK;
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
};

// Per-block activation chunk in the pair order of the unpacking:
//   Q4_0 (16 pairs): [4t+0]=(x4t,x4t+2) [4t+1]=(x4t+1,x4t+3)
//                    [4t+2]=(x16+4t,x16+4t+2) [4t+3]=(x16+4t+1,x16+4t+3)
//   Q8_0 (16 pairs): [2t+0]=(x4t,x4t+2) [2t+1]=(x4t+1,x4t+3), t < 8
//   F16  (16 pairs): natural pairs (x2i, x2i+1)
template <int WT>
__device__ __forceinline__ void load_xchunk(const uint16_t* __restrict__ xb, uint32_t xc[16]) {
    const u4* p = (const u4*)xb;
    uint32_t xw[16];   // xw[i] = (x2i, x2i+1)
#pragma unroll
    for (int v = 0; v < 4; v++) {
        u4 t = p[v];
        xw[4 * v + 0] = t[0]; xw[4 * v + 1] = t[1]; xw[4 * v + 2] = t[2]; xw[4 * v + 3] = t[3];
    }
    if (WT == TLHIP_Q4_0) {
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

// Weight payload of one 32-element block: Q4_0 1 x 16 B, Q8_0 2 x 16 B, F16 4 x 16 B.
template <int WT> struct BlkLoads { static constexpr int n = WT == TLHIP_Q4_0 ? 1 : (WT == TLHIP_Q8_0 ? 2 : 4); };

template <int WT>
__device__ __forceinline__ float block_dot(const u4* q, uint16_t dbits, const uint32_t xc[16], float acc) {
    if (WT == TLHIP_Q4_0) {
        h16 dh = __builtin_bit_cast(h16, dbits);
        h2 dd = {dh, dh};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            h2 r[4];
            q4_unpack(q[0][t], dd, r);
#pragma unroll
            for (int j = 0; j < 4; j++) acc = fdot2(r[j], as_h2(xc[4 * t + j]), acc);
        }
    } else if (WT == TLHIP_Q8_0) {
        h16 dh = __builtin_bit_cast(h16, dbits);
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

__device__ __forceinline__ void gemv_store(const GemvParams& p, int m, int row, float acc) {
    p.y[(size_t)m * p.ldy + row] = epilogue_h(p.epi, acc, p.bias, p.resid, (size_t)m * p.N + row, row);
}

// NB: blocks per lane (ceil(K/32/64)); RI: rows per wave; MX: max activation rows.
template <int WT, int NB, int RI, int MX>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int row0 = wave * RI;
    if (row0 >= p.N) return;
    const int nbr = p.K >> 5;
    constexpr int NL = BlkLoads<WT>::n;
    const size_t row_bytes = WT == TLHIP_Q4_0 ? (size_t)p.K / 2 : (WT == TLHIP_Q8_0 ? (size_t)p.K : (size_t)p.K * 2);

    // issue all weight loads first
    u4 q[RI][NB][NL];
    uint16_t ds[RI][NB];
#pragma unroll
    for (int ri = 0; ri < RI; ri++) {
        const int row = min(row0 + ri, p.N - 1);
        const uint8_t* wr = p.wq + (size_t)row * row_bytes;
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int b = min(lane + 64 * i, nbr - 1);
#pragma unroll
            for (int l = 0; l < NL; l++) q[ri][i][l] = *(const u4*)(wr + (size_t)b * (16 * NL) + 16 * l);
            ds[ri][i] = WT == TLHIP_F16 ? 0 : p.wd[(size_t)row * nbr + b];
        }
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
                    load_xchunk<WT>(p.x + (size_t)m * p.K + (size_t)b * 32, xc);
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

    if (lane == 0) {
        if (p.epi == EPI_SWIGLU_PAIR) {
            // rows (2i, 2i+1) hold (gate_i, up_i); RI is even and row0 even.
#pragma unroll
            for (int ri = 0; ri < RI; ri += 2) {
                const int row = row0 + ri;
                if (row + 1 < p.N)
#pragma unroll
                    for (int m = 0; m < MX; m++)
                        if (m < p.M)
                            p.y[(size_t)m * p.ldy + row / 2] = swiglu_h(f2h(acc[ri][m]), f2h(acc[ri + 1][m]));
            }
        } else {
#pragma unroll
            for (int ri = 0; ri < RI; ri++) {
                const int row = row0 + ri;
                if (row < p.N)
#pragma unroll
                    for (int m = 0; m < MX; m++)
                        if (m < p.M) gemv_store(p, m, row, acc[ri][m]);
            }
        }
    }
}

// Generic fallback for shapes the fast path does not cover (f16 W with
// K % 32 != 0, or K > 64*8*32): one wavefront per (row, m), scalar k loop.
__global__ __launch_bounds__(256) void gemv_generic_kernel(GemvParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wave >= (int64_t)p.N * p.M) return;
    const int row = (int)(wave % p.N), m = (int)(wave / p.N);
    const uint16_t* w = (const uint16_t*)p.wq + (size_t)row * p.K;
    const uint16_t* x = p.x + (size_t)m * p.K;
    float acc = 0.0f;
    for (int k = lane; k < p.K; k += 64) acc += h2f(x[k]) * h2f(w[k]);
    acc = wave_sum<64>(acc);
    if (lane == 0) gemv_store(p, m, row, acc);
}

template <int WT, int NB, int RI, int MX>
static void launch_one(hipStream_t s, const GemvParams& p) {
    int waves = (p.N + RI - 1) / RI;
    dim3 grid((unsigned)((waves + 3) / 4));
    hipLaunchKernelGGL((gemv_kernel<WT, NB, RI, MX>), grid, dim3(256), 0, s, p);
}

template <int WT, int NB, int MX>
static void launch_ri(hipStream_t s, const GemvParams& p, int ri) {
    if (ri >= 4) launch_one<WT, NB, 4, MX>(s, p);
    else if (ri == 2) launch_one<WT, NB, 2, MX>(s, p);
    else launch_one<WT, NB, 1, MX>(s, p);
}

template <int WT, int MX>
static bool launch_nb(hipStream_t s, const GemvParams& p, int nb, int ri) {
    switch (nb) {
        case 1: launch_ri<WT, 1, MX>(s, p, ri); return true;
        case 2: launch_ri<WT, 2, MX>(s, p, ri); return true;
        case 3: if (MX <= 2) { launch_ri<WT, 3, MX>(s, p, ri); return true; } return false;
        case 4: if (MX <= 2) { launch_ri<WT, 4, MX>(s, p, ri); return true; } return false;
        case 5: case 6: if (MX == 1) { launch_ri<WT, 6, MX>(s, p, ri); return true; } return false;
        case 7: case 8: if (MX == 1) { launch_ri<WT, 8, MX>(s, p, ri); return true; } return false;
        default: return false;
    }
}

template <int WT>
static bool launch_mx(hipStream_t s, const GemvParams& p, int nb, int ri) {
    if (p.M == 1) return launch_nb<WT, 1>(s, p, nb, ri);
    if (p.M == 2) return launch_nb<WT, 2>(s, p, nb, ri);
    if (p.M <= 4) return launch_nb<WT, 4>(s, p, nb, ri);
    return false;
}

tlhip_status launch_gemv(hipStream_t s, tlhip_dtype wt, const GemvArgs& a, int epi) {
    GemvParams p;
    p.x = a.x;
    p.wq = (const uint8_t*)a.wq;
    p.wd = a.wd;
    p.bias = a.bias;
    p.resid = a.resid;
    p.y = a.y;
    p.M = a.M;
    p.N = a.N;
    p.K = a.K;
    p.ldy = a.ldy ? a.ldy : (epi == EPI_SWIGLU_PAIR ? a.N / 2 : a.N);
    p.epi = epi;
    if (p.N <= 0 || p.M <= 0) return TLHIP_OK;
    bool done = false;
    if (p.K % 32 == 0 && p.K > 0) {
        const int nbr = p.K / 32;
        const int nb = (nbr + 63) / 64;
        // Rows per wave: enough waves to fill 256 CUs several times over,
        // more bytes in flight per lane when the matrix is tall.
        int ri = p.N >= 8192 ? 4 : (p.N >= 4096 ? 2 : 1);
        if (epi == EPI_SWIGLU_PAIR && ri < 2) ri = 2;
        if (wt == TLHIP_Q4_0) done = launch_mx<TLHIP_Q4_0>(s, p, nb, ri);
        else if (wt == TLHIP_Q8_0) done = launch_mx<TLHIP_Q8_0>(s, p, nb, ri);
        else done = launch_mx<TLHIP_F16>(s, p, nb, ri);
    }
    if (!done) {
        if (wt != TLHIP_F16 || epi == EPI_SWIGLU_PAIR)
            return fail(TLHIP_ERR_INVALID_OPERATION, "gemv: unsupported shape M=%d K=%d", p.M, p.K);
        int64_t waves = (int64_t)p.N * p.M;
        hipLaunchKernelGGL(gemv_generic_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, p);
    }
    return TLHIP_OK;
}

}  // namespace tlhip
