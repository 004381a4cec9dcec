// kernels_gemv.hip -- GGUF repack and dequantisation kernels, and the
// launches of the fused dequant-GEMV for decode (M <= 4), gfx950 / wave64.
// The GEMV's device code and kernel templates are in gemv_device.hpp; the
// normalised GEMVs of the decode step, specialised on their epilogue, are
// instantiated in kernels_gemv_norm.hip.
#include "gemv_device.hpp"

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

// Q6_K: one thread per 32-element group g of a source row (super-block
// g / 8, half n = (g % 8) / 4, quarter j = g % 4: elements 128n + 32j + l).
// Element value code q = low 4 bits from nibble j / 2 of ql[64n + 32(j % 2)
// + l], high 2 bits from bits 2j..2j+1 of qh[32n + l] (gguf.rs:170-190).
// Download (to_gguf) rebuilds a super-block from its eight groups: the
// threads of quarters 0/1 write the ql bytes they share with quarters 2/3,
// quarter-0 threads the qh bytes, group-0 threads d.
__global__ void repack_q6k_kernel(uint8_t* __restrict__ blocks, uint8_t* __restrict__ q4, uint8_t* __restrict__ q2,
                                  int8_t* __restrict__ sc, uint16_t* __restrict__ d, int64_t src_rows, int64_t K,
                                  int64_t dst_row0, int64_t dst_step, int to_gguf) {
    const int64_t gpr = K / 32;   // groups per row
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= src_rows * gpr) return;
    const int64_t r = t / gpr, g = t % gpr;
    const int64_t dr = dst_row0 + r * dst_step;
    uint8_t* blk = blocks + (r * (K / 256) + g / 8) * 210;
    const int n = (int)(g % 8) / 4, j = (int)(g % 4);
    uint8_t* ql = blk + 64 * n + 32 * (j % 2);
    uint8_t* qh = blk + 128 + 32 * n;
    int8_t* bsc = (int8_t*)(blk + 192) + 8 * n + 2 * j;
    uint8_t* o4 = q4 + dr * (K / 2) + g * 16;
    uint8_t* o2 = q2 + dr * (K / 4) + g * 8;
    int8_t* osc = sc + dr * (K / 16) + 2 * g;
    if (!to_gguf) {
        uint8_t code[32];
#pragma unroll
        for (int l = 0; l < 32; l++) code[l] = (uint8_t)(((ql[l] >> (4 * (j / 2))) & 15) | (((qh[l] >> (2 * j)) & 3) << 4));
#pragma unroll
        for (int i = 0; i < 16; i++) o4[i] = (uint8_t)((code[i] & 15) | ((code[i + 16] & 15) << 4));
#pragma unroll
        for (int w = 0; w < 2; w++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                uint8_t v = 0;
#pragma unroll
                for (int tt = 0; tt < 4; tt++) v |= (uint8_t)((code[16 * w + 4 * tt + b] >> 4) << (2 * tt));
                o2[4 * w + b] = v;
            }
        osc[0] = bsc[0];
        osc[1] = bsc[1];
        if (g % 8 == 0) d[dr * (K / 256) + g / 8] = (uint16_t)(blk[208] | (blk[209] << 8));
    } else {
        // code of element l of group gg (same row) from the planes
        auto code_of = [&](int64_t gg, int l) -> int {
            const uint8_t* a4 = q4 + dr * (K / 2) + gg * 16;
            const uint8_t* a2 = q2 + dr * (K / 4) + gg * 8;
            const int lo = l < 16 ? (a4[l] & 15) : (a4[l - 16] >> 4);
            const int w = l / 16, tt = (l % 16) / 4, b = l % 4;
            return lo | (((a2[4 * w + b] >> (2 * tt)) & 3) << 4);
        };
        if (j < 2)
            for (int l = 0; l < 32; l++) ql[l] = (uint8_t)(code_of(g, l) & 15) | (uint8_t)((code_of(g + 2, l) & 15) << 4);
        if (j == 0)
            for (int l = 0; l < 32; l++) {
                uint8_t v = 0;
                for (int jj = 0; jj < 4; jj++) v |= (uint8_t)((code_of(g + jj, l) >> 4) << (2 * jj));
                qh[l] = v;
            }
        bsc[0] = osc[0];
        bsc[1] = osc[1];
        if (g % 8 == 0) {
            const uint16_t dv = d[dr * (K / 256) + g / 8];
            blk[208] = (uint8_t)(dv & 0xff);
            blk[209] = (uint8_t)(dv >> 8);
        }
    }
}

tlhip_status launch_repack_rows(hipStream_t s, tlhip_dtype wt, const uint8_t* blocks, void* data,
                                uint16_t* d, int64_t src_rows, int64_t K, int64_t dst_rows, int64_t dst_row0,
                                int64_t dst_step, int to_gguf) {
    if (src_rows <= 0 || K <= 0) return TLHIP_OK;
    if (wt == TLHIP_Q6_K) {
        const int64_t n = src_rows * (K / 32);
        uint8_t* base = (uint8_t*)data;
        hipLaunchKernelGGL(repack_q6k_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (uint8_t*)blocks,
                           base, base + q6k_q2_offset(dst_rows, K), (int8_t*)(base + q6k_sc_offset(dst_rows, K)), d,
                           src_rows, K, dst_row0, dst_step, to_gguf);
        return TLHIP_OK;
    }
    const int64_t nblocks = src_rows * (K / 32), bpr = K / 32;
    dim3 grid((unsigned)((nblocks + 255) / 256));
    if (wt == TLHIP_Q4_0)
        hipLaunchKernelGGL((repack_kernel<18, 16>), grid, dim3(256), 0, s, blocks, (uint8_t*)data, d,
                           nblocks, bpr, dst_row0, dst_step, to_gguf);
    else
        hipLaunchKernelGGL((repack_kernel<34, 32>), grid, dim3(256), 0, s, blocks, (uint8_t*)data, d,
                           nblocks, bpr, dst_row0, dst_step, to_gguf);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// dequantisation to f16 (bit-exact with gguf.rs dequantize_q4_0 / q8_0)
// one thread per block; 32 outputs written as 4 x 16 bytes
// ---------------------------------------------------------------------------
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


// one thread per 32-element group; 32 outputs as 4 x 16 bytes
__global__ void dequant_q6k_kernel(const uint8_t* __restrict__ q4, const uint8_t* __restrict__ q2,
                                   const int8_t* __restrict__ sc, const uint16_t* __restrict__ d,
                                   uint16_t* __restrict__ out, int64_t ngroups) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= ngroups) return;
    const u4 q = *(const u4*)(q4 + g * 16);
    const uint2 h = *(const uint2*)(q2 + g * 8);
    const float dv = h2f(d[g / 8]);
    h2 r[16];
    q6k_unpack(q, h.x, h.y, dv * (float)sc[2 * g], dv * (float)sc[2 * g + 1], r);
    uint32_t o32[16];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        o32[2 * t] = pack_lo(as_u32(r[2 * t]), as_u32(r[2 * t + 1]));       // (e4t, e4t+1)
        o32[2 * t + 1] = pack_hi(as_u32(r[2 * t]), as_u32(r[2 * t + 1]));   // (e4t+2, e4t+3)
        o32[8 + 2 * t] = pack_lo(as_u32(r[8 + 2 * t]), as_u32(r[8 + 2 * t + 1]));
        o32[8 + 2 * t + 1] = pack_hi(as_u32(r[8 + 2 * t]), as_u32(r[8 + 2 * t + 1]));
    }
    u4* o = (u4*)(out + g * 32);
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = u4{o32[4 * i], o32[4 * i + 1], o32[4 * i + 2], o32[4 * i + 3]};
}

tlhip_status launch_dequant(hipStream_t s, tlhip_dtype wt, const void* qs, const uint16_t* d,
                            uint16_t* out, int64_t N, int64_t K) {
    int64_t nb = N * K / 32;
    if (nb <= 0) return TLHIP_OK;
    dim3 grid((unsigned)((nb + 255) / 256));
    if (wt == TLHIP_Q6_K) {
        const uint8_t* base = (const uint8_t*)qs;
        hipLaunchKernelGGL(dequant_q6k_kernel, grid, dim3(256), 0, s, base, base + q6k_q2_offset(N, K),
                           (const int8_t*)(base + q6k_sc_offset(N, K)), d, out, nb);
        return TLHIP_OK;
    }
    if (wt == TLHIP_Q4_0)
        hipLaunchKernelGGL(dequant_q4_0_kernel, grid, dim3(256), 0, s, (const uint8_t*)qs, d, out, nb);
    else
        hipLaunchKernelGGL(dequant_q8_0_kernel, grid, dim3(256), 0, s, (const uint8_t*)qs, d, out, nb);
    return TLHIP_OK;
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
    if (lane == 0)
        p.y[(size_t)m * p.ldy + row] = epilogue_v(p.epi, acc, p.bias ? p.bias[row] : 0,
                                                  p.resid ? p.resid[(size_t)m * p.N + row] : 0);
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

template <int WT, int NB>
static void launch_m1_ri(hipStream_t s, const Gemv1Params& p, int ri) {
    const int waves = (p.N + ri - 1) / ri;
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (ri == 2) hipLaunchKernelGGL((gemv_m1_kernel<WT, NB, 2>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gemv_m1_kernel<WT, NB, 1>), grid, dim3(256), 0, s, p);
}

template <int WT>
static bool launch_m1(hipStream_t s, const GemvParams& g, int nb, int ri) {
    const Gemv1Params p = {g.x, g.wq, g.wd, g.bias, g.resid, g.y, g.N, g.K, g.epi};
    if (launch_m1_epi(s, (tlhip_dtype)WT, p, nb, ri)) return true;
    switch (nb) {
        case 1: launch_m1_ri<WT, 1>(s, p, ri); return true;
        case 2: launch_m1_ri<WT, 2>(s, p, ri); return true;
        case 3: launch_m1_ri<WT, 3>(s, p, ri); return true;
        case 4: launch_m1_ri<WT, 4>(s, p, ri); return true;
        case 5: case 6: launch_m1_ri<WT, 6>(s, p, ri); return true;
        case 7: case 8: launch_m1_ri<WT, 8>(s, p, ri); return true;
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

// Normalised GEMV shapes: rows per wave and waves per workgroup chosen by
// the measured optimum of the decoder's shapes on MI355X (more rows per
// workgroup amortise the staging; tall matrices take 4 rows per wave).
template <int WT>
static bool launch_norm(hipStream_t s, const GemvParams& p, int nb, int pro) {
    if (launch_norm_epi(s, (tlhip_dtype)WT, p, nb, pro)) return true;
    if (nb == 1) {
        if (pro == PRO_RMS) launch_norm_shape<WT, 1, PRO_RMS>(s, p);
        else launch_norm_shape<WT, 1, PRO_LN>(s, p);
        return true;
    }
    if (nb == 2) {
        if (pro == PRO_RMS) launch_norm_shape<WT, 2, PRO_RMS>(s, p);
        else launch_norm_shape<WT, 2, PRO_LN>(s, p);
        return true;
    }
    return false;
}

int gemv_norm_slots(int N) {
    if (N >= 16384) return (N + 31) / 32;
    if (N >= 8192) return (N + 15) / 16;
    return (N + 7) / 8;
}

static GemvParams make_params(const GemvArgs& a, int epi) {
    GemvParams p = {};
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
    p.norm_w = a.norm_w;
    p.norm_b = a.norm_b;
    p.eps = a.eps;
    p.nq = a.nq;
    p.nk = a.nk;
    p.head_dim = a.head_dim;
    p.rot = a.rot;
    p.layout = a.layout;
    p.pos0 = a.pos0;
    p.rope_tab = a.rope_tab;
    p.d_pos = a.d_pos;
    p.q_out = a.q_out;
    p.kc = a.kc;
    p.vc = a.vc;
    p.embd = a.embd;
    p.d_token = a.d_token;
    p.x_out = a.x_out;
    p.xn_out = a.xn_out;
    p.amax_slots = a.amax_slots;
    p.x_add = a.x_add;
    return p;
}

tlhip_status launch_gemv(hipStream_t s, tlhip_dtype wt, const GemvArgs& a, int epi) {
    const GemvParams p = make_params(a, epi);
    if (p.N <= 0 || p.M <= 0) return TLHIP_OK;
    const bool pair_epi = epi == EPI_SWIGLU_PAIR || epi == EPI_QKV_ROPE;
    if (pair_epi && (p.N % 2))
        return fail(TLHIP_ERR_INVALID_DIMENSION, "gemv: paired epilogue needs an even row count (N=%d)", p.N);
    if (epi == EPI_QKV_ROPE && (p.head_dim <= 0 || p.head_dim % 2 || p.rot % 2 || p.rot > p.head_dim ||
                                p.nq % p.head_dim || p.nk % p.head_dim || p.nq + 2 * p.nk != p.N ||
                                !p.rope_tab || !p.q_out || !p.kc || !p.vc))
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "gemv: inconsistent QKV/RoPE epilogue arguments");
    const bool normed = a.pro != PRO_NONE;
    if (normed && (p.M != 1 || !p.norm_w || (a.pro == PRO_LN && !p.norm_b) || (p.embd && !p.d_token)))
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "gemv: fused normalisation needs M = 1 and its weights");
    if (epi == EPI_ARGMAX && (!normed || !p.amax_slots))
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "gemv: the argmax epilogue runs on the normalised GEMV");
    if (!normed && (p.embd || epi == EPI_ARGMAX || epi == EPI_QKV_ROPE))
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "gemv: embedding source needs the normalised GEMV");
    if (p.embd && epi != EPI_QKV_ROPE)
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "gemv: the embedding-row source is read by the QKV epilogue only");
    bool done = false;
    if (p.K % 32 == 0 && p.K > 0) {
        const int nbr = p.K / 32;
        const int nb = (nbr + 63) / 64;
        if (wt == TLHIP_Q6_K && p.K % 256 != 0) {
            done = false;
        } else if (normed) {
            if (wt == TLHIP_Q4_0) done = launch_norm<TLHIP_Q4_0>(s, p, nb, a.pro);
            else if (wt == TLHIP_Q8_0) done = launch_norm<TLHIP_Q8_0>(s, p, nb, a.pro);
            else if (wt == TLHIP_Q6_K) done = launch_norm<TLHIP_Q6_K>(s, p, nb, a.pro);
            else done = launch_norm<TLHIP_F16>(s, p, nb, a.pro);
        } else {
            // two rows per wave: the measured optimum for the decoder's shapes
            // (5632 x 2048 and 2048 x 5632); paired epilogues need it anyway
            int ri = p.N >= 1024 ? 2 : 1;
            if (pair_epi) ri = 2;
            if (p.M == 1 && !pair_epi) {   // single-row epilogues: the compact M = 1 kernel
                // one row per wave once a row takes three or more 64-block
                // passes (measured on MI355X, Q4_0 under graph replay:
                // [2560 x 10240] 7.96 -> 6.66 us, [2048 x 5632] 3.93 -> 3.87 us;
                // at K = 2048 two rows per wave stay faster, 2.58 vs 2.72 us)
                const int ri1 = nb >= 3 ? 1 : ri;
                if (wt == TLHIP_Q4_0) done = launch_m1<TLHIP_Q4_0>(s, p, nb, ri1);
                else if (wt == TLHIP_Q8_0) done = launch_m1<TLHIP_Q8_0>(s, p, nb, ri1);
                else if (wt == TLHIP_Q6_K) done = launch_m1<TLHIP_Q6_K>(s, p, nb, ri1);
                else done = launch_m1<TLHIP_F16>(s, p, nb, ri1);
            } else if (wt == TLHIP_Q4_0) done = launch_mx<TLHIP_Q4_0>(s, p, nb, ri);
            else if (wt == TLHIP_Q8_0) done = launch_mx<TLHIP_Q8_0>(s, p, nb, ri);
            else if (wt == TLHIP_Q6_K) done = launch_mx<TLHIP_Q6_K>(s, p, nb, ri);
            else done = launch_mx<TLHIP_F16>(s, p, nb, ri);
        }
    }
    if (!done) {
        if (wt != TLHIP_F16 || pair_epi || normed)
            return fail(TLHIP_ERR_INVALID_OPERATION, "gemv: unsupported shape M=%d K=%d", p.M, p.K);
        int64_t waves = (int64_t)p.N * p.M;
        hipLaunchKernelGGL(gemv_generic_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, p);
    }
    return TLHIP_OK;
}

// Final step of the fused greedy argmax: the largest of the workgroup keys
// (value, then index) is the token; advances the device decode state
// {token, pos, step} and logs the token, as argmax_kernel does.
__global__ __launch_bounds__(256) void argmax_slots_kernel(const unsigned long long* __restrict__ slots, int n,
                                                           int32_t* out, int32_t* token_log, int32_t* d_state) {
    __shared__ unsigned long long wk[4];
    // the state words are read with the keys, not after them
    const int32_t step = d_state ? d_state[2] : 0;
    const int32_t pos = d_state ? d_state[1] : 0;
    unsigned long long b = 0ull;
    // 8 keys per thread per round, all loads issued before the first max
    // (indices clamped to the last slot, a duplicate that cannot change the
    // maximum): one memory round trip for up to 2048 slots, where a plain
    // strided loop waits for each of its loads in turn
    for (int base = 0; base < n; base += 256 * 8) {
        unsigned long long v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = slots[min(base + (int)threadIdx.x + 256 * k, n - 1)];
#pragma unroll
        for (int k = 0; k < 8; k++) b = umax64(b, v[k]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)b, off, 64), hi = __shfl_xor((uint32_t)(b >> 32), off, 64);
        b = umax64(b, ((unsigned long long)hi << 32) | lo);
    }
    if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = b;
    __syncthreads();
    if (threadIdx.x == 0) {
        b = umax64(umax64(wk[0], wk[1]), umax64(wk[2], wk[3]));
        const int tok = (b >> 32) == 0ull ? 0 : (int)(uint32_t)b;
        if (out) out[0] = tok;
        if (d_state) {
            if (token_log) token_log[step] = tok;
            d_state[0] = tok;
            d_state[1] = pos + 1;
            d_state[2] = step + 1;
        }
    }
}

tlhip_status launch_argmax_slots(hipStream_t s, const unsigned long long* slots, int n, int32_t* out,
                                 int32_t* token_log, int32_t* d_state) {
    if (n <= 0) return fail(TLHIP_ERR_INVALID_DIMENSION, "argmax over no slots");
    hipLaunchKernelGGL(argmax_slots_kernel, dim3(1), dim3(256), 0, s, slots, n, out, token_log, d_state);
    return TLHIP_OK;
}

}  // namespace tlhip
