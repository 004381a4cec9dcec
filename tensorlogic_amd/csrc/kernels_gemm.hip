// kernels_gemm.hip -- dequant-GEMM for prefill (M > 4) on MFMA, gfx950.
//
// y[M, N] = x[M, K] . W[N, K]^T, W packed Q4_0 / Q8_0 or f16.  Each K step
// stages an activation tile and a weight tile in LDS; the weight tile is
// dequantised while it is written to LDS (RNE_f16((q-8)*d) / RNE_f16(q*d)
// with v_pk_mul_f16, the exact values of gguf.rs:22-112), then
// v_mfma_f32_32x32x8_f16 accumulates in fp32 as the reference's tiled
// matmul does (unified.metal:4291-4348).  Output f16 with the same epilogues
// as the GEMV (bias, residual add, SwiGLU on interleaved gate/up rows).
//
// Tile: 64 (M) x 64 (N) x 32 (K, one quant block) per 256-thread workgroup;
// four waves in a 2 x 2 arrangement, each owning a 32 x 32 accumulator.
#include "device_common.hpp"
#include "internal.hpp"

namespace tlhip {

struct GemmParams {
    const uint16_t* x;
    const uint8_t* wq;
    const uint16_t* wd;
    const uint16_t* bias;
    const uint16_t* resid;
    uint16_t* y;
    int M, N, K, ldy, epi;
};

constexpr int GBM = 64, GBN = 64, GBK = 32, GPAD = 8;

typedef h16 h4 __attribute__((ext_vector_type(4)));

template <int WT>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t As[GBM][GBK + GPAD];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[GBN][GBK + GPAD];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * GBM, n0 = blockIdx.x * GBN;
    const int nbr = p.K >> 5;
    f16v acc = {0};

    const int lr = tid >> 2, lq = tid & 3;   // loader row, quarter
    for (int kb = 0; kb < nbr; kb++) {
        // activation tile: 64 rows x 32 halves, 16 B per thread
        {
            const int m = m0 + lr;
            u4 v = {0u, 0u, 0u, 0u};
            if (m < p.M) v = *(const u4*)(p.x + (size_t)m * p.K + (size_t)kb * 32 + lq * 8);
            *(u4*)&As[lr][lq * 8] = v;
        }
        // weight tile: 64 rows x one block, dequantised into LDS
        {
            const int n = min(n0 + lr, p.N - 1);
            if (WT == TLHIP_Q4_0) {
                const uint8_t* qb = p.wq + (size_t)n * (p.K / 2) + (size_t)kb * 16;
                uint32_t w = *(const uint32_t*)(qb + 4 * lq);
                h16 dh = __builtin_bit_cast(h16, p.wd[(size_t)n * nbr + kb]);
                h2 dd = {dh, dh}, r[4];
                q4_unpack(w, dd, r);
                // r0=(e4q,e4q+2) r1=(e4q+1,e4q+3) r2/r3 the same at +16
                *(uint32_t*)&Bs[lr][4 * lq + 0] = pack_lo(as_u32(r[0]), as_u32(r[1]));
                *(uint32_t*)&Bs[lr][4 * lq + 2] = pack_hi(as_u32(r[0]), as_u32(r[1]));
                *(uint32_t*)&Bs[lr][16 + 4 * lq + 0] = pack_lo(as_u32(r[2]), as_u32(r[3]));
                *(uint32_t*)&Bs[lr][16 + 4 * lq + 2] = pack_hi(as_u32(r[2]), as_u32(r[3]));
            } else if (WT == TLHIP_Q8_0) {
                const uint8_t* qb = p.wq + (size_t)n * p.K + (size_t)kb * 32 + 8 * lq;
                uint32_t w0 = *(const uint32_t*)qb, w1 = *(const uint32_t*)(qb + 4);
                h16 dh = __builtin_bit_cast(h16, p.wd[(size_t)n * nbr + kb]);
                h2 dd = {dh, dh}, r[2];
                q8_unpack(w0, dd, r);
                *(uint32_t*)&Bs[lr][8 * lq + 0] = pack_lo(as_u32(r[0]), as_u32(r[1]));
                *(uint32_t*)&Bs[lr][8 * lq + 2] = pack_hi(as_u32(r[0]), as_u32(r[1]));
                q8_unpack(w1, dd, r);
                *(uint32_t*)&Bs[lr][8 * lq + 4] = pack_lo(as_u32(r[0]), as_u32(r[1]));
                *(uint32_t*)&Bs[lr][8 * lq + 6] = pack_hi(as_u32(r[0]), as_u32(r[1]));
            } else {
                const uint16_t* wr = (const uint16_t*)p.wq + (size_t)n * p.K + (size_t)kb * 32 + 8 * lq;
                *(u4*)&Bs[lr][8 * lq] = *(const u4*)wr;
            }
        }
        __syncthreads();
        // 4 x mfma 32x32x8: A rows (wm*32 + lane%32), B rows (wn*32 + lane%32)
#pragma unroll
        for (int ks = 0; ks < GBK; ks += 8) {
            const int kk = ks + 4 * (lane >> 5);
            h4 a = *(const h4*)&As[wm * 32 + (lane & 31)][kk];
            h4 b = *(const h4*)&Bs[wn * 32 + (lane & 31)][kk];
            acc = __builtin_amdgcn_mfma_f32_32x32x8f16(a, b, acc, 0, 0, 0);
        }
        __syncthreads();
    }

    // C layout: col j = lane%32 (weight row), row i = 8*(r/4) + 4*(lane/32) + r%4
    const int n = n0 + wn * 32 + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int m = m0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        float v = acc[r];
        if (p.epi == EPI_SWIGLU_PAIR) {
            float up = __shfl_down(v, 1, 64);
            if (m < p.M && n + 1 < p.N && (n & 1) == 0)
                p.y[(size_t)m * p.ldy + n / 2] = swiglu_h(f2h(v), f2h(up));
        } else if (m < p.M && n < p.N) {
            p.y[(size_t)m * p.ldy + n] = epilogue_h(p.epi, v, p.bias, p.resid, (size_t)m * p.N + n, n);
        }
    }
}

// ---------------------------------------------------------------------------
// Pipelined MFMA GEMM (K % 64 == 0): tile BM x BN x 64 (two quant blocks per
// K step), 256 threads as WM x WN waves, each wave owning (BM/WM) x (BN/WN)
// of C in 32 x 32 v_mfma_f32_32x32x16_f16 tiles.  Two LDS buffers: the
// global loads of step k+1 are issued into registers before the MFMAs of
// step k, then dequantised into the other buffer (one barrier per step).
// With split-K (gridDim.z > 1) each z-slice writes fp32 partials of a
// contiguous K range and gemm_reduce_kernel sums the slices in z order and
// applies the epilogue.
// ---------------------------------------------------------------------------
constexpr int G2_BK = 64, G2_PAD = 8;

template <int WT, int BN>
struct G2W {   // per-thread global weight registers of one K step
    static constexpr int NV = WT == TLHIP_F16 ? BN * 8 / 256 : (WT == TLHIP_Q8_0 ? BN * 4 / 256 : (BN * 2 + 255) / 256);
};

template <int WT, int BM, int BN>
__device__ __forceinline__ void g2_load(const GemmParams& p, int m0, int n0, int kt, int tid,
                                        u4 (&xr)[BM * 8 / 256], u4 (&wr)[G2W<WT, BN>::NV], uint16_t& dsc) {
    constexpr int XV = BM * 8 / 256;          // 16-byte chunks of x per thread
    constexpr int TPR = 8 / XV;               // threads per x row
    const int nbr = p.K >> 5;
    {
        const int r = tid / TPR, c0 = (tid % TPR) * XV;
        const int m = m0 + r;
#pragma unroll
        for (int v = 0; v < XV; v++)
            xr[v] = m < p.M ? *(const u4*)(p.x + (size_t)m * p.K + (size_t)kt * G2_BK + 8 * (c0 + v)) : u4{0u, 0u, 0u, 0u};
    }
    if (WT == TLHIP_Q4_0) {
        // (row, block) pairs: tid -> row tid/2, block tid%2; 16 payload bytes + scale
        if (tid < BN * 2) {
            const int n = min(n0 + (tid >> 1), p.N - 1), b = 2 * kt + (tid & 1);
            wr[0] = *(const u4*)(p.wq + (size_t)n * (p.K / 2) + (size_t)b * 16);
            dsc = p.wd[(size_t)n * nbr + b];
        }
    } else if (WT == TLHIP_Q8_0) {
        // tid -> row tid/4, block (tid/2)%2, half tid%2: 16 int8 + scale
        const int n = min(n0 + (tid >> 2), p.N - 1), b = 2 * kt + ((tid >> 1) & 1);
        wr[0] = *(const u4*)(p.wq + (size_t)n * p.K + (size_t)b * 32 + 16 * (tid & 1));
        dsc = p.wd[(size_t)n * nbr + b];
    } else {
        constexpr int NV = G2W<WT, BN>::NV;
        const int r = tid / (8 / NV), c0 = (tid % (8 / NV)) * NV;
        const int n = min(n0 + r, p.N - 1);
#pragma unroll
        for (int v = 0; v < NV; v++)
            wr[v] = *(const u4*)((const uint16_t*)p.wq + (size_t)n * p.K + (size_t)kt * G2_BK + 8 * (c0 + v));
    }
}

template <int WT, int BM, int BN>
__device__ __forceinline__ void g2_store(int tid, const u4 (&xr)[BM * 8 / 256], const u4 (&wr)[G2W<WT, BN>::NV],
                                         uint16_t dsc, uint16_t (*As)[G2_BK + G2_PAD],
                                         uint16_t (*Bs)[G2_BK + G2_PAD]) {
    constexpr int XV = BM * 8 / 256;
    constexpr int TPR = 8 / XV;
    {
        const int r = tid / TPR, c0 = (tid % TPR) * XV;
#pragma unroll
        for (int v = 0; v < XV; v++) *(u4*)&As[r][8 * (c0 + v)] = xr[v];
    }
    if (WT == TLHIP_Q4_0) {
        if (tid < BN * 2) {
            const int r = tid >> 1, c = 32 * (tid & 1);
            const h16 dh = __builtin_bit_cast(h16, dsc);
            const h2 dd = {dh, dh};
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                h2 q[4];
                q4_unpack(wr[0][t], dd, q);
                lo[2 * t] = pack_lo(as_u32(q[0]), as_u32(q[1]));
                lo[2 * t + 1] = pack_hi(as_u32(q[0]), as_u32(q[1]));
                hi[2 * t] = pack_lo(as_u32(q[2]), as_u32(q[3]));
                hi[2 * t + 1] = pack_hi(as_u32(q[2]), as_u32(q[3]));
            }
            *(u4*)&Bs[r][c + 0] = u4{lo[0], lo[1], lo[2], lo[3]};
            *(u4*)&Bs[r][c + 8] = u4{lo[4], lo[5], lo[6], lo[7]};
            *(u4*)&Bs[r][c + 16] = u4{hi[0], hi[1], hi[2], hi[3]};
            *(u4*)&Bs[r][c + 24] = u4{hi[4], hi[5], hi[6], hi[7]};
        }
    } else if (WT == TLHIP_Q8_0) {
        const int r = tid >> 2, c = 32 * ((tid >> 1) & 1) + 16 * (tid & 1);
        const h16 dh = __builtin_bit_cast(h16, dsc);
        const h2 dd = {dh, dh};
        uint32_t o[8];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            h2 q[2];
            q8_unpack(wr[0][t], dd, q);
            o[2 * t] = pack_lo(as_u32(q[0]), as_u32(q[1]));
            o[2 * t + 1] = pack_hi(as_u32(q[0]), as_u32(q[1]));
        }
        *(u4*)&Bs[r][c + 0] = u4{o[0], o[1], o[2], o[3]};
        *(u4*)&Bs[r][c + 8] = u4{o[4], o[5], o[6], o[7]};
    } else {
        constexpr int NV = G2W<WT, BN>::NV;
        const int r = tid / (8 / NV), c0 = (tid % (8 / NV)) * NV;
#pragma unroll
        for (int v = 0; v < NV; v++) *(u4*)&Bs[r][8 * (c0 + v)] = wr[v];
    }
}

__device__ __forceinline__ void gemm_store_one(const GemmParams& p, int m, int n, float v) {
    if (p.epi == EPI_SWIGLU_PAIR) {
        const float up = __shfl_down(v, 1, 64);
        if (m < p.M && n + 1 < p.N && (n & 1) == 0) p.y[(size_t)m * p.ldy + n / 2] = swiglu_h(f2h(v), f2h(up));
    } else if (m < p.M && n < p.N) {
        p.y[(size_t)m * p.ldy + n] = epilogue_h(p.epi, v, p.bias, p.resid, (size_t)m * p.N + n, n);
    }
}

template <int WT, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(256) void gemm2_kernel(GemmParams p, float* __restrict__ part) {
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][G2_BK + G2_PAD];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN][G2_BK + G2_PAD];
    constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
    constexpr int XV = BM * 8 / 256;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int nkt = p.K / G2_BK;
    const int kt0 = (int)((int64_t)nkt * blockIdx.z / gridDim.z), kt1 = (int)((int64_t)nkt * (blockIdx.z + 1) / gridDim.z);
    f16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = f16v{0};

    u4 xr[XV], wr[G2W<WT, BN>::NV];
    uint16_t dsc = 0;
    if (kt0 < kt1) {
        g2_load<WT, BM, BN>(p, m0, n0, kt0, tid, xr, wr, dsc);
        g2_store<WT, BM, BN>(tid, xr, wr, dsc, As[0], Bs[0]);
    }
    __syncthreads();
    for (int kt = kt0; kt < kt1; kt++) {
        const int buf = (kt - kt0) & 1;
        const bool more = kt + 1 < kt1;
        if (more) g2_load<WT, BM, BN>(p, m0, n0, kt + 1, tid, xr, wr, dsc);
#pragma unroll
        for (int ks = 0; ks < G2_BK; ks += 16) {
            const int kk = ks + 8 * (lane >> 5);
            h8 a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) a[i] = *(const h8*)&As[buf][wm * (BM / WM) + 32 * i + (lane & 31)][kk];
#pragma unroll
            for (int j = 0; j < TN; j++) b[j] = *(const h8*)&Bs[buf][wn * (BN / WN) + 32 * j + (lane & 31)][kk];
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (more) g2_store<WT, BM, BN>(tid, xr, wr, dsc, As[buf ^ 1], Bs[buf ^ 1]);
        __syncthreads();
    }

    // C layout: col = lane%32 (weight row n), row = 8*(r/4) + 4*(lane/32) + r%4 (activation row m)
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + wn * (BN / WN) + 32 * j + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * (BM / WM) + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const float v = acc[i][j][r];
                if (part) {
                    if (m < p.M && n < p.N) part[((size_t)blockIdx.z * p.M + m) * p.N + n] = v;
                } else {
                    gemm_store_one(p, m, n, v);
                }
            }
        }
}

// Sum of the split-K partials in slice order, then the epilogue.
__global__ void gemm_reduce_kernel(GemmParams p, const float* __restrict__ part, int splits) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)p.M * p.N;
    if (i >= total) return;
    const int m = (int)(i / p.N), n = (int)(i % p.N);
    float v = part[i];
    for (int z = 1; z < splits; z++) v += part[(size_t)z * total + i];
    if (p.epi == EPI_SWIGLU_PAIR) {
        if ((n & 1) == 0 && n + 1 < p.N) {
            float up = part[i + 1];
            for (int z = 1; z < splits; z++) up += part[(size_t)z * total + i + 1];
            p.y[(size_t)m * p.ldy + n / 2] = swiglu_h(f2h(v), f2h(up));
        }
    } else {
        p.y[(size_t)m * p.ldy + n] = epilogue_h(p.epi, v, p.bias, p.resid, (size_t)m * p.N + n, n);
    }
}

template <int WT>
static void launch_gemm2(hipStream_t s, const GemmParams& p, int splits, float* part) {
    if (p.M > 64) {
        dim3 grid((unsigned)((p.N + 63) / 64), (unsigned)((p.M + 127) / 128), (unsigned)splits);
        hipLaunchKernelGGL((gemm2_kernel<WT, 128, 64, 2, 2>), grid, dim3(256), 0, s, p, part);
    } else {
        dim3 grid((unsigned)((p.N + 63) / 64), (unsigned)((p.M + 63) / 64), (unsigned)splits);
        hipLaunchKernelGGL((gemm2_kernel<WT, 64, 64, 2, 2>), grid, dim3(256), 0, s, p, part);
    }
}

// split-K slices for a grid of `tiles` output tiles: enough workgroups to
// cover the 256 CUs about once, at least 4 K steps per slice.
int gemm_splits(int M, int N, int K) {
    if (K % G2_BK) return 1;
    const int tiles = ((N + 63) / 64) * (M > 64 ? (M + 127) / 128 : (M + 63) / 64);
    int sp = 1;
    while (sp < 8 && tiles * sp * 2 <= 512 && (K / G2_BK) / (sp * 2) >= 4) sp *= 2;
    return sp;
}

// Naive fp32-accumulate GEMM for f16 weights whose K is not a multiple of 32
// (reference unit-test shapes such as [50, 122]).
__global__ void gemm_naive_kernel(GemmParams p) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)p.M * p.N) return;
    int m = (int)(idx / p.N), n = (int)(idx % p.N);
    const uint16_t* w = (const uint16_t*)p.wq + (size_t)n * p.K;
    const uint16_t* x = p.x + (size_t)m * p.K;
    float acc = 0.0f;
    for (int k = 0; k < p.K; k++) acc += h2f(x[k]) * h2f(w[k]);
    p.y[(size_t)m * p.ldy + n] = epilogue_h(p.epi, acc, p.bias, p.resid, (size_t)m * p.N + n, n);
}

tlhip_status launch_gemm(hipStream_t s, tlhip_dtype wt, const GemvArgs& a, int epi) {
    GemmParams p;
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
    if (epi == EPI_QKV_ROPE || a.pro != PRO_NONE)
        return fail(TLHIP_ERR_INVALID_OPERATION, "gemm: fused normalisation / RoPE epilogue is GEMV-only");
    if (wt != TLHIP_F16 && wt != TLHIP_Q4_0 && wt != TLHIP_Q8_0)
        return fail(TLHIP_ERR_DTYPE, "gemm: weight dtype %d takes the dequantised f16 path", (int)wt);
    if (p.M <= 0 || p.N <= 0) return TLHIP_OK;
    if (p.K % 32 != 0) {
        if (wt != TLHIP_F16 || epi == EPI_SWIGLU_PAIR)
            return fail(TLHIP_ERR_INVALID_OPERATION, "gemm: K=%d not a multiple of 32", p.K);
        int64_t n = (int64_t)p.M * p.N;
        hipLaunchKernelGGL(gemm_naive_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p);
        return TLHIP_OK;
    }
    if (p.K % G2_BK == 0) {
        int splits = a.ws ? gemm_splits(p.M, p.N, p.K) : 1;
        if ((size_t)splits * p.M * p.N * sizeof(float) > a.ws_bytes) splits = 1;
        float* part = splits > 1 ? a.ws : nullptr;
        if (wt == TLHIP_Q4_0) launch_gemm2<TLHIP_Q4_0>(s, p, splits, part);
        else if (wt == TLHIP_Q8_0) launch_gemm2<TLHIP_Q8_0>(s, p, splits, part);
        else launch_gemm2<TLHIP_F16>(s, p, splits, part);
        if (splits > 1) {
            const int64_t total = (int64_t)p.M * p.N;
            hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, p,
                               (const float*)part, splits);
        }
        return TLHIP_OK;
    }
    dim3 grid((unsigned)((p.N + GBN - 1) / GBN), (unsigned)((p.M + GBM - 1) / GBM));
    if (wt == TLHIP_Q4_0) hipLaunchKernelGGL(gemm_kernel<TLHIP_Q4_0>, grid, dim3(256), 0, s, p);
    else if (wt == TLHIP_Q8_0) hipLaunchKernelGGL(gemm_kernel<TLHIP_Q8_0>, grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL(gemm_kernel<TLHIP_F16>, grid, dim3(256), 0, s, p);
    return TLHIP_OK;
}

}  // namespace tlhip
