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

__device__ __forceinline__ void q4_unpack_g(uint32_t w, h2 dd, h2 out[4]) {
    const h2 bias = {(h16)-1032.0f, (h16)-1032.0f};
    out[0] = (as_h2((w & 0x000F000Fu) | 0x64006400u) + bias) * dd;
    out[1] = (as_h2(((w >> 8) & 0x000F000Fu) | 0x64006400u) + bias) * dd;
    out[2] = (as_h2(((w >> 4) & 0x000F000Fu) | 0x64006400u) + bias) * dd;
    out[3] = (as_h2(((w >> 12) & 0x000F000Fu) | 0x64006400u) + bias) * dd;
}

__device__ __forceinline__ void q8_unpack_g(uint32_t w, h2 dd, h2 out[2]) {
    const h2 bias = {(h16)-1152.0f, (h16)-1152.0f};
    uint32_t v = w ^ 0x80808080u;
    out[0] = (as_h2((v & 0x00FF00FFu) | 0x64006400u) + bias) * dd;
    out[1] = (as_h2(((v >> 8) & 0x00FF00FFu) | 0x64006400u) + bias) * dd;
}

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
                q4_unpack_g(w, dd, r);
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
                q8_unpack_g(w0, dd, r);
                *(uint32_t*)&Bs[lr][8 * lq + 0] = pack_lo(as_u32(r[0]), as_u32(r[1]));
                *(uint32_t*)&Bs[lr][8 * lq + 2] = pack_hi(as_u32(r[0]), as_u32(r[1]));
                q8_unpack_g(w1, dd, r);
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
    if (p.M <= 0 || p.N <= 0) return TLHIP_OK;
    if (p.K % 32 != 0) {
        if (wt != TLHIP_F16 || epi == EPI_SWIGLU_PAIR)
            return fail(TLHIP_ERR_INVALID_OPERATION, "gemm: K=%d not a multiple of 32", p.K);
        int64_t n = (int64_t)p.M * p.N;
        hipLaunchKernelGGL(gemm_naive_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p);
        return TLHIP_OK;
    }
    dim3 grid((unsigned)((p.N + GBN - 1) / GBN), (unsigned)((p.M + GBM - 1) / GBM));
    if (wt == TLHIP_Q4_0) hipLaunchKernelGGL(gemm_kernel<TLHIP_Q4_0>, grid, dim3(256), 0, s, p);
    else if (wt == TLHIP_Q8_0) hipLaunchKernelGGL(gemm_kernel<TLHIP_Q8_0>, grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL(gemm_kernel<TLHIP_F16>, grid, dim3(256), 0, s, p);
    return TLHIP_OK;
}

}  // namespace tlhip
