// kernels_gemm.hip -- dequant-GEMM for prefill (M > 4) on MFMA, gfx950.
//
// y[M, N] = x[M, K] . W[N, K]^T, W packed Q4_0 / Q8_0 or f16.  Each K step
// stages an activation tile and a weight tile in LDS; the weight tile is
// dequantised while it is written to LDS (RNE_f16((q-8)*d) / RNE_f16(q*d)
// with v_pk_mul_f16, the exact values of gguf.rs:22-112), then the matrix
// cores accumulate in fp32 as the reference's tiled matmul does
// (unified.metal:4291-4348): v_mfma_f32_32x32x16_f16 in gemm2_kernel and
// gemm_lds_kernel, v_mfma_f32_16x16x32_f16 in gemm_skinny_kernel, and
// v_mfma_f32_32x32x8_f16 in the K % 64 != 0 fallback gemm_kernel.  Output
// f16 with the same epilogues as the GEMV (bias, residual add, SwiGLU on
// interleaved gate/up rows).
//
// Four kernels: gemm_kernel (K % 64 != 0; 64 x 64 x 32 tiles),
// gemm_skinny_kernel (M <= 64: a ring of LDS stages per wave filled by
// direct global->LDS loads, split over K with a fence-free exchange),
// gemm2_kernel (register-staged, two LDS buffers, where the skinny plan does
// not apply) and gemm_lds_kernel (M > 64: 128 x 128 tiles, three or four
// LDS stages filled by direct global->LDS loads).
#include <type_traits>

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
    // skinny GEMM split over K: fp32 partials [splits][M][N] and one arrival
    // counter per 32-row tile (zero between launches)
    float* part = nullptr;
    uint32_t* flags = nullptr;
    int splits = 1;
    int mtiles = 1;   // skinny GEMM: workgroups along M
    // skinny GEMM, EPI_QKV_ROPE: columns [0, nq) are q, [nq, nq + nk) k, the
    // rest v; row m is position pos0 + m (as the GEMV's fused epilogue)
    int nq = 0, nk = 0, head_dim = 0, rot = 0, layout = 0, pos0 = 0;
    const float* rope_tab = nullptr;
    uint16_t* q_out = nullptr;
    uint16_t* kc = nullptr;
    uint16_t* vc = nullptr;
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

// ---------------------------------------------------------------------------
// Multi-stage MFMA dequant-GEMM (K % 64 == 0).  Workgroup tile BM x BN x 64,
// 512 threads = 8 waves in a 2 (M) x 4 (N) grid, each wave (BM/2) x (BN/4) of
// C in 32 x 32 v_mfma_f32_32x32x16_f16 tiles.  NS LDS stages are filled by
// direct global->LDS loads (global_load_lds_dwordx4 / _dword, no VGPR
// staging), so NS - 1 K steps are in flight while one is computed.  The LDS
// keeps the GGUF payload as stored (Q4_0 nibbles, Q8_0 int8 or f16) plus the
// block scales; each wave dequantises its B operand from LDS into registers
// right before its MFMAs, with the same RNE_f16((q-8)*d) / RNE_f16(q*d) as
// every other path.
//
// K order inside a 64-wide step: MFMA lane half h (lane / 32) carries the
// elements 32h + 8t .. 32h + 8t + 7 at sub-step t = 0..3 (quant block h of
// the step) for A and B alike, so every k is summed once in fp32.
//
// LDS rows are XOR-swizzled in 16-byte chunks so that the 32 rows a wave
// reads at one chunk index fall in distinct banks: A / f16 B rows (128 B)
// chunk c -> c ^ ((r >> 1) & 7); Q8_0 rows (64 B) c -> c ^ ((r >> 2) & 3); Q4_0 rows
// (32 B) c -> c ^ ((r >> 3) & 1).  A direct load writes lane l's 16 (4) bytes
// at LDS base + 16 l (4 l); each lane fetches the global chunk that the
// swizzle puts in its slot.
//
// Workgroups are dispatched round-robin over the 8 XCDs (workgroup id mod
// 8); the id -> tile map gives each XCD a contiguous run of tiles with the
// M tiles of one N tile adjacent, so the BM-row tiles that share a weight
// tile run on one XCD and read it through one L2.
// ---------------------------------------------------------------------------

template <int WT>
struct GlRow {   // LDS bytes of one weight row per 64-wide K step
    static constexpr int B = WT == TLHIP_F16 ? 128 : (WT == TLHIP_Q8_0 ? 64 : 32);
};

// direct loads of one LDS region of R bytes by 512 threads: 16-byte loads
// when R is a multiple of 8 KB, else 4-byte loads (R multiple of 2 KB)
template <int R>
struct GlDma {
    static constexpr int SZ = R % 8192 == 0 ? 16 : 4;
    static constexpr int N = R / (512 * SZ);
    static_assert(R % 2048 == 0, "region");
};

template <int WT, int BM, int BN, int NS>
struct Gl {
    static constexpr int A_BYTES = BM * 128;
    static constexpr int B_BYTES = BN * GlRow<WT>::B;
    static constexpr int S_BYTES = WT == TLHIP_F16 ? 0 : BN * 4;
    static constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;
    static constexpr int VMC = GlDma<A_BYTES>::N + GlDma<B_BYTES>::N + (S_BYTES ? 1 : 0);
    static_assert((NS - 2) * VMC < 64, "vmcnt range");
    static_assert(BN / 8 <= 64, "scale rows per wave");
};

template <int N>
__device__ __forceinline__ void gl_wait_vm() {   // s_waitcnt vmcnt(N), gfx9 encoding
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}
template <int VMC, int K>
__device__ __forceinline__ void gl_wait_stage(int ahead) {   // wait until <= ahead stages outstanding
    if constexpr (K == 0) {
        gl_wait_vm<0>();
    } else {
        if (ahead >= K) gl_wait_vm<K * VMC>();
        else gl_wait_stage<VMC, K - 1>(ahead);
    }
}

template <int SZ>
__device__ __forceinline__ void gl_dma(const void* g, uint8_t* lds) {
    if constexpr (SZ == 16) __builtin_amdgcn_global_load_lds(g, (gl_lds_t)lds, 16, 0, 0);
    else __builtin_amdgcn_global_load_lds(g, (gl_lds_t)lds, 4, 0, 0);
}

// Four payload bytes -> two f16 pairs in element order (e0,e1) (e2,e3).
__device__ __forceinline__ void q8_pairs(uint32_t w, h2 dd, uint32_t& p01, uint32_t& p23) {
    const h2 bias = {(h16)-1152.0f, (h16)-1152.0f};
    const uint32_t v = w ^ 0x80808080u;
    p01 = as_u32((as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x04010400u)) + bias) * dd);
    p23 = as_u32((as_h2(__builtin_amdgcn_perm(0x64646464u, v, 0x04030402u)) + bias) * dd);
}
__device__ __forceinline__ void q4_pairs(uint32_t nib, h2 dd, uint32_t& p01, uint32_t& p23) {
    const h2 bias = {(h16)-1032.0f, (h16)-1032.0f};
    p01 = as_u32((as_h2(__builtin_amdgcn_perm(0x64646464u, nib, 0x04010400u)) + bias) * dd);
    p23 = as_u32((as_h2(__builtin_amdgcn_perm(0x64646464u, nib, 0x04030402u)) + bias) * dd);
}

__device__ __forceinline__ int gl_tile(int id, int T) {   // XCD-contiguous tile order
    const int x = id & 7, s = id >> 3, q = T >> 3, r = T & 7;
    return x * q + min(x, r) + s;
}

// ---------------------------------------------------------------------------
// Skinny dequant-GEMM (4 < M <= 64, K % 64 == 0) on v_mfma_f32_16x16x32_f16:
// one launch, no workspace by default.  A workgroup reads its activation
// rows and weight rows once; both enter the CU as whole 64-byte pieces,
// because the vector L1 handles a load one piece per lane-run of adjacent
// addresses: an MFMA operand read straight from a row-major matrix (one row
// per lane) costs one L1 access per lane, here one per 64 bytes.  What
// bounds it is the bytes each CU takes in: the activation rows (which every
// workgroup of the same rows re-reads) plus its own weight rows.  The host
// plan (sk_plan) picks per shape how many 16-row M tiles a workgroup covers
// (MT) and how many 16-row weight tiles (NT), so that the largest per-CU
// byte count is smallest.
//
// A workgroup (4 waves) owns MT x 16 activation rows and 16 NT weight rows;
// wave w takes K part w (the workgroup's 64-k steps split into 4 ranges) for
// all of them.  Each wave streams its part through a private ring of L::ST
// LDS stages with buffer loads to LDS (16 bytes per lane, adjacent lanes on
// adjacent bytes; the 16-byte pieces of a row XOR-swizzled by row so the
// operand reads below spread over the banks), then reads the operands of
// sub-step t = 0, 1 in the natural 16 x 16 x 32 layout -- lane l (tile row /
// column l % 16, group g = l / 16) holds k = 64 q + 32 t + 8 g + i:
//   A (activation row 16 mt + l % 16): 16 bytes;
//   B (weight row): f16 16 bytes; Q8_0 8 bytes of block 2q + t; Q4_0 8
//   bytes of block 2q + t (low nibbles for g < 2, high for g >= 2), with the
//   block's scale,
// dequantised with the correctly rounded RNE_f16((q - 8) d) / RNE_f16(q d)
// of every other path.  A wave issues only the stages of its own range and
// waits for a stage with the exact count of loads issued after it.  Rows
// past M and weight rows past N are read from offsets outside the buffers
// (zeros, no memory access).  The four K parts' fp32 accumulators meet in
// LDS and are added in a fixed order (part 0 + 1 + 2 + 3) before the
// epilogue.  C layout of a 16 x 16 tile: lane l holds column (weight row)
// l % 16 and activation rows 4 (l / 16) + r.
//
// K may also be split over p.splits workgroups per tile (block b: slice
// b % splits).  Each writes its fp32 tile to p.part and counts itself in on
// the tile's counter; the last to arrive adds the slices in slice order --
// the same bits whichever arrives last -- applies the epilogue and resets
// the counter to zero for the next launch, so no second kernel runs.  The
// exchange costs a few microseconds of memory round trips, so the plan
// splits only where that pays.  Every choice but the split leaves each
// output's summation order, and so its bits, unchanged.
// ---------------------------------------------------------------------------
constexpr int SK_LDS = 160 * 1024 - 1024;   // LDS the rings may take
constexpr uint32_t SK_OOB = 0x80000000u;    // a buffer offset past every tensor
constexpr int SK_MAX_SPLITS = 8;

template <int WT, int MT, int NT, int KP>
struct SkL {   // LDS bytes of one stage (one 64-k step) of one wave
    static constexpr int ROWS = 16 * NT;      // weight rows per workgroup
    static constexpr int X = MT * 16 * 128;   // activation rows, 128 bytes each
    static constexpr int WROW = WT == TLHIP_F16 ? 128 : (WT == TLHIP_Q8_0 ? 64 : 32);
    static constexpr int W = ROWS * WROW;
    static constexpr int S = WT == TLHIP_F16 ? 0 : 256;   // ROWS x 2 scales, one 4-byte load per lane
    static constexpr int STAGE = X + W + S;
    static constexpr int NX = X / 1024, NW = W / 1024, NS = S ? 1 : 0;
    static constexpr int C = NX + NW + NS;   // loads per stage
    // stages per wave: as many as the LDS holds (the deeper the ring, the
    // fewer memory round trips a wave's part takes), at most 6; a shape with
    // fewer than 2 is not launched (sk_plan)
    static constexpr int ST0 = SK_LDS / (KP * STAGE);
    static constexpr int ST = ST0 < 6 ? ST0 : 6;
    static constexpr bool OK = ST >= 2 && (ST - 1) * C < 64;
    static_assert(X % 1024 == 0 && W % 1024 == 0 && ROWS * 4 <= 256, "load shapes");
};

// wait until at most `ahead` stages of C loads each are outstanding
template <int C, int K>
__device__ __forceinline__ void sk_wait_stages(int ahead) {
    if constexpr (K == 0) {
        sk_wait_vm<0>();
    } else {
        if (ahead >= K) sk_wait_vm<K * C>();
        else sk_wait_stages<C, K - 1>(ahead);
    }
}

// Operand layout of one 64-k step (the k order inside an MFMA is free as
// long as both operands follow it).  Lane l = (column / row l % 16, group
// g = l / 16) holds at sub-step t the 8 elements k = 64 q + 8 c + i of its
// activation row, c = sk_piece(g, t), and of its weight row:
//   f16:  c = 4t + g, 16 bytes per sub-step;
//   Q8_0: c = 4(g/2) + 2(g%2) + t -- 16 bytes of block 2q + g/2 (elements
//         16(g%2) .. +15) give both sub-steps;
//   Q4_0: c = 4(g/2) + 2t + g%2 -- 8 bytes of block 2q + g/2 (bytes
//         8(g%2) .. +7) give both: low nibbles (elements 8(g%2) .. +7) at
//         t = 0, high nibbles (elements 16 + 8(g%2) .. +7) at t = 1;
// each block dequantised with its scale as RNE_f16((q - 8) d) / RNE_f16(q d).
template <int WT>
__device__ __forceinline__ int sk_piece(int g, int t) {
    if constexpr (WT == TLHIP_F16) return 4 * t + g;
    else if constexpr (WT == TLHIP_Q8_0) return 4 * (g >> 1) + 2 * (g & 1) + t;
    else return 4 * (g >> 1) + 2 * t + (g & 1);
}

template <int WT, int MT, int NT, int KP>
__global__ __launch_bounds__(64 * KP) void gemm_skinny_kernel(GemmParams p) {
    using L = SkL<WT, MT, NT, KP>;
    static_assert(L::OK, "ring");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[KP * L::ST * L::STAGE];
    const int lane = threadIdx.x & 63;
    const int kp = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);   // wave-uniform
    const int nl = lane & 15, g = lane >> 4;
    const int z = (int)blockIdx.x % p.splits, mn = (int)blockIdx.x / p.splits;   // K slice, (M tile, N tile)
    const int m0 = mn % p.mtiles * 16 * MT, n0 = mn / p.mtiles * L::ROWS;
    const int nq = p.K >> 6;
    const int za = nq * z / p.splits, nz = nq * (z + 1) / p.splits - za;   // this workgroup's K slice (steps)
    const int qa = za + nz * kp / KP, nst = za + nz * (kp + 1) / KP - qa;
    uint8_t* const ring = smem + kp * L::ST * L::STAGE;
    const uint32_t ring_lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(gl_lds_t)ring);
    const uint32_t K = (uint32_t)p.K;

    constexpr uint32_t WSTEP = WT == TLHIP_F16 ? 128u : (WT == TLHIP_Q8_0 ? 64u : 32u);   // weight bytes per row and step
    const uint32_t wrow = WT == TLHIP_F16 ? 2u * K : (WT == TLHIP_Q8_0 ? K : K / 2u);
    const __amdgpu_buffer_rsrc_t rx = sk_rsrc(p.x, (uint32_t)p.M * K * 2u);
    const __amdgpu_buffer_rsrc_t rw = sk_rsrc(p.wq, (uint32_t)p.N * wrow);
    const __amdgpu_buffer_rsrc_t rd = sk_rsrc(WT == TLHIP_F16 ? (const void*)p.wq : (const void*)p.wd,
                                              WT == TLHIP_F16 ? 0u : (uint32_t)p.N * (K / 32u) * 2u);

    // source byte offsets (step 0) of this lane's 16 bytes in each load:
    // LDS piece P = 64 u + lane of the region, rows of 8 (x, f16 weights),
    // 4 (Q8_0) or 2 (Q4_0) pieces, XOR-swizzled by row
    uint32_t xsrc[L::NX], wsrc[L::NW], dsrc = SK_OOB;
#pragma unroll
    for (int u = 0; u < L::NX; u++) {
        const int P = 64 * u + lane, r = P >> 3, c = (P & 7) ^ (r & 7);
        xsrc[u] = m0 + r < p.M ? (uint32_t)(m0 + r) * K * 2u + 16u * c : SK_OOB;
    }
#pragma unroll
    for (int u = 0; u < L::NW; u++) {
        const int P = 64 * u + lane;
        int n, c;
        if (WT == TLHIP_F16) { n = P >> 3; c = (P & 7) ^ (n & 7); }
        else if (WT == TLHIP_Q8_0) { n = P >> 2; c = (P & 3) ^ ((n >> 1) & 3); }
        else { n = P >> 1; c = (P & 1) ^ ((n >> 2) & 1); }
        wsrc[u] = n0 + n < p.N ? (uint32_t)(n0 + n) * wrow + 16u * c : SK_OOB;
    }
    if (L::NS && lane < L::ROWS && n0 + lane < p.N) dsrc = (uint32_t)(n0 + lane) * (K / 32u) * 2u;

    // operand offsets inside a stage
    int xrd[MT][2], wrd[NT][2], drd[NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int r = 16 * mt + nl;
            xrd[mt][t] = r * 128 + 16 * (sk_piece<WT>(g, t) ^ (r & 7));
        }
#pragma unroll
    for (int j = 0; j < NT; j++) {
        const int n = 16 * j + nl;
#pragma unroll
        for (int t = 0; t < 2; t++) {
            if (WT == TLHIP_F16) wrd[j][t] = L::X + n * 128 + 16 * ((4 * t + g) ^ (n & 7));
            else if (WT == TLHIP_Q8_0) wrd[j][t] = L::X + n * 64 + 16 * ((2 * (g >> 1) + (g & 1)) ^ ((n >> 1) & 3));
            else wrd[j][t] = L::X + n * 32 + 16 * ((g >> 1) ^ ((n >> 2) & 1)) + 8 * (g & 1);
        }
        drd[j] = L::X + L::W + 4 * n + 2 * (g >> 1);   // this lane's block's scale
    }

    // one stage's loads: step q into stage st
    auto issue = [&](int q, int st) {
        const uint32_t base = ring_lds + (uint32_t)(st * L::STAGE);
#pragma unroll
        for (int u = 0; u < L::NX; u++) sk_dma<16>(rx, base + 1024u * u, xsrc[u] + (uint32_t)q * 128u);
#pragma unroll
        for (int u = 0; u < L::NW; u++) sk_dma<16>(rw, base + L::X + 1024u * u, wsrc[u] + (uint32_t)q * WSTEP);
        if constexpr (L::NS > 0) sk_dma<4>(rd, base + L::X + L::W, dsrc + (uint32_t)q * 4u);
    };

    const bool rope = p.epi == EPI_QKV_ROPE;
    const bool use_b = p.epi == EPI_BIAS || p.epi == EPI_BIAS_RESID || p.epi == EPI_BIAS_GELU || (rope && p.bias);
    const bool use_r = p.epi == EPI_RESID || p.epi == EPI_BIAS_RESID;
    constexpr int NP = (NT * MT + KP - 1) / KP;   // pairs per wave
    uint32_t bv[NP], rv[NP][4];
    float rc[NP][4], rsn[NP][4];   // EPI_QKV_ROPE: the rotation of this lane's column pair at each row
#pragma unroll
    for (int i = 0; i < NP; i++) {   // epilogue operands, loaded while the K loop runs
        const int pr = kp + KP * i, j = pr % NT, mt = pr / NT;
        const int n = min(n0 + 16 * j + nl, p.N - 1);
        bv[i] = use_b && mt < MT ? (uint32_t)p.bias[n] : 0u;
        // EPI_QKV_ROPE: this column pair's place in its head (one division
        // per column, not per row)
        int re = -1;
        if (rope && mt < MT) {
            const int ne = n & ~1, D = p.head_dim;
            re = ne < p.nq ? ne % D : (ne < p.nq + p.nk ? (ne - p.nq) % D : -1);
            if (re >= p.rot) re = -1;
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = min(m0 + 16 * mt + 4 * g + r, p.M - 1);
            rv[i][r] = use_r && mt < MT ? (uint32_t)p.resid[(size_t)m * p.N + n] : 0u;
            rc[i][r] = 1.0f;
            rsn[i][r] = 0.0f;
            if (re >= 0) {
                const size_t ti = 2 * ((size_t)(p.pos0 + m) * (p.rot >> 1) + (re >> 1));
                rc[i][r] = p.rope_tab[ti];
                rsn[i][r] = p.rope_tab[ti + 1];
            }
        }
    }

    f4 acc[NT][MT];
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[j][mt] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // the operands of one stage and its MFMAs
    auto compute = [&](int st) {
        const uint8_t* base = ring + st * L::STAGE;
        h8 a[MT][2], b[NT][2];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int t = 0; t < 2; t++) a[mt][t] = *(const h8*)(base + xrd[mt][t]);
        if constexpr (WT == TLHIP_F16) {
#pragma unroll
            for (int j = 0; j < NT; j++)
#pragma unroll
                for (int t = 0; t < 2; t++) b[j][t] = *(const h8*)(base + wrd[j][t]);
        } else {
#pragma unroll
            for (int j = 0; j < NT; j++) {
                const h16 dh = *(const h16*)(base + drd[j]);
                const h2 dd = {dh, dh};
                uint32_t o[8];
                if constexpr (WT == TLHIP_Q8_0) {
                    const u4 w = *(const u4*)(base + wrd[j][0]);   // 16 elements: t = 0 bytes 0-7, t = 1 bytes 8-15
                    q8_pairs(w[0], dd, o[0], o[1]);
                    q8_pairs(w[1], dd, o[2], o[3]);
                    q8_pairs(w[2], dd, o[4], o[5]);
                    q8_pairs(w[3], dd, o[6], o[7]);
                } else {
                    const uint2 w = *(const uint2*)(base + wrd[j][0]);   // low nibbles t = 0, high nibbles t = 1
                    q4_pairs(w.x & 0x0F0F0F0Fu, dd, o[0], o[1]);
                    q4_pairs(w.y & 0x0F0F0F0Fu, dd, o[2], o[3]);
                    q4_pairs((w.x >> 4) & 0x0F0F0F0Fu, dd, o[4], o[5]);
                    q4_pairs((w.y >> 4) & 0x0F0F0F0Fu, dd, o[6], o[7]);
                }
                b[j][0] = __builtin_bit_cast(h8, u4{o[0], o[1], o[2], o[3]});
                b[j][1] = __builtin_bit_cast(h8, u4{o[4], o[5], o[6], o[7]});
            }
        }
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int j = 0; j < NT; j++)
                    acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt][t], b[j][t], acc[j][mt], 0, 0, 0);
    };

#pragma unroll
    for (int st = 0; st < L::ST; st++)
        if (st < nst) issue(qa + st, st);
    // steady state: every step refills its stage, so L::ST - 1 stages are
    // always in flight after it; then the last L::ST - 1 steps (fewer if the
    // part is short) drain the ring
    int st = 0, i = 0;
    for (; i + L::ST < nst; i++) {
        sk_wait_vm<(L::ST - 1) * L::C>();   // this step's stage has landed (loads complete in order)
        compute(st);
        // the stage's reads have returned before its refill is issued
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        issue(qa + i + L::ST, st);
        __builtin_amdgcn_sched_barrier(0);
        st = st + 1 == L::ST ? 0 : st + 1;
    }
    for (; i < nst; i++) {
        sk_wait_stages<L::C, L::ST - 1>(nst - 1 - i);
        compute(st);
        st = st + 1 == L::ST ? 0 : st + 1;
    }

    // every part's partial tiles to LDS (over the rings: every wave's loads
    // have landed); wave w then reduces (weight tile, M tile) pairs w,
    // w + KP, ... in part order and applies the epilogue
    __syncthreads();
    float (*red)[NT][MT * 4][64] = (float (*)[NT][MT * 4][64])smem;
    static_assert(sizeof(float) * KP * NT * MT * 4 * 64 <= sizeof(smem), "reduction fits the rings");
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[kp][j][mt * 4 + r][lane] = acc[j][mt][r];
    __syncthreads();
    float vs[NP][4];
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int pr = kp + KP * i, j = pr % NT, mt = pr / NT;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float v = 0.0f;
            if (mt < MT) {
                v = red[0][j][mt * 4 + r][lane];
#pragma unroll
                for (int u = 1; u < KP; u++) v += red[u][j][mt * 4 + r][lane];
            }
            vs[i][r] = v;
        }
    }
    if (p.splits > 1) {
        // This slice's tile to the partials; the last slice to arrive sums
        // them.  Partials and counter are written and read as device-scope
        // relaxed atomics, which go past this XCD's L2 to the memory every
        // XCD sees; waiting for the stores to complete before the count
        // orders them.  (Device-scope fences would instead write back and
        // invalidate the whole L2, which the other workgroups on the XCD
        // are streaming through.)
        __shared__ int sk_last;
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int pr = kp + KP * i, j = pr % NT, mt = pr / NT;
            const int ncol = n0 + 16 * j + nl;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + 16 * mt + 4 * g + r;
                if (mt < MT && m < p.M && ncol < p.N)
                    __hip_atomic_store(p.part + ((size_t)z * p.M + m) * p.N + ncol, vs[i][r], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0)
            sk_last = __hip_atomic_fetch_add(p.flags + mn, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      (uint32_t)(p.splits - 1);
        __syncthreads();
        if (!sk_last) return;
        if (threadIdx.x == 0) __hip_atomic_store(p.flags + mn, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < NP; i++) {
            const int pr = kp + KP * i, j = pr % NT, mt = pr / NT;
            const int ncol = min(n0 + 16 * j + nl, p.N - 1);
            float t[4][SK_MAX_SPLITS];   // every slice's value loaded before the in-order sum
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = min(m0 + 16 * mt + 4 * g + r, p.M - 1);
#pragma unroll
                for (int zz = 0; zz < SK_MAX_SPLITS; zz++)
                    t[r][zz] = mt < MT && zz < p.splits
                                   ? __hip_atomic_load(p.part + ((size_t)zz * p.M + m) * p.N + ncol, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT)
                                   : 0.0f;
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float v = t[r][0];
#pragma unroll
                for (int zz = 1; zz < SK_MAX_SPLITS; zz++) v += t[r][zz];
                vs[i][r] = v;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int pr = kp + KP * i, j = pr % NT, mt = pr / NT;
        if (mt >= MT) break;
        const int ncol = n0 + 16 * j + nl;
        // EPI_QKV_ROPE: destination of this column pair (per column, not per row)
        int sect = 0, hoff = 0, e = 0;
        if (rope) {
            const int D = p.head_dim;
            if (ncol < p.nq) {
                hoff = ncol / D * D;
                e = ncol - hoff;
            } else if (ncol < p.nq + p.nk) {
                sect = 1;
                hoff = (ncol - p.nq) / D * D;
                e = ncol - p.nq - hoff;
            } else {
                sect = 2;
                hoff = ncol - p.nq - p.nk;
            }
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float v = vs[i][r];
            const int m = m0 + 16 * mt + 4 * g + r;
            if (rope) {
                // the f16 projection (plus bias) of this column and of its
                // pair partner (column ^ 1, the neighbouring lane), rotated
                // and stored as the GEMV's fused epilogue does
                uint16_t x = f2h(v);
                if (p.bias) x = add_h(x, (uint16_t)bv[i]);
                const uint32_t xo = (uint32_t)__shfl_xor((int)x, 1, 64);
                if ((ncol & 1) == 0 && m < p.M && ncol + 1 < p.N) {
                    const int pos = p.pos0 + m;
                    if (sect == 2) {
                        p.vc[(size_t)pos * p.nk + hoff] = x;
                        p.vc[(size_t)pos * p.nk + hoff + 1] = (uint16_t)xo;
                        continue;
                    }
                    uint16_t* dst = sect ? p.kc + (size_t)pos * p.nk + hoff : p.q_out + (size_t)m * p.nq + hoff;
                    if (e < p.rot) {
                        const int half = p.rot >> 1, ip = e >> 1;
                        const float x0 = h2f(x), x1 = h2f((uint16_t)xo), c = rc[i][r], sn = rsn[i][r];
                        const float o0 = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, sn));
                        const float o1 = __fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, c));
                        dst[p.layout ? ip : 2 * ip] = f2h(o0);
                        dst[p.layout ? ip + half : 2 * ip + 1] = f2h(o1);
                    } else {
                        dst[e] = x;
                        dst[e + 1] = (uint16_t)xo;
                    }
                }
            } else if (p.epi == EPI_SWIGLU_PAIR) {
                const float up = __shfl_down(v, 1, 64);
                if (m < p.M && ncol + 1 < p.N && (ncol & 1) == 0)
                    p.y[(size_t)m * p.ldy + ncol / 2] = swiglu_h(f2h(v), f2h(up));
            } else if (m < p.M && ncol < p.N) {
                p.y[(size_t)m * p.ldy + ncol] = epilogue_v(p.epi, v, (uint16_t)bv[i], (uint16_t)rv[i][r]);
            }
        }
    }
}

bool gemm_skinny_ok(int M, int N, int K, int wt) {
    // byte offsets of the buffer loads are 32-bit, the padding offset
    // SK_OOB above every tensor
    const uint64_t wrow = wt == TLHIP_F16 ? 2ull * K : (wt == TLHIP_Q4_0 ? K / 2ull : (uint64_t)K);
    return M > 4 && M <= 64 && K % 64 == 0 && (wt == TLHIP_F16 || wt == TLHIP_Q8_0 || wt == TLHIP_Q4_0) &&
           (uint64_t)N * wrow < SK_OOB && 2ull * M * K < SK_OOB;
}

// The skinny GEMM's launch shape for (M, N, K, weight type): M tiles per
// workgroup (mt), 16-row weight tiles per workgroup (nt), waves (K parts)
// per workgroup (kp) and K slices.  A cost model fitted to the measured
// kernel (M = 46, cold weights): a workgroup takes its activation bytes in
// at about 50 GB/s (they are in L2: every weight tile reads them again) and
// its weight bytes at about 25 GB/s, plus 2.5 us of fixed time per round of
// workgroups (one workgroup per CU: the rings fill the LDS), plus 2.5 us
// for the exchange of a K split.  Where the weight tiles alone fill the
// device, splitting K with every row in one workgroup moves fewer bytes
// per CU (Q4_0 [2048 x 5632]: 13.8 -> 11.0 us; Q8_0: 15.7 -> 12.1 us).
// Eight waves (two per SIMD, so one's dequantisation overlaps the other's
// MFMAs and waits) wherever the LDS still holds a two-stage ring for each:
// four measured slower at every shape tried, so they are taken only when
// nothing else fits; a split leaves each wave at least two 64-k steps.
struct SkPlan {
    int mt = 1, nt = 2, kp = 4, mtiles = 1, splits = 1;
};
static int sk_stage_bytes(int wt, int mt, int nt) {
    const int wrow = wt == TLHIP_F16 ? 128 : (wt == TLHIP_Q8_0 ? 64 : 32);
    return mt * 16 * 128 + 16 * nt * wrow + (wt == TLHIP_F16 ? 0 : 256);
}
static SkPlan sk_plan(int M, int N, int K, int wt) {
    const double bpe = wt == TLHIP_F16 ? 2.0 : (wt == TLHIP_Q8_0 ? 34.0 / 32 : 18.0 / 32);
    const int mt16 = (M + 15) / 16;
    SkPlan best;
    for (int allow4 = 0; allow4 < 2; allow4++) {
        double best_us = 1e30;
        for (int nt : {2, 4})
            for (int mt = 1; mt <= mt16; mt++) {
                const int sb = sk_stage_bytes(wt, mt, nt);
                const int kp = SK_LDS / (8 * sb) >= 2 ? 8 : 4;
                if ((kp == 4 && !allow4) || SK_LDS / (kp * sb) < 2) continue;
                for (int sp = 1; sp <= SK_MAX_SPLITS; sp *= 2) {
                    const int mtiles = (mt16 + mt - 1) / mt, ntiles = (N + 16 * nt - 1) / (16 * nt);
                    if (sp > 1 && ((K / 64) / sp < 2 * kp || mtiles * ntiles > SK_MAX_TILES_SPLIT)) continue;
                    const long wgs = (long)mtiles * ntiles * sp;
                    const double rounds = (double)((wgs + 255) / 256);
                    const double bx = std::min(16 * mt, M) * 2.0 * K / sp, bw = 16 * nt * bpe * K / sp;
                    const double us = rounds * (bx / 50e3 + bw / 25e3 + 2.5) + (sp > 1 ? 2.5 : 0.0);
                    if (us < best_us - 1e-9) {
                        best_us = us;
                        best.mt = mt;
                        best.nt = nt;
                        best.kp = kp;
                        best.mtiles = mtiles;
                        best.splits = sp;
                    }
                }
            }
        if (best_us < 1e30) break;
    }
    return best;
}

template <int WT, int MT, int NT, int KP>
static void launch_skinny_one(hipStream_t s, const GemmParams& p) {
    if constexpr (SkL<WT, MT, NT, KP>::OK) {
        const dim3 grid((unsigned)(p.mtiles * ((p.N + 16 * NT - 1) / (16 * NT)) * p.splits));
        hipLaunchKernelGGL((gemm_skinny_kernel<WT, MT, NT, KP>), grid, dim3(64 * KP), 0, s, p);
    }
}
template <int WT, int NT, int KP>
static void launch_skinny_mt(hipStream_t s, const GemmParams& p, int mt) {
    switch (mt) {
        case 1: launch_skinny_one<WT, 1, NT, KP>(s, p); break;
        case 2: launch_skinny_one<WT, 2, NT, KP>(s, p); break;
        case 3: launch_skinny_one<WT, 3, NT, KP>(s, p); break;
        default: launch_skinny_one<WT, 4, NT, KP>(s, p); break;
    }
}
template <int WT>
static void launch_skinny(hipStream_t s, const GemmParams& p, const SkPlan& pl) {
    if (pl.nt == 4) {
        if (pl.kp == 8) launch_skinny_mt<WT, 4, 8>(s, p, pl.mt);
        else launch_skinny_mt<WT, 4, 4>(s, p, pl.mt);
    } else {
        if (pl.kp == 8) launch_skinny_mt<WT, 2, 8>(s, p, pl.mt);
        else launch_skinny_mt<WT, 2, 4>(s, p, pl.mt);
    }
}

template <int WT, int BM, int BN, int NS>
__global__ __launch_bounds__(512) void gemm_lds_kernel(GemmParams p, float* __restrict__ part, int mT, int nT, int splits) {
    using L = Gl<WT, BM, BN, NS>;
    constexpr int TM = BM / 64, TN = BN / 128;   // 32x32 tiles per wave
    constexpr int WTN = BN / 4;                   // wave tile width
    static_assert(TN >= 1 && BN % 128 == 0, "BN");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * L::STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3, hh = lane >> 5, l32 = lane & 31;
    const int T = mT * nT;
    const int q = gl_tile((int)blockIdx.x, T * splits);
    const int z = q / T, qt = q % T;
    const int m0 = (qt % mT) * BM, n0 = (qt / mT) * BN;
    const int nkt = p.K / 64;
    const int kt0 = (int)((int64_t)nkt * z / splits), kt1 = (int)((int64_t)nkt * (z + 1) / splits);
    const int nk = kt1 - kt0;
    const int nbr = p.K >> 5;

    using DA = GlDma<L::A_BYTES>;
    using DB = GlDma<L::B_BYTES>;
    const uint8_t* a_src[DA::N];
#pragma unroll
    for (int u = 0; u < DA::N; u++) {
        const int P = (u * 8 + wave) * 64 * DA::SZ + lane * DA::SZ;
        const int r = P >> 7, c = ((P >> 4) & 7) ^ ((r >> 1) & 7);
        const int m = min(m0 + r, p.M - 1);
        a_src[u] = (const uint8_t*)(p.x + (size_t)m * p.K + (size_t)kt0 * 64 + 8 * c) + (P & 15);
    }
    const uint8_t* b_src[DB::N];
#pragma unroll
    for (int u = 0; u < DB::N; u++) {
        constexpr int RB = GlRow<WT>::B;
        const int P = (u * 8 + wave) * 64 * DB::SZ + lane * DB::SZ;
        const int r = P / RB, cp = (P % RB) >> 4, byte = P & 15;
        const int n = min(n0 + r, p.N - 1);
        if (WT == TLHIP_F16) {
            b_src[u] = p.wq + ((size_t)n * p.K + (size_t)kt0 * 64 + 8 * (cp ^ ((r >> 1) & 7))) * 2 + byte;
        } else if (WT == TLHIP_Q8_0) {
            b_src[u] = p.wq + (size_t)n * p.K + (size_t)kt0 * 64 + 16 * (cp ^ ((r >> 2) & 3)) + byte;
        } else {
            b_src[u] = p.wq + (size_t)n * (p.K / 2) + (size_t)kt0 * 32 + 16 * (cp ^ ((r >> 3) & 1)) + byte;
        }
    }
    // scales: wave w, lanes < BN/8 -> row w*BN/8 + lane, both blocks of the step (4 bytes)
    constexpr int SR = BN / 8;
    const bool s_lane = lane < SR;
    const uint8_t* s_src = nullptr;
    if (L::S_BYTES) {
        const int n = min(n0 + wave * SR + (s_lane ? lane : 0), p.N - 1);
        s_src = (const uint8_t*)(p.wd + (size_t)n * nbr + 2 * (size_t)kt0);
    }
    constexpr int B_STEP = GlRow<WT>::B == 128 ? 128 : GlRow<WT>::B;

    auto issue = [&](int step, int s) {   // step = kt - kt0
        uint8_t* st = smem + s * L::STAGE;
#pragma unroll
        for (int u = 0; u < DA::N; u++) gl_dma<DA::SZ>(a_src[u] + (size_t)step * 128, st + (u * 8 + wave) * 64 * DA::SZ);
#pragma unroll
        for (int u = 0; u < DB::N; u++)
            gl_dma<DB::SZ>(b_src[u] + (size_t)step * B_STEP, st + L::A_BYTES + (u * 8 + wave) * 64 * DB::SZ);
        if (L::S_BYTES && s_lane) gl_dma<4>(s_src + (size_t)step * 4, st + L::A_BYTES + L::B_BYTES + wave * SR * 4);
    };

    f16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = f16v{0};

#pragma unroll
    for (int s = 0; s < NS - 1; s++)
        if (s < nk) issue(s, s);

    // per-lane LDS offsets inside a stage (constant over the K loop)
    int a_off[TM][4], b_off[TN][4];
#pragma unroll
    for (int ii = 0; ii < TM; ii++) {
        const int m = wm * (BM / 2) + 32 * ii + l32;
#pragma unroll
        for (int t = 0; t < 4; t++) a_off[ii][t] = 128 * m + 16 * ((4 * hh + t) ^ ((m >> 1) & 7));
    }
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = wn * WTN + 32 * j + l32;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            if (WT == TLHIP_F16) b_off[j][t] = L::A_BYTES + 128 * n + 16 * ((4 * hh + t) ^ ((n >> 1) & 7));
            else if (WT == TLHIP_Q8_0) b_off[j][t] = t < 2 ? L::A_BYTES + 64 * n + 16 * ((2 * hh + t) ^ ((n >> 2) & 3))
                                                           : L::A_BYTES + L::B_BYTES + 4 * n + 2 * hh;
            else b_off[j][t] = t == 0 ? L::A_BYTES + 32 * n + 16 * (hh ^ ((n >> 3) & 1))
                                      : L::A_BYTES + L::B_BYTES + 4 * n + 2 * hh;
        }
    }

    for (int i = 0; i < nk; i++) {
        gl_wait_stage<L::VMC, NS - 2>(min(nk - 1 - i, NS - 2));
        lds_barrier();   // stage i landed for every wave; stage i-1 fully read
        if (i + NS - 1 < nk) issue(i + NS - 1, (i + NS - 1) % NS);

        const uint8_t* st = smem + (i % NS) * L::STAGE;
        // all LDS reads of the step first, then dequantise, then the MFMAs
        h8 aop[TM][4];
#pragma unroll
        for (int ii = 0; ii < TM; ii++)
#pragma unroll
            for (int t = 0; t < 4; t++) aop[ii][t] = *(const h8*)(st + a_off[ii][t]);
        h8 bop[TN][4];
        if (WT == TLHIP_F16) {
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int t = 0; t < 4; t++) bop[j][t] = *(const h8*)(st + b_off[j][t]);
        } else if (WT == TLHIP_Q8_0) {
            u4 raw[TN][2];
            h16 dh[TN];
#pragma unroll
            for (int j = 0; j < TN; j++) {
                raw[j][0] = *(const u4*)(st + b_off[j][0]);
                raw[j][1] = *(const u4*)(st + b_off[j][1]);
                dh[j] = *(const h16*)(st + b_off[j][2]);
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const h2 dd = {dh[j], dh[j]};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    uint32_t o0, o1, o2, o3;
                    q8_pairs(raw[j][t >> 1][2 * (t & 1)], dd, o0, o1);
                    q8_pairs(raw[j][t >> 1][2 * (t & 1) + 1], dd, o2, o3);
                    bop[j][t] = __builtin_bit_cast(h8, u4{o0, o1, o2, o3});
                }
            }
        } else {
            u4 raw[TN];
            h16 dh[TN];
#pragma unroll
            for (int j = 0; j < TN; j++) {
                raw[j] = *(const u4*)(st + b_off[j][0]);
                dh[j] = *(const h16*)(st + b_off[j][1]);
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const h2 dd = {dh[j], dh[j]};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    // t = 0/1: low nibbles of bytes 0-7 / 8-15; t = 2/3: high nibbles
                    const uint32_t w0 = raw[j][2 * (t & 1)], w1 = raw[j][2 * (t & 1) + 1];
                    const uint32_t n0w = t < 2 ? (w0 & 0x0F0F0F0Fu) : ((w0 >> 4) & 0x0F0F0F0Fu);
                    const uint32_t n1w = t < 2 ? (w1 & 0x0F0F0F0Fu) : ((w1 >> 4) & 0x0F0F0F0Fu);
                    uint32_t o0, o1, o2, o3;
                    q4_pairs(n0w, dd, o0, o1);
                    q4_pairs(n1w, dd, o2, o3);
                    bop[j][t] = __builtin_bit_cast(h8, u4{o0, o1, o2, o3});
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int ii = 0; ii < TM; ii++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[ii][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aop[ii][t], bop[j][t], acc[ii][j], 0, 0, 0);
    }

    // C layout: col = lane%32 (weight row n), row = 8*(r/4) + 4*(lane/32) + r%4 (activation row m)
#pragma unroll
    for (int ii = 0; ii < TM; ii++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + wn * WTN + 32 * j + l32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * (BM / 2) + 32 * ii + 8 * (r >> 2) + 4 * hh + (r & 3);
                const float v = acc[ii][j][r];
                if (part) {
                    if (m < p.M && n < p.N) part[((size_t)z * p.M + m) * p.N + n] = v;
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

// gemm_reduce_kernel for 4 consecutive columns per thread (16-byte partial
// loads, one 8-byte store; the SwiGLU pair epilogue: two outputs, one
// 4-byte store): the same sums in slice order and the same epilogue per
// element.  N and the output row stride multiples of 4 (SwiGLU: of 2 for
// the output), the partials 16-byte and the other pointers 8-byte aligned.
__global__ void gemm_reduce4_kernel(GemmParams p, const float* __restrict__ part, int splits) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    const int64_t total = (int64_t)p.M * p.N;
    if (i >= total) return;
    const int m = (int)(i / p.N), n = (int)(i % p.N);
    float4 v = *(const float4*)(part + i);
    for (int z = 1; z < splits; z++) {
        const float4 t = *(const float4*)(part + (size_t)z * total + i);
        v.x += t.x;
        v.y += t.y;
        v.z += t.z;
        v.w += t.w;
    }
    if (p.epi == EPI_SWIGLU_PAIR) {
        const uint32_t o0 = swiglu_h(f2h(v.x), f2h(v.y)), o1 = swiglu_h(f2h(v.z), f2h(v.w));
        *(uint32_t*)(p.y + (size_t)m * p.ldy + n / 2) = o0 | (o1 << 16);
        return;
    }
    const size_t ri = (size_t)m * p.N + n;
    const uint32_t o0 = epilogue_h(p.epi, v.x, p.bias, p.resid, ri, n);
    const uint32_t o1 = epilogue_h(p.epi, v.y, p.bias, p.resid, ri + 1, n + 1);
    const uint32_t o2 = epilogue_h(p.epi, v.z, p.bias, p.resid, ri + 2, n + 2);
    const uint32_t o3 = epilogue_h(p.epi, v.w, p.bias, p.resid, ri + 3, n + 3);
    *(uint2*)(p.y + (size_t)m * p.ldy + n) = uint2{o0 | (o1 << 16), o2 | (o3 << 16)};
}

constexpr int GL_BM = 128, GL_BN = 128;

template <int WT>
static void launch_gemm2(hipStream_t s, const GemmParams& p, int splits, float* part) {
    if (p.M > 64) {
        // four stages (one workgroup per CU) while the grid fits the 256 CUs;
        // beyond that three stages, so that two workgroups share a CU
        const int mT = (p.M + GL_BM - 1) / GL_BM, nT = (p.N + GL_BN - 1) / GL_BN;
        const unsigned grid = (unsigned)(mT * nT * splits);
        if (grid > 256)
            hipLaunchKernelGGL((gemm_lds_kernel<WT, GL_BM, GL_BN, 3>), dim3(grid), dim3(512), 0, s, p, part, mT, nT, splits);
        else
            hipLaunchKernelGGL((gemm_lds_kernel<WT, GL_BM, GL_BN, 4>), dim3(grid), dim3(512), 0, s, p, part, mT, nT, splits);
    } else {
        dim3 grid((unsigned)((p.N + 63) / 64), (unsigned)((p.M + 63) / 64), (unsigned)splits);
        hipLaunchKernelGGL((gemm2_kernel<WT, 64, 64, 2, 2>), grid, dim3(256), 0, s, p, part);
    }
}

// split-K slices.  M <= 64 (register-staged 64 x 64 tiles): enough
// workgroups to cover the 256 CUs about once, at least 4 K steps per slice.
// M > 64 (multi-stage 128 x 128 tiles, one workgroup per CU): up to 4
// slices while the grid stays within 320 workgroups, at least 8 K steps
// per slice.
// The bound GEMM_SPLIT_PARTIALS_MAX states for each branch below (the fixed
// workspace of the no-allocation entry point is sized by it).
static_assert((size_t)GEMM_SPLIT_TILE_CAP * GL_BM * GL_BN * sizeof(float) <= GEMM_SPLIT_PARTIALS_MAX, "M > 64 split");
static_assert((size_t)SK_MAX_SPLITS * 64 * (SK_MAX_TILES_SPLIT * 16 * 4) * sizeof(float) <= GEMM_SPLIT_PARTIALS_MAX,
              "skinny split (64 rows, N <= SK_MAX_TILES_SPLIT tiles of 16 x 4 weight rows)");
static_assert((size_t)512 * 64 * 64 * sizeof(float) <= GEMM_SPLIT_PARTIALS_MAX, "M <= 64 split");
int gemm_splits(int M, int N, int K, int wt) {
    if (wt < 0) {   // any weight type: the largest count any of them takes
        int sp = 1;
        for (int t : {(int)TLHIP_F16, (int)TLHIP_Q8_0, (int)TLHIP_Q4_0, (int)TLHIP_Q6_K}) sp = std::max(sp, gemm_splits(M, N, K, t));
        return sp;
    }
    if (gemm_skinny_ok(M, N, K, wt)) return sk_plan(M, N, K, wt).splits;
    if (K % G2_BK) return 1;
    int sp = 1;
    if (M > 64) {
        const int tiles = ((N + GL_BN - 1) / GL_BN) * ((M + GL_BM - 1) / GL_BM);
        while (sp < 4 && tiles * sp * 2 <= GEMM_SPLIT_TILE_CAP && (K / G2_BK) / (sp * 2) >= 8) sp *= 2;
        return sp;
    }
    const int tiles = ((N + 63) / 64) * ((M + 63) / 64);
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
    if (a.pro != PRO_NONE)
        return fail(TLHIP_ERR_INVALID_OPERATION, "gemm: the fused normalisation prologue is GEMV-only");
    if (epi == EPI_QKV_ROPE) {
        if (!gemm_skinny_ok(p.M, p.N, p.K, wt) || a.d_pos || !a.rope_tab || !a.q_out || !a.kc || !a.vc ||
            a.head_dim <= 0 || a.head_dim % 2 || a.rot % 2 || a.rot > a.head_dim || a.nq % a.head_dim ||
            a.nk % a.head_dim || a.nq + 2 * a.nk != p.N)
            return fail(TLHIP_ERR_INVALID_OPERATION, "gemm: the RoPE epilogue needs the skinny GEMM and a q/k/v layout");
        p.nq = a.nq;
        p.nk = a.nk;
        p.head_dim = a.head_dim;
        p.rot = a.rot;
        p.layout = a.layout;
        p.pos0 = a.pos0;
        p.rope_tab = a.rope_tab;
        p.q_out = a.q_out;
        p.kc = a.kc;
        p.vc = a.vc;
    }
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
    if (gemm_skinny_ok(p.M, p.N, p.K, wt)) {
        // K split over workgroups only with a workspace for the partials and
        // the per-tile counters
        const SkPlan pl = sk_plan(p.M, p.N, p.K, wt);
        p.mtiles = pl.mtiles;
        if (pl.splits > 1 && a.ws && a.tile_flags && (size_t)pl.splits * p.M * p.N * sizeof(float) <= a.ws_bytes) {
            p.splits = pl.splits;
            p.part = a.ws;
            p.flags = a.tile_flags;
        }
        if (wt == TLHIP_Q4_0) launch_skinny<TLHIP_Q4_0>(s, p, pl);
        else if (wt == TLHIP_Q8_0) launch_skinny<TLHIP_Q8_0>(s, p, pl);
        else launch_skinny<TLHIP_F16>(s, p, pl);
        return TLHIP_OK;
    }
    if (p.K % G2_BK == 0) {
        int splits = a.ws ? gemm_splits(p.M, p.N, p.K, wt) : 1;
        if ((size_t)splits * p.M * p.N * sizeof(float) > a.ws_bytes) splits = 1;
        float* part = splits > 1 ? a.ws : nullptr;
        if (wt == TLHIP_Q4_0) launch_gemm2<TLHIP_Q4_0>(s, p, splits, part);
        else if (wt == TLHIP_Q8_0) launch_gemm2<TLHIP_Q8_0>(s, p, splits, part);
        else launch_gemm2<TLHIP_F16>(s, p, splits, part);
        if (splits > 1) {
            const int64_t total = (int64_t)p.M * p.N;
            const bool vec = p.N % 4 == 0 && p.ldy % (p.epi == EPI_SWIGLU_PAIR ? 2 : 4) == 0 &&
                             ((uintptr_t)p.y | (uintptr_t)p.bias | (uintptr_t)p.resid) % 8 == 0 && (uintptr_t)part % 16 == 0;
            if (vec)
                hipLaunchKernelGGL(gemm_reduce4_kernel, dim3((unsigned)((total / 4 + 255) / 256)), dim3(256), 0, s, p,
                                   (const float*)part, splits);
            else
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

// ---------------------------------------------------------------------------
// linear() on f32 tensors (the TensorF32 arm, builtin_math.rs:121-175:
// x.matmul_transposed_b(w), then result.add(bias)).  Every output is the
// reference kernel's sum (matmul_transposed_b_tiled_32x32_f32,
// unified.metal:4409-4461): k in order from +0, one fused multiply-add per
// term (the contraction Metal's default fast math makes of `sum += a * b`),
// the row padded with zero terms to a multiple of 32 as its tiles are; the
// bias is a separate f32 add.  A workgroup of 256 threads computes a 64 x 64
// tile, 4 x 4 outputs per thread, from 64 x 32 slices of x and w staged
// k-major in LDS.  Not on the decode path (the LLM programs are f16): plain
// VALU arithmetic, no MFMA (v_mfma_f32_*_xf32 would change the sums' order).
// ---------------------------------------------------------------------------
constexpr int LF_BM = 64, LF_BN = 64, LF_BK = 32;

__global__ __launch_bounds__(256) void linear_f32_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                         const float* __restrict__ bias, float* __restrict__ y, int M,
                                                         int N, int K) {
    __shared__ float as[LF_BK][LF_BM + 4];
    __shared__ float bs[LF_BK][LF_BN + 4];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int m0 = blockIdx.y * LF_BM, n0 = blockIdx.x * LF_BN;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
    const int kp = (K + LF_BK - 1) / LF_BK * LF_BK;   // zero terms up to a multiple of 32
    for (int k0 = 0; k0 < kp; k0 += LF_BK) {
#pragma unroll
        for (int i = 0; i < 8; i++) {   // 64 rows x 32 k of each operand, 8 per thread
            const int idx = tid + 256 * i, r = idx >> 5, c = idx & 31;
            const int k = k0 + c;
            as[c][r] = (m0 + r < M && k < K) ? x[(size_t)(m0 + r) * K + k] : 0.0f;
            bs[c][r] = (n0 + r < N && k < K) ? w[(size_t)(n0 + r) * K + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < LF_BK; kk++) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] = as[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; j++) b[j] = bs[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = m0 + ty * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = n0 + tx * 4 + j;
            if (n < N) y[(size_t)m * N + n] = bias ? acc[i][j] + bias[n] : acc[i][j];
        }
    }
}

tlhip_status launch_linear_f32(hipStream_t s, const float* x, const float* w, const float* bias, float* y, int M, int N,
                               int K) {
    if (M <= 0 || N <= 0) return TLHIP_OK;
    const dim3 grid((unsigned)((N + LF_BN - 1) / LF_BN), (unsigned)((M + LF_BM - 1) / LF_BM));
    if (grid.y > 65535) return fail(TLHIP_ERR_INVALID_DIMENSION, "linear f32: %d rows", M);
    hipLaunchKernelGGL(linear_f32_kernel, grid, dim3(256), 0, s, x, w, bias, y, M, N, K);
    return TLHIP_OK;
}

}  // namespace tlhip
