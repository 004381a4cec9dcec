// kernels_attn.hip -- attention over an f16 KV cache, gfx950.
//
// Restates the TL attention sequence (chat_demo_optimized.tl:52-97;
// debug/chat_demo_with_kvcache.tl:250-277) without materialising the
// GQA-expanded K/V or the [S, H, J] score tensor:
//   s_j  = f16(sum_d q_d k_jd)                 einsum_ihd_jhd_ihj_f16 (fp32 acc)
//   s_j  = f16(s_j * f16(scale))               scores * 0.125
//   mask: j > query position -> -10000         apply_attention_mask(causal_mask)
//   P    = softmax(s) as softmax_f16 (exp in f32, exp stored f16, f32 sum,
//          P_j = f16(f16(e_j) / sum))
//   o_d  = f16(sum_j P_j v_jd)                 einsum_ihj_jhd_ihd_f16, fp32 acc
// Query head h reads KV head h / (H / Hkv) (broadcast_to [J,Hkv,1,D] ->
// [J,Hkv,H/Hkv,D]).  Masked keys are skipped: exp(-10000 - max) is exactly
// 0 in f32 for any max a real score can take, so they add nothing to the
// sum or the output; the degenerate all-non-finite row falls back to the
// reference's uniform 1/J over every key.
#include "device_common.hpp"
#include "internal.hpp"

namespace tlhip {

constexpr int ATT_MAX_J = 8192;   // keys held in LDS by the single-pass kernel

__device__ __forceinline__ float bsum(float v, float* red) {
    v = wave_sum<64>(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ __forceinline__ float bmax(float v, float* red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// One workgroup (256 threads) per (query row s, head h).
// Every field of the argument block in SGPRs at once (one wait for the
// kernel-argument loads instead of one per first use; see kernarg_fence in
// kernels_gemv.hip).
__device__ __forceinline__ void attn_kernarg_fence(const AttnArgs& a, int J_fixed) {
    asm volatile("" ::"s"(a.q), "s"(a.k), "s"(a.v), "s"(a.out), "s"(a.S), "s"(a.H), "s"(a.Hkv), "s"(a.D),
                 "s"(a.q_pos0), "s"(a.d_pos), "s"(a.causal), "s"(a.scale_h), "s"(a.q_stride), "s"(a.out_stride),
                 "s"(a.kv_rows), "s"(J_fixed));
    __builtin_amdgcn_sched_barrier(0);   // nothing that uses them moves above
}

__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a, int J_fixed) {
    __shared__ float sc[ATT_MAX_J];
    __shared__ float qf[256];
    __shared__ float red[4];
    __shared__ float part[4][256];
    const int s = blockIdx.x, h = blockIdx.y;
    const int D = a.D, Hkv = a.Hkv;
    const int kvh = h / (a.H / Hkv);
    const int qpos = (a.d_pos ? *a.d_pos : a.q_pos0) + s;
    const int J = min(a.d_pos ? qpos + 1 : J_fixed, ATT_MAX_J);   // keys in the score row
    const int Jv = a.causal ? min(J, qpos + 1) : J;           // keys not masked
    const int qs = a.q_stride ? a.q_stride : a.H * D;
    const int os = a.out_stride ? a.out_stride : a.H * D;
    const uint16_t* q = a.q + (size_t)s * qs + (size_t)h * D;
    for (int d = threadIdx.x; d < D; d += 256) qf[d] = h2f(q[d]);
    __syncthreads();

    // scores, rounded and scaled as the reference stores them
    const size_t kstride = (size_t)Hkv * D;
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < Jv; j += 256) {
        const uint16_t* kr = a.k + (size_t)j * kstride + (size_t)kvh * D;
        float acc = 0.0f;
        for (int d = 0; d < D; d++) acc += qf[d] * h2f(kr[d]);
        const float v = h2f(f2h(h2f(f2h(acc)) * a.scale_h));
        sc[j] = v;
        if (isfinite(v)) mx = fmaxf(mx, v);
    }
    mx = bmax(mx, red);
    if (!isfinite(mx)) mx = 0.0f;
    float sum = 0.0f;
    for (int j = threadIdx.x; j < Jv; j += 256) {
        const float v = sc[j];
        const float e = isfinite(v) ? expf(v - mx) : 0.0f;
        sc[j] = h2f(f2h(e));
        sum += e;
    }
    sum = bsum(sum, red);
    const bool degenerate = !(sum > 0.0f && isfinite(sum));
    const int Jp = degenerate ? J : Jv;
    const float uni = h2f(f2h(1.0f / (float)J));
    for (int j = threadIdx.x; j < Jp; j += 256) sc[j] = degenerate ? uni : h2f(f2h(sc[j] / sum));
    __syncthreads();

    // context: thread (g, d) sums keys j = g, g+G, ... ; partials combined in order
    const int G = min(4, 256 / D);
    const int g = threadIdx.x / D, d = threadIdx.x % D;
    float acc = 0.0f;
    if (g < G)
        for (int j = g; j < Jp; j += G) acc += sc[j] * h2f(a.v[(size_t)j * kstride + (size_t)kvh * D + d]);
    if (g < G) part[g][d] = acc;
    __syncthreads();
    if (threadIdx.x < D) {
        float t = part[0][threadIdx.x];
        for (int gg = 1; gg < G; gg++) t += part[gg][threadIdx.x];
        a.out[(size_t)s * os + (size_t)h * D + threadIdx.x] = f2h(t);
    }
}

// Head-dim-64 variant with the same arithmetic and storage points, laid out
// for the memory system: a key is read by 8 lanes with one 16-byte load each
// (a head's 128-byte K/V row in one coalesced access), 32 keys per pass, and
// the loads of UNR passes are issued before their dot products so several
// L2/HBM round trips overlap.  Scores: the 8 lanes' partial dot products are
// combined with an xor tree.  Context: thread (g, c) accumulates dims
// 8c..8c+7 over keys g, g+32, ...; the 32 partial rows are summed in g order.
constexpr int A64_UNR = 8;

template <int NT>
__global__ __launch_bounds__(NT) void attention64_kernel(AttnArgs a, int J_fixed) {
    constexpr int NWV = NT / 64, NG = NT / 8;
    __shared__ float sc[ATT_MAX_J];
    __shared__ float red[2][NWV];
    __shared__ float part[NWV][64];
    attn_kernarg_fence(a, J_fixed);
    const int s = blockIdx.x, h = blockIdx.y;
    const int Hkv = a.Hkv;
    const int kvh = h / (a.H / Hkv);
    const int qs = a.q_stride ? a.q_stride : a.H * 64;
    const int os = a.out_stride ? a.out_stride : a.H * 64;
    const int tid = threadIdx.x, c = tid & 7, g = tid >> 3;
    const size_t kstride = (size_t)Hkv * 64;
    const uint16_t* kbase = a.k + (size_t)kvh * 64 + 8 * c;
    const uint16_t* vbase = a.v + (size_t)kvh * 64 + 8 * c;
    // Loads that do not depend on the decode position go out first: q, and
    // the first pass of K and V rows.  Row indices are clamped to the rows
    // allocated (kv_lim), so every address is in bounds; the key count never
    // exceeds kv_lim, so a clamped row is only ever loaded for a key that is
    // not used.  The loads are unconditional: a load under a per-row branch
    // makes the compiler wait for it at the branch join, which serialised
    // the pass into several memory round trips.
    const u4 qv = *(const u4*)(a.q + (size_t)s * qs + (size_t)h * 64 + 8 * c);
    const int kv_lim = a.kv_rows > 0 ? (a.d_pos ? a.kv_rows : min(a.kv_rows, J_fixed)) : min(J_fixed, ATT_MAX_J);
    u4 k0[A64_UNR], vv[A64_UNR];
    if (kv_lim > 0) {   // (uniform; 0 only when neither a key count nor the rows allocated is known)
#pragma unroll
        for (int u = 0; u < A64_UNR; u++) k0[u] = *(const u4*)(kbase + (size_t)min(g + NG * u, kv_lim - 1) * kstride);
#pragma unroll
        for (int u = 0; u < A64_UNR; u++) vv[u] = *(const u4*)(vbase + (size_t)min(g + NG * u, kv_lim - 1) * kstride);
    } else {
#pragma unroll
        for (int u = 0; u < A64_UNR; u++) k0[u] = vv[u] = u4{0u, 0u, 0u, 0u};
    }
    const int qpos = (a.d_pos ? *a.d_pos : a.q_pos0) + s;
    const int J = min(a.d_pos ? qpos + 1 : J_fixed, ATT_MAX_J);
    const int Jv = a.causal ? min(J, qpos + 1) : J;

    float qf[8];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const h2 p2 = as_h2(qv[t]);
        qf[2 * t] = (float)p2[0];
        qf[2 * t + 1] = (float)p2[1];
    }

    // One pass covers NG * A64_UNR keys; the first pass uses the rows loaded
    // above.  When the unmasked row fits in that pass, the V rows loaded
    // with it are used directly (one round trip to memory in all).
    const bool one_pass = Jv <= NG * A64_UNR;
    float mx = -INFINITY;
    for (int j0 = g; j0 < Jv; j0 += NG * A64_UNR) {
        u4 kv[A64_UNR];
        if (j0 == g) {
#pragma unroll
            for (int u = 0; u < A64_UNR; u++) kv[u] = k0[u];
        } else {
#pragma unroll
            for (int u = 0; u < A64_UNR; u++) {
                const int j = j0 + NG * u;
                kv[u] = j < Jv ? *(const u4*)(kbase + (size_t)j * kstride) : u4{0u, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int u = 0; u < A64_UNR; u++) {
            float acc = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const h2 k2 = as_h2(kv[u][t]);
                acc += qf[2 * t] * (float)k2[0];
                acc += qf[2 * t + 1] * (float)k2[1];
            }
            acc = group8_sum(acc);
            const int j = j0 + NG * u;
            if (j < Jv) {
                const float v = h2f(f2h(h2f(f2h(acc)) * a.scale_h));
                if (c == 0) sc[j] = v;
                if (isfinite(v)) mx = fmaxf(mx, v);
            }
        }
    }
    mx = block_max1<NWV>(mx, red[0]);   // (its barrier also publishes sc[])
    if (!isfinite(mx)) mx = 0.0f;
    float sum = 0.0f;
    for (int j = tid; j < Jv; j += NT) {
        const float v = sc[j];
        const float e = isfinite(v) ? expf(v - mx) : 0.0f;
        sc[j] = h2f(f2h(e));
        sum += e;
    }
    sum = block_sum1<NWV>(sum, red[1]);
    const bool degenerate = !(sum > 0.0f && isfinite(sum));
    const int Jp = degenerate ? J : Jv;
    const float uni = h2f(f2h(1.0f / (float)J));
    for (int j = tid; j < Jp; j += NT) sc[j] = degenerate ? uni : h2f(f2h(sc[j] / sum));
    __syncthreads();

    float o[8];
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = 0.0f;
    if (one_pass && !degenerate) {
#pragma unroll
        for (int u = 0; u < A64_UNR; u++) {
            const int j = g + NG * u;
            if (j < Jp) {
                const float pj = sc[j];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const h2 v2 = as_h2(vv[u][t]);
                    o[2 * t] += pj * (float)v2[0];
                    o[2 * t + 1] += pj * (float)v2[1];
                }
            }
        }
    } else {
        for (int j0 = g; j0 < Jp; j0 += NG * A64_UNR) {
#pragma unroll
            for (int u = 0; u < A64_UNR; u++) {
                const int j = j0 + NG * u;
                vv[u] = j < Jp ? *(const u4*)(vbase + (size_t)j * kstride) : u4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < A64_UNR; u++) {
                const int j = j0 + NG * u;
                if (j < Jp) {
                    const float pj = sc[j];
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const h2 v2 = as_h2(vv[u][t]);
                        o[2 * t] += pj * (float)v2[0];
                        o[2 * t + 1] += pj * (float)v2[1];
                    }
                }
            }
        }
    }
    // the 8 key groups of each wave (lanes with the same c), then the 4 waves
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = stride8_sum(o[e]);
    if ((tid & 63) < 8)
#pragma unroll
        for (int e = 0; e < 8; e++) part[tid >> 6][8 * c + e] = o[e];
    lds_barrier();
    if (tid < 64) {
        float t = part[0][tid];
#pragma unroll
        for (int wv = 1; wv < NWV; wv++) t += part[wv][tid];
        a.out[(size_t)s * os + (size_t)h * 64 + tid] = f2h(t);
    }
}

// The same kernel for other even head dims D = 8 * EPL (Phi-2: 80): lane c
// of a key's 8 lanes holds dims EPL*c .. EPL*c + EPL - 1, read as EPL/2
// 4-byte words; ADK_THREADS threads (8 lanes per key) cover 64 * ADK_UNR
// keys per pass; the first 256 keys' K and V rows are loaded before the
// decode position is read (as attention64_kernel), the rest of the first
// pass right after, so up to 512 keys cost about one round trip to memory; the partial context rows are summed over the key
// groups of a wave, then over the waves, in a fixed order.
constexpr int ADK_UNR = 8, ADK_THREADS = 512;   // 64 key groups x 8 = 512 keys per pass

// NW consecutive 4-byte words of one key row: 16-byte loads for each full
// group of four (rows are only 4-byte aligned for D = 80; the loads do not
// need more), single words for the rest -- 2 requests per lane for D = 80
// instead of 5.
template <int NW>
__device__ __forceinline__ void load_row_words(const uint32_t* __restrict__ p, uint32_t (&w)[NW]) {
#pragma unroll
    for (int t = 0; t + 4 <= NW; t += 4) {
        u4 v;
        __builtin_memcpy(&v, p + t, 16);
        w[t] = v[0]; w[t + 1] = v[1]; w[t + 2] = v[2]; w[t + 3] = v[3];
    }
#pragma unroll
    for (int t = NW / 4 * 4; t < NW; t++) w[t] = p[t];
}
template <int D>
__global__ __launch_bounds__(ADK_THREADS) void attention_dk_kernel(AttnArgs a, int J_fixed) {
    constexpr int EPL = D / 8, NW = EPL / 2, U = ADK_UNR, NT = ADK_THREADS, NWV = NT / 64, NG = NT / 8;
    __shared__ float sc[ATT_MAX_J];
    __shared__ float red[2][NWV];
    __shared__ float part[NWV][D];
    attn_kernarg_fence(a, J_fixed);
    const int s = blockIdx.x, h = blockIdx.y;
    const int Hkv = a.Hkv;
    const int kvh = h / (a.H / Hkv);
    const int qs = a.q_stride ? a.q_stride : a.H * D;
    const int os = a.out_stride ? a.out_stride : a.H * D;
    const int tid = threadIdx.x, c = tid & 7, g = tid >> 3;
    const size_t kstride = (size_t)Hkv * D;
    const uint32_t* kbase = (const uint32_t*)(a.k + (size_t)kvh * D + EPL * c);
    const uint32_t* vbase = (const uint32_t*)(a.v + (size_t)kvh * D + EPL * c);
    const size_t wstride = kstride / 2;   // row stride in 4-byte words
    // Loads that do not depend on the decode position go out first: q, and
    // the first pass of K and V rows (bounded by the rows allocated).
    // (the first half of the pass before the decode position is known, the
    // rest once it is, for the keys that exist)
    const int kv_lim = a.kv_rows > 0 ? (a.d_pos ? a.kv_rows : min(a.kv_rows, J_fixed)) : min(J_fixed, ATT_MAX_J);
    // (clamped, unconditional loads, as in attention64_kernel)
    uint32_t k0[U][NW], v0[U][NW];
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
        for (int t = 0; t < NW; t++) k0[u][t] = v0[u][t] = 0u;
    if (kv_lim > 0) {
#pragma unroll
        for (int u = 0; u < U / 2; u++) load_row_words<NW>(kbase + (size_t)min(g + NG * u, kv_lim - 1) * wstride, k0[u]);
#pragma unroll
        for (int u = 0; u < U / 2; u++) load_row_words<NW>(vbase + (size_t)min(g + NG * u, kv_lim - 1) * wstride, v0[u]);
    }
    float qf[EPL];
    {
        const uint32_t* qw = (const uint32_t*)(a.q + (size_t)s * qs + (size_t)h * D + EPL * c);
#pragma unroll
        for (int t = 0; t < NW; t++) {
            const h2 p2 = as_h2(qw[t]);
            qf[2 * t] = (float)p2[0];
            qf[2 * t + 1] = (float)p2[1];
        }
    }
    const int qpos = (a.d_pos ? *a.d_pos : a.q_pos0) + s;
    const int J = min(a.d_pos ? qpos + 1 : J_fixed, ATT_MAX_J);
    const int Jv = a.causal ? min(J, qpos + 1) : J;
    if (kv_lim > 0 && Jv > NG * (U / 2)) {   // (uniform)
        const int jl = min(Jv, kv_lim) - 1;
#pragma unroll
        for (int u = U / 2; u < U; u++) load_row_words<NW>(kbase + (size_t)min(g + NG * u, jl) * wstride, k0[u]);
#pragma unroll
        for (int u = U / 2; u < U; u++) load_row_words<NW>(vbase + (size_t)min(g + NG * u, jl) * wstride, v0[u]);
    }

    float mx = -INFINITY;
    for (int j0 = g; j0 < Jv; j0 += NG * U) {
        uint32_t kw[U][NW];
        if (j0 == g) {
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int t = 0; t < NW; t++) kw[u][t] = k0[u][t];
        } else {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int j = j0 + NG * u;
                if (j < Jv) load_row_words<NW>(kbase + (size_t)j * wstride, kw[u]);
                else
#pragma unroll
                    for (int t = 0; t < NW; t++) kw[u][t] = 0u;
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            float acc = 0.0f;
#pragma unroll
            for (int t = 0; t < NW; t++) {
                const h2 k2 = as_h2(kw[u][t]);
                acc += qf[2 * t] * (float)k2[0];
                acc += qf[2 * t + 1] * (float)k2[1];
            }
            acc = group8_sum(acc);
            const int j = j0 + NG * u;
            if (j < Jv) {
                const float v = h2f(f2h(h2f(f2h(acc)) * a.scale_h));
                if (c == 0) sc[j] = v;
                if (isfinite(v)) mx = fmaxf(mx, v);
            }
        }
    }
    mx = block_max1<NWV>(mx, red[0]);
    if (!isfinite(mx)) mx = 0.0f;
    float sum = 0.0f;
    for (int j = tid; j < Jv; j += NT) {
        const float v = sc[j];
        const float e = isfinite(v) ? expf(v - mx) : 0.0f;
        sc[j] = h2f(f2h(e));
        sum += e;
    }
    sum = block_sum1<NWV>(sum, red[1]);
    const bool degenerate = !(sum > 0.0f && isfinite(sum));
    const int Jp = degenerate ? J : Jv;
    const float uni = h2f(f2h(1.0f / (float)J));
    for (int j = tid; j < Jp; j += NT) sc[j] = degenerate ? uni : h2f(f2h(sc[j] / sum));
    __syncthreads();

    float o[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = 0.0f;
    for (int j0 = g; j0 < Jp; j0 += NG * U) {
        uint32_t vw[U][NW];
        if (j0 == g) {
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int t = 0; t < NW; t++) vw[u][t] = v0[u][t];
        } else {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int j = j0 + NG * u;
                if (j < Jp) load_row_words<NW>(vbase + (size_t)j * wstride, vw[u]);
                else
#pragma unroll
                    for (int t = 0; t < NW; t++) vw[u][t] = 0u;
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = j0 + NG * u;
            if (j < Jp) {
                const float pj = sc[j];
#pragma unroll
                for (int t = 0; t < NW; t++) {
                    const h2 v2 = as_h2(vw[u][t]);
                    o[2 * t] += pj * (float)v2[0];
                    o[2 * t + 1] += pj * (float)v2[1];
                }
            }
        }
    }
    // the 8 key groups of each wave (lanes with the same c), then the waves
#pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = stride8_sum(o[e]);
    if ((tid & 63) < 8)
#pragma unroll
        for (int e = 0; e < EPL; e++) part[tid >> 6][EPL * c + e] = o[e];
    lds_barrier();
    if (tid < D) {
        float t = part[0][tid];
#pragma unroll
        for (int wv = 1; wv < NWV; wv++) t += part[wv][tid];
        a.out[(size_t)s * os + (size_t)h * D + tid] = f2h(t);
    }
}

// ---------------------------------------------------------------------------
// Decode attention split over key chunks (head dims 80 / 128, long caches).
// One workgroup per head streams every K/V row of the head through one CU
// (~17 GB/s per CU for Phi-2's 5 KB-strided rows); here each head's keys
// are cut into AS_CH-key chunks handled by separate workgroups, keeping the
// rounding points of attention_dk_kernel:
//   1 asplit_scores : s_j = f16(f16(q.k_j) * scale) (same lane order as the
//                     one-workgroup kernel, so the same values), each
//                     chunk's max m_c over finite scores and its sum of
//                     exp(s_j - m_c)
//   2 asplit_pv     : global max M = max m_c (0 when none is finite), global
//                     sum = sum_c sum_c * exp(m_c - M) in chunk order (the
//                     reference's sum of exp(s_j - M), re-associated: ~1e-7
//                     relative), e_j = f16(exp(s_j - M)) (0 for non-finite
//                     s_j), P_j = f16(e_j / sum) (the uniform f16(1/J) when
//                     the sum is not a positive finite number), fp32 P.V
//                     partials per chunk
//   3 asplit_combine: the partials summed in chunk order, f16 out.
// Decode only (one query row, causal, position read on the device); rows
// are read at min(j, kv_rows - 1), inside the allocation.
constexpr int AS_CH = 128, AS_NT = 256, AS_NG = AS_NT / 8, AS_U = AS_CH / AS_NG;

struct SplitBufs {
    float* e;      // [H][kv_rows] scores
    float* mx;     // [H][nch] chunk maxima
    float* sum;    // [H][nch] chunk sums of exp(s - chunk max)
    float* o;      // [H][nch][D] P.V partials
    int nch;
};

__device__ __forceinline__ int asplit_keys(const AttnArgs& a) {
    return min(*a.d_pos + 1, a.kv_rows);
}

template <int D>
__global__ __launch_bounds__(AS_NT) void asplit_scores_kernel(AttnArgs a, SplitBufs b) {
    constexpr int EPL = D / 8, NW = EPL / 2, NWV = AS_NT / 64;
    __shared__ float red[2][NWV];
    const int ch = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, c = tid & 7, g = tid >> 3;
    const int kvh = h / (a.H / a.Hkv);
    const size_t wstride = (size_t)a.Hkv * D / 2;
    const uint32_t* kbase = (const uint32_t*)(a.k + (size_t)kvh * D + EPL * c);
    const int j0 = ch * AS_CH;
    uint32_t kw[AS_U][NW];
#pragma unroll
    for (int u = 0; u < AS_U; u++) load_row_words<NW>(kbase + (size_t)min(j0 + g + AS_NG * u, a.kv_rows - 1) * wstride, kw[u]);
    float qf[EPL];
    {
        const uint32_t* qw = (const uint32_t*)(a.q + (size_t)h * D + EPL * c);
#pragma unroll
        for (int t = 0; t < NW; t++) {
            const h2 p2 = as_h2(qw[t]);
            qf[2 * t] = (float)p2[0];
            qf[2 * t + 1] = (float)p2[1];
        }
    }
    const int J = asplit_keys(a);
    if (j0 >= J) return;   // (uniform: chunk past the keys)
    float mx = -INFINITY, sv[AS_U];
#pragma unroll
    for (int u = 0; u < AS_U; u++) {
        float acc = 0.0f;
#pragma unroll
        for (int t = 0; t < NW; t++) {
            const h2 k2 = as_h2(kw[u][t]);
            acc += qf[2 * t] * (float)k2[0];
            acc += qf[2 * t + 1] * (float)k2[1];
        }
        acc = group8_sum(acc);
        const int j = j0 + g + AS_NG * u;
        sv[u] = -INFINITY;
        if (j < J) {
            const float v = h2f(f2h(h2f(f2h(acc)) * a.scale_h));
            if (c == 0) b.e[(size_t)h * a.kv_rows + j] = v;
            if (isfinite(v)) {
                mx = fmaxf(mx, v);
                sv[u] = v;
            }
        }
    }
    mx = block_max1<NWV>(mx, red[0]);
    // the chunk's sum of exp(s - chunk max), one term per key (lane c = 0)
    float se = 0.0f;
    if (c == 0 && isfinite(mx))
#pragma unroll
        for (int u = 0; u < AS_U; u++)
            if (isfinite(sv[u])) se += expf(sv[u] - mx);
    se = block_sum1<NWV>(se, red[1]);
    if (tid == 0) {
        b.mx[(size_t)h * b.nch + ch] = mx;
        b.sum[(size_t)h * b.nch + ch] = se;
    }
}

template <int D>
__global__ __launch_bounds__(AS_NT) void asplit_pv_kernel(AttnArgs a, SplitBufs b) {
    constexpr int EPL = D / 8, NW = EPL / 2, NWV = AS_NT / 64;
    __shared__ float part[NWV][D];
    const int ch = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, c = tid & 7, g = tid >> 3;
    const int kvh = h / (a.H / a.Hkv);
    const size_t wstride = (size_t)a.Hkv * D / 2;
    const uint32_t* vbase = (const uint32_t*)(a.v + (size_t)kvh * D + EPL * c);
    const int j0 = ch * AS_CH;
    uint32_t vw[AS_U][NW];
#pragma unroll
    for (int u = 0; u < AS_U; u++) load_row_words<NW>(vbase + (size_t)min(j0 + g + AS_NG * u, a.kv_rows - 1) * wstride, vw[u]);
    const int J = asplit_keys(a);
    const int nc = (J + AS_CH - 1) / AS_CH;
    if (ch >= nc) return;
    float gmax = -INFINITY;
    for (int k = 0; k < nc; k++) gmax = fmaxf(gmax, b.mx[(size_t)h * b.nch + k]);
    if (!isfinite(gmax)) gmax = 0.0f;
    float gsum = 0.0f;
    for (int k = 0; k < nc; k++) {
        const float mk = b.mx[(size_t)h * b.nch + k];
        if (isfinite(mk)) gsum += b.sum[(size_t)h * b.nch + k] * expf(mk - gmax);
    }
    const bool degenerate = !(gsum > 0.0f && isfinite(gsum));
    const float uni = h2f(f2h(1.0f / (float)J));
    float o[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = 0.0f;
#pragma unroll
    for (int u = 0; u < AS_U; u++) {
        const int j = j0 + g + AS_NG * u;
        if (j < J) {
            const float sj = b.e[(size_t)h * a.kv_rows + j];
            const float ej = isfinite(sj) ? h2f(f2h(expf(sj - gmax))) : 0.0f;
            const float pj = degenerate ? uni : h2f(f2h(ej / gsum));
#pragma unroll
            for (int t = 0; t < NW; t++) {
                const h2 v2 = as_h2(vw[u][t]);
                o[2 * t] += pj * (float)v2[0];
                o[2 * t + 1] += pj * (float)v2[1];
            }
        }
    }
#pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = stride8_sum(o[e]);
    if ((tid & 63) < 8)
#pragma unroll
        for (int e = 0; e < EPL; e++) part[tid >> 6][EPL * c + e] = o[e];
    lds_barrier();
    if (tid < D) {
        float t = part[0][tid];
#pragma unroll
        for (int wv = 1; wv < NWV; wv++) t += part[wv][tid];
        b.o[((size_t)h * b.nch + ch) * D + tid] = t;
    }
}

template <int D>
__global__ __launch_bounds__(D) void asplit_combine_kernel(AttnArgs a, SplitBufs b) {
    const int h = blockIdx.x, tid = threadIdx.x;
    const int J = asplit_keys(a);
    const int nc = (J + AS_CH - 1) / AS_CH;
    float t = 0.0f;
    for (int k = 0; k < nc; k++) t += b.o[((size_t)h * b.nch + k) * D + tid];
    a.out[(size_t)h * D + tid] = f2h(t);   // (one query row)
}

bool attention_split_ok(const AttnArgs& a) {
    return a.d_pos && a.S == 1 && a.causal && (a.D == 80 || a.D == 128) && a.kv_rows > 512 && a.Hkv > 0 &&
           a.H % a.Hkv == 0;
}

size_t attention_split_scratch(int H, int kv_rows, int D) {
    const size_t nch = (size_t)(kv_rows + AS_CH - 1) / AS_CH;
    return ((size_t)H * kv_rows + 2 * (size_t)H * nch + (size_t)H * nch * D) * sizeof(float);
}

tlhip_status launch_attention_split(hipStream_t s, const AttnArgs& a, float* scratch) {
    if (!attention_split_ok(a) || !scratch)
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "attention: split decode path needs a device position, S = 1, D 80/128");
    SplitBufs b;
    b.nch = (a.kv_rows + AS_CH - 1) / AS_CH;
    b.e = scratch;
    b.mx = b.e + (size_t)a.H * a.kv_rows;
    b.sum = b.mx + (size_t)a.H * b.nch;
    b.o = b.sum + (size_t)a.H * b.nch;
    const dim3 grid((unsigned)b.nch, (unsigned)a.H);
    if (a.D == 80) {
        hipLaunchKernelGGL(asplit_scores_kernel<80>, grid, dim3(AS_NT), 0, s, a, b);
        hipLaunchKernelGGL(asplit_pv_kernel<80>, grid, dim3(AS_NT), 0, s, a, b);
        hipLaunchKernelGGL(asplit_combine_kernel<80>, dim3((unsigned)a.H), dim3(80), 0, s, a, b);
    } else {
        hipLaunchKernelGGL(asplit_scores_kernel<128>, grid, dim3(AS_NT), 0, s, a, b);
        hipLaunchKernelGGL(asplit_pv_kernel<128>, grid, dim3(AS_NT), 0, s, a, b);
        hipLaunchKernelGGL(asplit_combine_kernel<128>, dim3((unsigned)a.H), dim3(128), 0, s, a, b);
    }
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// Prefill attention on the matrix cores (S >= 32 query rows, head_dim a
// multiple of 16 up to 128).  Same arithmetic and rounding points as the
// kernels above -- f16 scores, f16 scale, masked keys skipped, exp in f32,
// P = f16(f16(e) / sum), fp32 accumulation of P.V -- organised so the two
// contractions run as v_mfma_f32_32x32x16_f16:
//   S^T[key][query] = K . Q^T  (A = 32 keys x 16 dims from K rows, B = 32
//                              queries x 16 dims from Q rows)
//   O[query][d]     = P . V    (A = P straight from S^T's accumulators,
//                              B = V^T rows from a transposed copy of V)
// In S^T's accumulator layout lane l owns query l%32 and keys
// 8(r/4) + 4(l/32) + r%4 (r = 0..15): the row statistics are per lane plus
// one exchange with lane l^32, and registers 8t..8t+7 are exactly the
// A operand of k-step t under the key order 16t + 8(i/4) + 4(l/32) + i%4,
// which V^T is read in (two 4-key runs per lane).
// Pass 1 over the key tiles keeps a running max and a rescaled sum of
// exp(s - max); pass 2 recomputes the scores, forms P with the final max and
// sum, and accumulates P.V.  Two waves own one head and a 32-row query tile
// (causal: the pair of tiles t and n-1-t, so every workgroup does the same
// work), each taking half of the key tiles; their row statistics meet in LDS
// after pass 1 and the upper half's partial O is added by the lower half
// after pass 2.  A workgroup holds four heads (two for head_dim 128), which
// under GQA share their K/V head in L1/L2.
// ---------------------------------------------------------------------------

// V [J, Hkv, D] -> Vt [Hkv, D, Jp], zero for keys J..Jp-1 (Jp % 32 == 0).
__global__ __launch_bounds__(256) void vt_transpose_kernel(const uint16_t* __restrict__ v, uint16_t* __restrict__ vt,
                                                         int J, int Jp, int Hkv, int D) {
    __shared__ uint16_t tile[128][33];
    const int j0 = blockIdx.x * 32, kvh = blockIdx.y;
    const size_t kstride = (size_t)Hkv * D;
    for (int d0 = 0; d0 < D; d0 += 128) {
        const int dn = min(128, D - d0);
        for (int i = threadIdx.x; i < 32 * dn; i += 256) {
            const int jj = i / dn, d = i % dn, j = j0 + jj;
            tile[d][jj] = j < J ? v[(size_t)j * kstride + (size_t)kvh * D + d0 + d] : (uint16_t)0;
        }
        __syncthreads();
        for (int i = threadIdx.x; i < 32 * dn; i += 256) {
            const int d = i / 32, jj = i % 32;
            vt[((size_t)kvh * D + d0 + d) * Jp + j0 + jj] = tile[d][jj];
        }
        __syncthreads();
    }
}

__device__ __forceinline__ h8 zero_h8() {
    h8 z;
#pragma unroll
    for (int i = 0; i < 8; i++) z[i] = (h16)0.0f;
    return z;
}

// The correctly rounded quotient a / b given r ~ 1/b (one residual
// correction of the product; a in [0, 1], b >= 1 here).
__device__ __forceinline__ float div_corr(float a, float b, float r) {
    const float q = a * r;
    return fmaf(fmaf(-b, q, a), r, q);
}

// Score of an excluded key: finite, so differences stay finite, and far
// enough below any f16 score that its exponential is exactly 0.
constexpr float FA_NEG = -1.0e30f;

// e^x for x <= 0 to a few f32 ulps: the terms of the softmax denominator,
// whose sum only needs f32-level relative accuracy.
__device__ __forceinline__ float exp_sum(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269502162933349609375f);
}

// Running (max, sum) pairs combined: each sum rescaled to the common max.
__device__ __forceinline__ float fa_merge(float m1, float s1, float m2, float s2, float m) {
    return (m1 > FA_NEG ? s1 * exp_sum(m1 - m) : 0.0f) + (m2 > FA_NEG ? s2 * exp_sum(m2 - m) : 0.0f);
}

template <int D>
struct FaWave {
    static constexpr int KS = D / 16;          // k-steps of QK^T
    static constexpr int NT = (D + 31) / 32;   // 32-wide output tiles of P.V

    AttnArgs a;
    const uint16_t* vt;
    int J, Jp, h, kvh, lane, qs, os;
    size_t kstride;

    __device__ FaWave(const AttnArgs& a_, const uint16_t* vt_, int J_, int Jp_, int h_)
        : a(a_), vt(vt_), J(J_), Jp(Jp_), h(h_) {
        kvh = h / (a.H / a.Hkv);
        lane = threadIdx.x & 63;
        qs = a.q_stride ? a.q_stride : a.H * D;
        os = a.out_stride ? a.out_stride : a.H * D;
        kstride = (size_t)a.Hkv * D;
    }

    // K rows of tile kt (rows past J read row J-1: their scores are masked)
    __device__ __forceinline__ void load_k(int kt, h8 (&kf)[KS]) const {
        const int j = min(kt * 32 + (lane & 31), J - 1);
        const uint16_t* kr = a.k + (size_t)j * kstride + (size_t)kvh * D + 8 * (lane >> 5);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) kf[ks] = *(const h8*)(kr + 16 * ks);
    }

    // V^T operands of tile kt (columns past D read column D-1: their output
    // columns are not stored; keys J..Jp-1 are zero in vt)
    __device__ __forceinline__ void load_v(int kt, h8 (&vb)[NT][2]) const {
        const int jb = kt * 32 + 4 * (lane >> 5);
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const int d = min(32 * n + (lane & 31), D - 1);
            const uint16_t* vr = vt + ((size_t)kvh * D + d) * Jp + jb;
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint2 lo = *(const uint2*)(vr + 16 * t);
                const uint2 hi = *(const uint2*)(vr + 16 * t + 8);
                const u4 w = {lo.x, lo.y, hi.x, hi.y};
                vb[n][t] = __builtin_bit_cast(h8, w);
            }
        }
    }

    __device__ __forceinline__ f16v qk(const h8 (&qf)[KS], const h8 (&kf)[KS]) const {
        f16v acc = {};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[ks], qf[ks], acc, 0, 0, 0);
        return acc;
    }

    // scores of key tile kt for this lane's query, as the reference stores
    // them (f16 dot product, then the f16 product with the f16 scale);
    // excluded keys (masked, past J, non-finite) come back as FA_NEG.
    // FULL: every key of the tile is unmasked for every query of the wave.
    template <bool FULL>
    __device__ __forceinline__ void scores(int kt, const f16v& acc, int jlim, float (&sv)[16]) const {
        const int jb = kt * 32 + 4 * (lane >> 5);
        const h2 sc2 = {(h16)a.scale_h, (h16)a.scale_h};
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            h2 x = {(h16)acc[r], (h16)acc[r + 1]};
            x = x * sc2;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float v = (float)x[u];
                bool ok = isfinite(v);
                if (!FULL) ok = ok && jb + 8 * ((r + u) >> 2) + ((r + u) & 3) <= jlim;
                sv[r + u] = ok ? v : FA_NEG;
            }
        }
    }

    // pass 1 over tiles [k0, k1): running max and rescaled sum of exp(s - max)
    __device__ __forceinline__ void pass1(const h8 (&qf)[KS], int k0, int k1, int nfull, int jlim, float& mx,
                                          float& sum) const {
        mx = FA_NEG;
        sum = 0.0f;
        if (k0 >= k1) return;
        // the QK^T product of tile kt+1 runs on the matrix core while the
        // vector unit works on tile kt
        h8 kf[KS];
        load_k(k0, kf);
        f16v acc = qk(qf, kf);
        if (k0 + 1 < k1) load_k(k0 + 1, kf);
        for (int kt = k0; kt < k1; kt++) {
            f16v accn = acc;
            if (kt + 1 < k1) accn = qk(qf, kf);
            if (kt + 2 < k1) load_k(kt + 2, kf);
            float sv[16];
            if (kt < nfull) scores<true>(kt, acc, jlim, sv);
            else scores<false>(kt, acc, jlim, sv);
            acc = accn;
            float mt = sv[0];
#pragma unroll
            for (int r = 1; r < 16; r++) mt = fmaxf(mt, sv[r]);
            if (mt > mx) {
                sum = sum * exp_sum(mx - mt);
                mx = mt;
            }
            float es[16];
#pragma unroll
            for (int r = 0; r < 16; r++) es[r] = exp_sum(sv[r] - mx);
            // pairwise, so the adds are not one dependent chain
#pragma unroll
            for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
                for (int r = 0; r < w; r++) es[r] += es[r + w];
            if (mx > FA_NEG) sum += es[0];
        }
    }

    // pass 2 over tiles [k0, k1): P = f16(f16(e) / sum) (DEG: rows with no
    // finite score weight every key < J by f16(1/J)), O += P . V
    template <bool DEG>
    __device__ __forceinline__ void pass2(const h8 (&qf)[KS], int k0, int k1, int nfull, int jlim, float m,
                                          float tot, bool deg, f16v (&o)[NT]) const {
        if (k0 >= k1) return;
        const float rt = 1.0f / tot;
        const float uni = h2f(f2h(1.0f / (float)J));
        // the QK^T product of tile kt+1 runs on the matrix core while the
        // vector unit forms P of tile kt
        h8 kf[KS];
        load_k(k0, kf);
        f16v acc = qk(qf, kf);
        if (k0 + 1 < k1) load_k(k0 + 1, kf);
        for (int kt = k0; kt < k1; kt++) {
            h8 vb[NT][2];
            load_v(kt, vb);
            f16v accn = acc;
            if (kt + 1 < k1) accn = qk(qf, kf);
            if (kt + 2 < k1) load_k(kt + 2, kf);
            float sv[16];
            if (kt < nfull) scores<true>(kt, acc, jlim, sv);
            else scores<false>(kt, acc, jlim, sv);
            acc = accn;
            // e = f16(exp(x)), x = s - max <= 0: 2^(x log2 e) on v_exp_f32,
            // with the rounding error of the product x * f32(log2 e) and the
            // tail of log2 e added back as a first-order term, so e stays
            // within about an ulp of exp(x) before its f16 rounding.  Written
            // stage by stage over the 16 scores, so 16 independent chains
            // stand between dependent instructions.
            constexpr float L1 = 1.44269502162933349609375f, L2 = 1.925963033500011e-8f;
            constexpr float LN2 = 0.6931471805599453f;
            float x[16], t[16], e[16], c[16];
#pragma unroll
            for (int r = 0; r < 16; r++) x[r] = sv[r] - m;
#pragma unroll
            for (int r = 0; r < 16; r++) t[r] = x[r] * L1;
#pragma unroll
            for (int r = 0; r < 16; r++) e[r] = __builtin_amdgcn_exp2f(t[r]);
#pragma unroll
            for (int r = 0; r < 16; r++) c[r] = fmaf(x[r], L2, fmaf(x[r], L1, -t[r]));
            h8 pa[2];
#pragma unroll
            for (int r = 0; r < 16; r++) pa[r >> 3][r & 7] = (h16)fmaf(e[r] * LN2, c[r], e[r]);   // f16(exp(x))
#pragma unroll
            for (int r = 0; r < 16; r++) e[r] = (float)pa[r >> 3][r & 7];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float pv = div_corr(e[r], tot, rt);
                if (DEG) {
                    const int j = kt * 32 + 4 * (lane >> 5) + 8 * (r >> 2) + (r & 3);
                    pv = deg ? (j < J ? uni : 0.0f) : pv;
                }
                pa[r >> 3][r & 7] = (h16)pv;
            }
#pragma unroll
            for (int n = 0; n < NT; n++)
#pragma unroll
                for (int t = 0; t < 2; t++) o[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa[t], vb[n][t], o[n], 0, 0, 0);
        }
    }

    // Query tile qt, key half `half` of its tiles.  stm/sts: this head's
    // [2][32] exchange of row statistics; ob: [NT][16][64] partial O of the
    // upper half.  Two workgroup barriers, reached by every wave.
    __device__ void run(int qt, int half, bool store, float* stm, float* sts, float* ob) const {
        const int s0 = qt * 32;
        const int myq = s0 + (lane & 31);
        const int qpos = a.q_pos0 + myq;
        const int last = min(s0 + 31, a.S - 1);
        const int kend = a.causal ? min(J, a.q_pos0 + last + 1) : J;
        const int nkt = (kend + 31) / 32;
        const int jlim = a.causal ? min(J - 1, qpos) : J - 1;
        // tiles below every query's limit need no mask test
        const int lo_lim = a.causal ? min(J - 1, a.q_pos0 + s0) : J - 1;
        const int nfull = (lo_lim + 1) / 32;
        const int nh = (nkt + 1) / 2;

        h8 qf[KS];
        {
            const uint16_t* qr = a.q + (size_t)min(myq, a.S - 1) * qs + (size_t)h * D + 8 * (lane >> 5);
#pragma unroll
            for (int ks = 0; ks < KS; ks++) qf[ks] = *(const h8*)(qr + 16 * ks);
        }

        float mx, sum;
        pass1(qf, half ? nh : 0, half ? nkt : nh, nfull, jlim, mx, sum);
        // the other 16 keys of every tile sit in lane l ^ 32, the other key
        // half in the partner wave; both sides form the same sums
        const float mo = __shfl_xor(mx, 32, 64), so = __shfl_xor(sum, 32, 64);
        const float m1 = fmaxf(mx, mo);
        const float t1 = fa_merge(mx, sum, mo, so, m1);
        if (lane < 32) {
            stm[half * 32 + lane] = m1;
            sts[half * 32 + lane] = t1;
        }
        __syncthreads();
        const float m2 = stm[(half ^ 1) * 32 + (lane & 31)], t2 = sts[(half ^ 1) * 32 + (lane & 31)];
        const float m = fmaxf(m1, m2);
        const float tot = fa_merge(m1, t1, m2, t2, m);
        const bool deg = !(tot > 0.0f && isfinite(tot)) && myq < a.S;

        f16v o[NT];
#pragma unroll
        for (int n = 0; n < NT; n++) o[n] = f16v{};
        if (__any(deg)) {
            const int nk = Jp / 32, nhd = (nk + 1) / 2;
            pass2<true>(qf, half ? nhd : 0, half ? nk : nhd, 0, jlim, m, tot, deg, o);
        } else {
            pass2<false>(qf, half ? nh : 0, half ? nkt : nh, nfull, jlim, m, tot, false, o);
        }

        if (half) {
#pragma unroll
            for (int n = 0; n < NT; n++)
#pragma unroll
                for (int r = 0; r < 16; r++) ob[(n * 16 + r) * 64 + lane] = o[n][r];
        }
        __syncthreads();
        if (!half && store) {
            // O accumulators: column d = 32n + l%32, rows 8(r/4) + 4(l/32) + r%4
#pragma unroll
            for (int n = 0; n < NT; n++) {
                const int d = 32 * n + (lane & 31);
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = s0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    const float t = o[n][r] + ob[(n * 16 + r) * 64 + lane];
                    if (row < a.S && d < D) a.out[(size_t)row * os + (size_t)h * D + d] = f2h(t);
                }
            }
        }
    }
};

// Heads per workgroup (each head = two waves, one per key half).
template <int D>
constexpr int fa_heads() { return D > 80 ? 2 : 4; }

template <int D>
__global__ __launch_bounds__(fa_heads<D>() * 128) void attention_mfma_kernel(AttnArgs a, const uint16_t* __restrict__ vt, int J,
                                                             int Jp, int nqt) {
    constexpr int HPW = fa_heads<D>(), NT = (D + 31) / 32;
    __shared__ float stm[HPW][64], sts[HPW][64];
    __shared__ float ob[HPW][NT * 16 * 64];
    const int w = threadIdx.x >> 6, hw = w % HPW, half = w / HPW;
    const int hh = blockIdx.y * HPW + hw;
    const FaWave<D> fw(a, vt, J, Jp, min(hh, a.H - 1));
    const bool store = hh < a.H;
    if (a.causal) {
        const int t0 = nqt - 1 - (int)blockIdx.x, t1 = blockIdx.x;
        fw.run(t0, half, store, stm[hw], sts[hw], ob[hw]);
        if (t1 < t0) fw.run(t1, half, store, stm[hw], sts[hw], ob[hw]);
    } else {
        fw.run(blockIdx.x, half, store, stm[hw], sts[hw], ob[hw]);
    }
}

bool attention_mfma_ok(const AttnArgs& a, int J) {
    const int qs = a.q_stride ? a.q_stride : a.H * a.D;
    return a.S >= 128 && J >= 1 && (a.D == 64 || a.D == 80 || a.D == 128) && !a.d_pos && qs % 8 == 0 &&
           ((uintptr_t)a.q % 16) == 0 && ((uintptr_t)a.k % 16) == 0;
}

size_t attention_mfma_scratch(int J, int Hkv, int D) {
    return (size_t)Hkv * D * (size_t)((J + 31) / 32 * 32) * sizeof(uint16_t);
}

// Prefill over J keys through the matrix cores; vt holds
// attention_mfma_scratch(J, Hkv, D) bytes.
tlhip_status launch_attention_mfma(hipStream_t s, const AttnArgs& a, int J, uint16_t* vt) {
    if (!attention_mfma_ok(a, J) || !vt)
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "attention: shape not on the matrix-core path");
    if (a.Hkv <= 0 || a.H % a.Hkv) return fail(TLHIP_ERR_INVALID_DIMENSION, "attention: heads %d/%d", a.H, a.Hkv);
    if (J > ATT_MAX_J) return fail(TLHIP_ERR_INVALID_DIMENSION, "attention: %d keys > %d", J, ATT_MAX_J);
    const int Jp = (J + 31) / 32 * 32;
    hipLaunchKernelGGL(vt_transpose_kernel, dim3(Jp / 32, a.Hkv), dim3(256), 0, s, a.v, vt, J, Jp, a.Hkv, a.D);
    const int nqt = (a.S + 31) / 32;
    const int gx = a.causal ? (nqt + 1) / 2 : nqt;
    if (a.D == 64)
        hipLaunchKernelGGL(attention_mfma_kernel<64>, dim3(gx, (a.H + 3) / 4), dim3(512), 0, s, a, vt, J, Jp, nqt);
    else if (a.D == 80)
        hipLaunchKernelGGL(attention_mfma_kernel<80>, dim3(gx, (a.H + 3) / 4), dim3(512), 0, s, a, vt, J, Jp, nqt);
    else
        hipLaunchKernelGGL(attention_mfma_kernel<128>, dim3(gx, (a.H + 1) / 2), dim3(256), 0, s, a, vt, J, Jp, nqt);
    return TLHIP_OK;
}

static void launch_attn_any(hipStream_t s, const AttnArgs& a, int J) {
    // a key count known at launch above one 256-key pass takes the 512-thread
    // variant (512 keys per pass); decode (J read on the device) keeps 256
    if (a.D == 64 && !a.d_pos && J > 256) hipLaunchKernelGGL(attention64_kernel<512>, dim3(a.S, a.H), dim3(512), 0, s, a, J);
    else if (a.D == 64) hipLaunchKernelGGL(attention64_kernel<256>, dim3(a.S, a.H), dim3(256), 0, s, a, J);
    else if (a.D == 80) hipLaunchKernelGGL(attention_dk_kernel<80>, dim3(a.S, a.H), dim3(ADK_THREADS), 0, s, a, J);
    else if (a.D == 128) hipLaunchKernelGGL(attention_dk_kernel<128>, dim3(a.S, a.H), dim3(ADK_THREADS), 0, s, a, J);
    else hipLaunchKernelGGL(attention_kernel, dim3(a.S, a.H), dim3(256), 0, s, a, J);
}

tlhip_status launch_attention(hipStream_t s, const AttnArgs& a) {
    if (a.D > 256 || a.D <= 0) return fail(TLHIP_ERR_INVALID_DIMENSION, "attention: head_dim %d", a.D);
    if (a.Hkv <= 0 || a.H % a.Hkv) return fail(TLHIP_ERR_INVALID_DIMENSION, "attention: heads %d/%d", a.H, a.Hkv);
    if (a.S <= 0) return TLHIP_OK;
    launch_attn_any(s, a, 0);
    return TLHIP_OK;
}

tlhip_status launch_attention_j(hipStream_t s, const AttnArgs& a, int J) {
    if (J > ATT_MAX_J) return fail(TLHIP_ERR_INVALID_DIMENSION, "attention: %d keys > %d", J, ATT_MAX_J);
    if (a.D > 256 || a.D <= 0) return fail(TLHIP_ERR_INVALID_DIMENSION, "attention: head_dim %d", a.D);
    if (a.Hkv <= 0 || a.H % a.Hkv) return fail(TLHIP_ERR_INVALID_DIMENSION, "attention: heads %d/%d", a.H, a.Hkv);
    if (a.S <= 0) return TLHIP_OK;
    launch_attn_any(s, a, J);
    return TLHIP_OK;
}

// einsum("ihd,jhd->ihj"): one thread per output, fp32 accumulate in d order.
__global__ void scores_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                              uint16_t* __restrict__ out, int I, int J, int H, int Hkv, int D) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)I * H * J) return;
    const int j = (int)(idx % J);
    const int h = (int)((idx / J) % H);
    const int i = (int)(idx / ((int64_t)J * H));
    const int kvh = h / (H / Hkv);
    const uint16_t* qr = q + ((size_t)i * H + h) * D;
    const uint16_t* kr = k + ((size_t)j * Hkv + kvh) * D;
    float acc = 0.0f;
    for (int d = 0; d < D; d++) acc += h2f(qr[d]) * h2f(kr[d]);
    out[idx] = f2h(acc);
}

// einsum("ihj,jhd->ihd") with fp32 accumulation in j order.
__global__ void context_kernel(const uint16_t* __restrict__ p, const uint16_t* __restrict__ v,
                               uint16_t* __restrict__ out, int I, int J, int H, int Hkv, int D) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)I * H * D) return;
    const int d = (int)(idx % D);
    const int h = (int)((idx / D) % H);
    const int i = (int)(idx / ((int64_t)D * H));
    const int kvh = h / (H / Hkv);
    const uint16_t* pr = p + ((size_t)i * H + h) * J;
    float acc = 0.0f;
    for (int j = 0; j < J; j++) acc += h2f(pr[j]) * h2f(v[((size_t)j * Hkv + kvh) * D + d]);
    out[idx] = f2h(acc);
}

tlhip_status launch_scores(hipStream_t s, const uint16_t* q, const uint16_t* k, uint16_t* sc, int I,
                           int J, int H, int Hkv, int D) {
    int64_t n = (int64_t)I * H * J;
    if (n <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(scores_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, q, k, sc, I, J, H,
                       Hkv, D);
    return TLHIP_OK;
}

tlhip_status launch_context(hipStream_t s, const uint16_t* p, const uint16_t* v, uint16_t* out, int I,
                            int J, int H, int Hkv, int D) {
    int64_t n = (int64_t)I * H * D;
    if (n <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(context_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, v, out, I, J,
                       H, Hkv, D);
    return TLHIP_OK;
}

}  // namespace tlhip
