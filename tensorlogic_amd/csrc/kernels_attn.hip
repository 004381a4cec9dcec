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

__global__ __launch_bounds__(256) void attention64_kernel(AttnArgs a, int J_fixed) {
    __shared__ float sc[ATT_MAX_J];
    __shared__ float red[4];
    __shared__ float part[4][64];
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
    // the first pass of K and V rows (bounded by the rows allocated, so
    // every address is in bounds; rows past the key count are never used).
    const u4 qv = *(const u4*)(a.q + (size_t)s * qs + (size_t)h * 64 + 8 * c);
    const int kv_lim = a.kv_rows > 0 ? a.kv_rows : min(J_fixed, ATT_MAX_J);
    u4 k0[A64_UNR], vv[A64_UNR];
#pragma unroll
    for (int u = 0; u < A64_UNR; u++) {
        const int j = g + 32 * u;
        k0[u] = j < kv_lim ? *(const u4*)(kbase + (size_t)j * kstride) : u4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < A64_UNR; u++) {
        const int j = g + 32 * u;
        vv[u] = j < kv_lim ? *(const u4*)(vbase + (size_t)j * kstride) : u4{0u, 0u, 0u, 0u};
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

    // One pass covers 32 * A64_UNR keys; the first pass uses the rows loaded
    // above.  When the unmasked row fits in that pass, the V rows loaded
    // with it are used directly (one round trip to memory in all).
    const bool one_pass = Jv <= 32 * A64_UNR;
    float mx = -INFINITY;
    for (int j0 = g; j0 < Jv; j0 += 32 * A64_UNR) {
        u4 kv[A64_UNR];
        if (j0 == g) {
#pragma unroll
            for (int u = 0; u < A64_UNR; u++) kv[u] = k0[u];
        } else {
#pragma unroll
            for (int u = 0; u < A64_UNR; u++) {
                const int j = j0 + 32 * u;
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
            const int j = j0 + 32 * u;
            if (j < Jv) {
                const float v = h2f(f2h(h2f(f2h(acc)) * a.scale_h));
                if (c == 0) sc[j] = v;
                if (isfinite(v)) mx = fmaxf(mx, v);
            }
        }
    }
    mx = bmax(mx, red);   // (its barriers also publish sc[])
    if (!isfinite(mx)) mx = 0.0f;
    float sum = 0.0f;
    for (int j = tid; j < Jv; j += 256) {
        const float v = sc[j];
        const float e = isfinite(v) ? expf(v - mx) : 0.0f;
        sc[j] = h2f(f2h(e));
        sum += e;
    }
    sum = bsum(sum, red);
    const bool degenerate = !(sum > 0.0f && isfinite(sum));
    const int Jp = degenerate ? J : Jv;
    const float uni = h2f(f2h(1.0f / (float)J));
    for (int j = tid; j < Jp; j += 256) sc[j] = degenerate ? uni : h2f(f2h(sc[j] / sum));
    __syncthreads();

    float o[8];
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = 0.0f;
    if (one_pass && !degenerate) {
#pragma unroll
        for (int u = 0; u < A64_UNR; u++) {
            const int j = g + 32 * u;
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
        for (int j0 = g; j0 < Jp; j0 += 32 * A64_UNR) {
#pragma unroll
            for (int u = 0; u < A64_UNR; u++) {
                const int j = j0 + 32 * u;
                vv[u] = j < Jp ? *(const u4*)(vbase + (size_t)j * kstride) : u4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < A64_UNR; u++) {
                const int j = j0 + 32 * u;
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
        const float t = (part[0][tid] + part[1][tid]) + (part[2][tid] + part[3][tid]);
        a.out[(size_t)s * os + (size_t)h * 64 + tid] = f2h(t);
    }
}

// The same kernel for other even head dims D = 8 * EPL (Phi-2: 80): lane c
// of a key's 8 lanes holds dims EPL*c .. EPL*c + EPL - 1, read as EPL/2
// 4-byte words; one pass covers 32 keys; partial context rows are summed
// in key-group order.
template <int D>
__global__ __launch_bounds__(256) void attention_dk_kernel(AttnArgs a, int J_fixed) {
    constexpr int EPL = D / 8, NW = EPL / 2;
    __shared__ float sc[ATT_MAX_J];
    __shared__ float red[4];
    __shared__ float part[32][D + 1];
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

    float mx = -INFINITY;
    for (int j0 = g; j0 < Jv; j0 += 32 * 4) {
        uint32_t kw[4][NW];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int j = j0 + 32 * u;
#pragma unroll
            for (int t = 0; t < NW; t++) kw[u][t] = j < Jv ? kbase[(size_t)j * wstride + t] : 0u;
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            float acc = 0.0f;
#pragma unroll
            for (int t = 0; t < NW; t++) {
                const h2 k2 = as_h2(kw[u][t]);
                acc += qf[2 * t] * (float)k2[0];
                acc += qf[2 * t + 1] * (float)k2[1];
            }
            acc = group8_sum(acc);
            const int j = j0 + 32 * u;
            if (j < Jv) {
                const float v = h2f(f2h(h2f(f2h(acc)) * a.scale_h));
                if (c == 0) sc[j] = v;
                if (isfinite(v)) mx = fmaxf(mx, v);
            }
        }
    }
    mx = bmax(mx, red);
    if (!isfinite(mx)) mx = 0.0f;
    float sum = 0.0f;
    for (int j = tid; j < Jv; j += 256) {
        const float v = sc[j];
        const float e = isfinite(v) ? expf(v - mx) : 0.0f;
        sc[j] = h2f(f2h(e));
        sum += e;
    }
    sum = bsum(sum, red);
    const bool degenerate = !(sum > 0.0f && isfinite(sum));
    const int Jp = degenerate ? J : Jv;
    const float uni = h2f(f2h(1.0f / (float)J));
    for (int j = tid; j < Jp; j += 256) sc[j] = degenerate ? uni : h2f(f2h(sc[j] / sum));
    __syncthreads();

    float o[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = 0.0f;
    for (int j0 = g; j0 < Jp; j0 += 32 * 4) {
        uint32_t vw[4][NW];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int j = j0 + 32 * u;
#pragma unroll
            for (int t = 0; t < NW; t++) vw[u][t] = j < Jp ? vbase[(size_t)j * wstride + t] : 0u;
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int j = j0 + 32 * u;
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
#pragma unroll
    for (int e = 0; e < EPL; e++) part[g][EPL * c + e] = o[e];
    __syncthreads();
    if (tid < D) {
        float t = part[0][tid];
        for (int gg = 1; gg < 32; gg++) t += part[gg][tid];
        a.out[(size_t)s * os + (size_t)h * D + tid] = f2h(t);
    }
}

static void launch_attn_any(hipStream_t s, const AttnArgs& a, int J) {
    if (a.D == 64) hipLaunchKernelGGL(attention64_kernel, dim3(a.S, a.H), dim3(256), 0, s, a, J);
    else if (a.D == 80) hipLaunchKernelGGL(attention_dk_kernel<80>, dim3(a.S, a.H), dim3(256), 0, s, a, J);
    else if (a.D == 128) hipLaunchKernelGGL(attention_dk_kernel<128>, dim3(a.S, a.H), dim3(256), 0, s, a, J);
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
