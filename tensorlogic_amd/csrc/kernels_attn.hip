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
#include "gemv_device.hpp"
#include "internal.hpp"

namespace tlhip {

constexpr int ATT_MAX_J = kAttnRowKeys;   // keys held in LDS by the single-pass kernel

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

// JMAX: keys the score row holds; below ATT_MAX_J only for a key count
// known at launch (no d_pos) of at most JMAX -- the smaller row lets more
// workgroups share a CU.  UNR: K / V rows per key group and pass (fewer
// registers, so more workgroups per CU, for short rows).
// DEC: the decode step's launch (one query row, position read from d_pos,
// causal, default row strides, the cache's allocated rows known) with those
// facts as constants, so the compiler drops the other cases' code.
__device__ __forceinline__ AttnArgs attn_dec_view(const AttnArgs& k) {
    AttnArgs a;
    a.q = k.q;
    a.k = k.k;
    a.v = k.v;
    a.out = k.out;
    a.S = 1;
    a.H = k.H;
    a.Hkv = k.Hkv;
    a.D = 64;
    a.q_pos0 = 0;
    a.d_pos = k.d_pos;
    a.causal = 1;
    a.scale_h = k.scale_h;
    a.q_stride = 0;
    a.out_stride = 0;
    a.kv_rows = k.kv_rows;
    return a;
}

template <int NT, int JMAX = ATT_MAX_J, int UNR = A64_UNR, bool DEC = false>
__global__ __launch_bounds__(NT) void attention64_kernel(AttnArgs ak, int J_fixed) {
    constexpr int NWV = NT / 64, NG = NT / 8;
    __shared__ float sc[JMAX];
    __shared__ float red[2][NWV];
    __shared__ float part[NWV][64];
    const AttnArgs a = DEC ? attn_dec_view(ak) : ak;
    if constexpr (DEC) {   // (the launch checks both)
        J_fixed = 0;
        __builtin_assume(a.d_pos != nullptr);
        __builtin_assume(a.kv_rows > 0);
    }
    attn_kernarg_fence(a, J_fixed);
    const int s = DEC ? 0 : (int)blockIdx.x;
    // One query row: workgroup i runs on XCD i % 8, so heads are dealt out
    // XCD-major (XCD x takes heads x * H/8 .. x * H/8 + H/8 - 1) and the
    // query heads that share a KV head read its rows through one or two
    // L2s instead of all eight.
    const int h = ((DEC || gridDim.x == 1) && (a.H & 7) == 0) ? (blockIdx.y & 7) * (a.H >> 3) + (blockIdx.y >> 3) : blockIdx.y;
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
    const int kv_lim = a.kv_rows > 0 ? (a.d_pos ? a.kv_rows : min(a.kv_rows, J_fixed)) : min(J_fixed, JMAX);
    u4 k0[UNR], vv[UNR];
    if (kv_lim > 0) {   // (uniform; 0 only when neither a key count nor the rows allocated is known)
#pragma unroll
        for (int u = 0; u < UNR; u++) k0[u] = *(const u4*)(kbase + (size_t)min(g + NG * u, kv_lim - 1) * kstride);
#pragma unroll
        for (int u = 0; u < UNR; u++) vv[u] = *(const u4*)(vbase + (size_t)min(g + NG * u, kv_lim - 1) * kstride);
    } else {
#pragma unroll
        for (int u = 0; u < UNR; u++) k0[u] = vv[u] = u4{0u, 0u, 0u, 0u};
    }
    const int qpos = (a.d_pos ? *a.d_pos : a.q_pos0) + s;
    const int J = min(a.d_pos ? qpos + 1 : J_fixed, JMAX);
    const int Jv = a.causal ? min(J, qpos + 1) : J;

    float qf[8];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const h2 p2 = as_h2(qv[t]);
        qf[2 * t] = (float)p2[0];
        qf[2 * t + 1] = (float)p2[1];
    }

    // One pass covers NG * UNR keys; the first pass uses the rows loaded
    // above.  When the unmasked row fits in that pass, the V rows loaded
    // with it are used directly (one round trip to memory in all).
    const bool one_pass = Jv <= NG * UNR;
    float mx = -INFINITY;
    for (int j0 = g; j0 < Jv; j0 += NG * UNR) {
        u4 kv[UNR];
        if (j0 == g) {
#pragma unroll
            for (int u = 0; u < UNR; u++) kv[u] = k0[u];
        } else {
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const int j = j0 + NG * u;
                kv[u] = j < Jv ? *(const u4*)(kbase + (size_t)j * kstride) : u4{0u, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int u = 0; u < UNR; u++) {
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
    sum = block_sum1<NWV>(sum, red[1]);   // (its barrier also publishes the e values in sc[])
    const bool degenerate = !(sum > 0.0f && isfinite(sum));
    const int Jp = degenerate ? J : Jv;
    const float uni = h2f(f2h(1.0f / (float)J));
    // P_j = f16(e_j / sum), or the uniform row, formed by the lanes that use
    // it: no pass over the score row and no barrier between the sum and P.V
    auto pval = [&](int j) { return degenerate ? uni : h2f(f2h(sc[j] / sum)); };

    float o[8];
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = 0.0f;
    if (one_pass && !degenerate) {
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int j = g + NG * u;
            if (j < Jp) {
                const float pj = pval(j);
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const h2 v2 = as_h2(vv[u][t]);
                    o[2 * t] += pj * (float)v2[0];
                    o[2 * t + 1] += pj * (float)v2[1];
                }
            }
        }
    } else {
        for (int j0 = g; j0 < Jp; j0 += NG * UNR) {
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const int j = j0 + NG * u;
                vv[u] = j < Jp ? *(const u4*)(vbase + (size_t)j * kstride) : u4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const int j = j0 + NG * u;
                if (j < Jp) {
                    const float pj = pval(j);
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
template <int D, int JMAX = ATT_MAX_J>   // JMAX as in attention64_kernel
__global__ __launch_bounds__(ADK_THREADS) void attention_dk_kernel(AttnArgs a, int J_fixed) {
    constexpr int EPL = D / 8, NW = EPL / 2, U = ADK_UNR, NT = ADK_THREADS, NWV = NT / 64, NG = NT / 8;
    __shared__ float sc[JMAX];
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
    const int kv_lim = a.kv_rows > 0 ? (a.d_pos ? a.kv_rows : min(a.kv_rows, J_fixed)) : min(J_fixed, JMAX);
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
    const int J = min(a.d_pos ? qpos + 1 : J_fixed, JMAX);
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
    sum = block_sum1<NWV>(sum, red[1]);   // (its barrier also publishes the e values in sc[])
    const bool degenerate = !(sum > 0.0f && isfinite(sum));
    const int Jp = degenerate ? J : Jv;
    const float uni = h2f(f2h(1.0f / (float)J));
    // P_j formed where it is used, as in attention64_kernel
    auto pval = [&](int j) { return degenerate ? uni : h2f(f2h(sc[j] / sum)); };

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
                const float pj = pval(j);
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
// Decode attention split over key chunks (head dims 80 / 128, long caches),
// one launch (flash decoding).  One workgroup per head streams every K/V
// row of the head through one CU (~17 GB/s per CU for Phi-2's 5 KB-strided
// rows); here each head's keys are cut into CH-key chunks handled by
// separate workgroups.  A chunk's workgroup computes
//   s_j  = f16(f16(q.k_j) * scale)      (the one-workgroup kernels' lane
//                                        order, so the same score values)
//   m_c  = max of the chunk's finite s_j,  p_j = exp(s_j - m_c) in fp32
//          (0 for a non-finite s_j),  S_c = sum p_j,  o_c = sum p_j v_j,
// and publishes (m_c, S_c, o_c); the last of the head's workgroups to arrive
// (or, for heads of more than AS_XCH_CHUNKS chunks, asplit_combine_kernel
// after the kernel boundary) combines them in chunk order:
//   M = max m_c,  w_c = exp(m_c - M),  out = f16(sum_c w_c o_c / sum_c w_c S_c),
// the reference's softmax re-associated by chunk (its e_j and P_j are
// rounded to f16 before the P.V sum; here they stay fp32 -- the departure
// the matrix-core prefill attention makes too).  A chunk with no finite
// score keeps p_j = 1 (its plain V sum): when no chunk of the head has one,
// the row is the reference's degenerate uniform f16(1/J) over every key.
// The in-kernel exchange is the skinny GEMM's: partials stored as agent-scope relaxed
// atomics (past this XCD's L2 to the memory every XCD sees), the stores
// waited for before the arrival count, the last arriver reading them back
// the same way and resetting the head's counter to zero for the next launch
// -- no second kernel, no fence that writes back the L2.
// One query row: the decode step (causal, position read on the device) or
// a single row over a key count known at launch, which is also how a row
// attends more keys than the one-workgroup kernels' LDS score row holds
// (ATT_MAX_J).  Rows are read at min(j, kv_rows - 1), inside the allocation.
// CH keys per chunk: AS_CH, or 2 * AS_CH for rows of AS_XCH_ROWS + 1 ..
// AS_NT_ROWS keys (fewer, longer chunks, combined by the second kernel).
// Measured on MI355X, one row over 2048 keys at head dim 64 (32 / 4 heads),
// per call: 128-key chunks 8.5 us, 256 7.55 us, 512 8.7 us (all with the
// combine kernel; the in-kernel exchange at 8 chunks of 256: 8.2 us).
// Not for shorter rows: Phi-2 decode (head dim 80, 513..776 cache rows) ran
// 819 (exchange) / 809 (combine kernel) tok/s in 256-key chunks against 855.5
// in 128-key chunks with the exchange.
constexpr int AS_CH = 128;
// NT threads per chunk workgroup: NT / 8 key groups of 8 lanes, each
// holding CH / (NT / 8) of the chunk's K / V rows.  512 threads up to 2048
// cache rows, 256 beyond (measured on MI355X with the earlier three-launch
// split: 512 threads faster at up to 2048 keys, slower at 8192; with
// 256-key chunks at 2048 keys, 1024 threads 7.7 us and 256 threads 8.3 us
// against 7.55 us for 512).
constexpr int AS_NT_ROWS = 2048;
template <int NT, int CH>
struct As {
    static constexpr int NG = NT / 8, U = CH / NG, NWV = NT / 64;
    static_assert(U >= 1 && CH % NG == 0, "chunk rows per key group");
};
// key chunks of one head at the longest row any entry point attends (65,536
// keys), at the shorter chunk length (the scratch bound for both)
constexpr int AS_MAX_CH = kAttnMaxKeys / AS_CH;

struct SplitBufs {
    float* mx;     // [H][nch] chunk maxima (-inf: no finite score)
    float* sum;    // [H][nch] chunk sums of exp(s - chunk max)
    float* o;      // [H][nch][D] P.V partials
    uint32_t* flags;   // [H] arrival counters, zero between launches
    int nch;
    int keys;      // keys attended when no device position is given
};

__device__ __forceinline__ int asplit_keys(const AttnArgs& a, const SplitBufs& b) {
    return a.d_pos ? min(*a.d_pos + 1, a.kv_rows) : b.keys;
}

__device__ __forceinline__ void st_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Dim tid of one head's result from its nc chunk partials (m_c, S_c, o_c),
// summed in chunk order. Every chunk's three loads are in flight at once,
// AS_B chunks at a time (indices clamped, loads unconditional); up to AS_B
// chunks that is one round trip in all. The loads are agent-scope relaxed
// atomics in both callers: the last arriver needs them (the partials were
// published by other workgroups of the same launch, past this XCD's L2), and
// for the combine kernel they keep the compiler from turning the
// uniform-address m_c / S_c loads into scalar loads sunk into the per-chunk
// branches, one round trip per chunk.
__device__ __forceinline__ float asplit_combine(const float* pm, const float* ps, const float* po, int D, int nc, int J) {
    constexpr int AS_B = 16;
    float M = -INFINITY, num = 0.0f, den = 0.0f;
    if (nc <= AS_B) {
        float mv[AS_B], sv2[AS_B], ov[AS_B];
#pragma unroll
        for (int u = 0; u < AS_B; u++) {
            const int kk = min(u, nc - 1);
            mv[u] = ld_agent(pm + kk);
            sv2[u] = ld_agent(ps + kk);
            ov[u] = ld_agent(po + (size_t)kk * D);
        }
#pragma unroll
        for (int u = 0; u < AS_B; u++)
            if (u < nc) M = fmaxf(M, mv[u]);
        const bool degenerate = !isfinite(M);
#pragma unroll
        for (int u = 0; u < AS_B; u++) {
            if (u < nc) {
                if (degenerate) {
                    num += ov[u];
                } else if (isfinite(mv[u])) {
                    const float w = expf(mv[u] - M);
                    num += w * ov[u];
                    den += w * sv2[u];
                }
            }
        }
    } else {
        for (int k = 0; k < nc; k += AS_B) {
            float mv[AS_B];
#pragma unroll
            for (int u = 0; u < AS_B; u++) mv[u] = ld_agent(pm + min(k + u, nc - 1));
#pragma unroll
            for (int u = 0; u < AS_B; u++) M = fmaxf(M, mv[u]);   // (clamped repeats change nothing)
        }
        const bool degenerate = !isfinite(M);
        for (int k = 0; k < nc; k += AS_B) {
            float mv[AS_B], sv2[AS_B], ov[AS_B];
#pragma unroll
            for (int u = 0; u < AS_B; u++) {
                const int kk = min(k + u, nc - 1);
                mv[u] = ld_agent(pm + kk);
                sv2[u] = ld_agent(ps + kk);
                ov[u] = ld_agent(po + (size_t)kk * D);
            }
#pragma unroll
            for (int u = 0; u < AS_B; u++) {
                if (k + u < nc) {
                    if (degenerate) {
                        num += ov[u];
                    } else if (isfinite(mv[u])) {
                        const float w = expf(mv[u] - M);
                        num += w * ov[u];
                        den += w * sv2[u];
                    }
                }
            }
        }
    }
    return !isfinite(M) ? h2f(f2h(1.0f / (float)J)) * num : num / den;
}

// The body takes the workgroup's place (bx = chunk slot, by = head slot,
// gx = chunk slots per head), so that a launch of another kernel can run it
// on some of its workgroups (NT threads each).
template <int D, int NT, bool XCH, int CH>
__device__ __forceinline__ void asplit_body(const AttnArgs& a, const SplitBufs& b, int bx, int by, int gx) {
    constexpr int EPL = D / 8, NW = EPL / 2, NWV = As<NT, CH>::NWV, AS_NG = As<NT, CH>::NG, AS_U = As<NT, CH>::U;
    __shared__ float red[2][NWV];
    __shared__ float part[NWV][D];
    __shared__ int last;
    // Workgroup i runs on XCD i % 8.  With GQA the default order (chunk
    // fastest) gives each XCD the same chunk of every head, so a KV head's
    // rows are read by one XCD per chunk.  Without GQA (H == Hkv) heads share
    // nothing but the cache lines at their row boundaries (Phi-2: 160-byte
    // head rows), so each XCD takes H/8 consecutive heads, all chunks, and
    // its L2 fetches a shared line once.
    int ch = bx, h = by;
    if (a.H == a.Hkv && (a.H & 7) == 0) {
        const int id = bx + gx * by, q = id >> 3;
        h = (id & 7) * (a.H >> 3) + q / gx;
        ch = q % gx;
    }
    const int tid = threadIdx.x, c = tid & 7, g = tid >> 3;
    const int kvh = h / (a.H / a.Hkv);
    const size_t wstride = (size_t)a.Hkv * D / 2;
    const uint32_t* kbase = (const uint32_t*)(a.k + (size_t)kvh * D + EPL * c);
    const uint32_t* vbase = (const uint32_t*)(a.v + (size_t)kvh * D + EPL * c);
    const int j0 = ch * CH;
    // every K and V row of the chunk in flight before anything waits
    uint32_t kw[AS_U][NW], vw[AS_U][NW];
#pragma unroll
    for (int u = 0; u < AS_U; u++) load_row_words<NW>(kbase + (size_t)min(j0 + g + AS_NG * u, a.kv_rows - 1) * wstride, kw[u]);
#pragma unroll
    for (int u = 0; u < AS_U; u++) load_row_words<NW>(vbase + (size_t)min(j0 + g + AS_NG * u, a.kv_rows - 1) * wstride, vw[u]);
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
    const int J = asplit_keys(a, b);
    const int nc = (J + CH - 1) / CH;
    if (ch >= nc) return;   // (uniform: chunk past the keys; it is not counted)
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
        sv[u] = -INFINITY;
        if (j0 + g + AS_NG * u < J) {
            const float v = h2f(f2h(h2f(f2h(acc)) * a.scale_h));
            sv[u] = isfinite(v) ? v : NAN;   // NaN: a key that takes no weight
            if (isfinite(v)) mx = fmaxf(mx, v);
        }
    }
    mx = block_max1<NWV>(mx, red[0]);
    const bool fin = isfinite(mx);
    // p_j and the partial P.V sums; the 8 lanes of a key hold the same p_j,
    // lane c = 0 counts it into the chunk sum
    float o[EPL], se = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = 0.0f;
#pragma unroll
    for (int u = 0; u < AS_U; u++) {
        if (j0 + g + AS_NG * u < J) {
            const float pj = fin ? (isfinite(sv[u]) ? expf(sv[u] - mx) : 0.0f) : 1.0f;
            if (c == 0) se += pj;
#pragma unroll
            for (int t = 0; t < NW; t++) {
                const h2 v2 = as_h2(vw[u][t]);
                o[2 * t] += pj * (float)v2[0];
                o[2 * t + 1] += pj * (float)v2[1];
            }
        }
    }
    // the 8 key groups of each wave (lanes with the same c), then the waves,
    // in a fixed order; the chunk sum rides along (one barrier for both)
#pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = stride8_sum(o[e]);
    se = wave_sum<64>(se);
    if ((tid & 63) < 8)
#pragma unroll
        for (int e = 0; e < EPL; e++) part[tid >> 6][EPL * c + e] = o[e];
    if ((tid & 63) == 0) red[1][tid >> 6] = se;
    lds_barrier();
    const size_t hc = (size_t)h * b.nch;
    if (tid < D) {
        float t = part[0][tid];
#pragma unroll
        for (int wv = 1; wv < NWV; wv++) t += part[wv][tid];
        if (XCH) st_agent(b.o + (hc + ch) * D + tid, t);
        else b.o[(hc + ch) * D + tid] = t;
    }
    if (tid == 0) {
        float ssum = red[1][0];
#pragma unroll
        for (int wv = 1; wv < NWV; wv++) ssum += red[1][wv];
        if (XCH) {
            st_agent(b.mx + hc + ch, fin ? mx : -INFINITY);
            st_agent(b.sum + hc + ch, ssum);
        } else {
            b.mx[hc + ch] = fin ? mx : -INFINITY;
            b.sum[hc + ch] = ssum;
        }
    }
    if constexpr (!XCH) return;
    // publish, then count in; the last chunk of the head to arrive combines
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(b.flags + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(nc - 1);
    __syncthreads();
    if (!last) return;
    if (tid == 0) __hip_atomic_store(b.flags + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid >= D) return;
    const float r = asplit_combine(b.mx + hc, b.sum + hc, b.o + hc * D + tid, D, nc, J);
    a.out[(size_t)h * D + tid] = f2h(r);   // (one query row)
}

template <int D, int NT, bool XCH, int CH>
__global__ __launch_bounds__(NT) void asplit_kernel(AttnArgs a, SplitBufs b) {
    asplit_body<D, NT, XCH, CH>(a, b, (int)blockIdx.x, (int)blockIdx.y, (int)gridDim.x);
}

// The chunks of a head combined by a kernel of its own (the kernel boundary
// orders the partials' stores before these loads): one workgroup per head,
// thread d sums dim d over the chunks in chunk order.
template <int D, int CH>
__global__ __launch_bounds__(D) void asplit_combine_kernel(AttnArgs a, SplitBufs b) {
    const int h = blockIdx.x, tid = threadIdx.x;
    const int J = asplit_keys(a, b);
    const int nc = (J + CH - 1) / CH;
    const size_t hc = (size_t)h * b.nch;
    const float r = asplit_combine(b.mx + hc, b.sum + hc, b.o + hc * D + tid, D, nc, J);
    a.out[(size_t)h * D + tid] = f2h(r);   // (one query row)
}

// Decode: head dims 80 / 128 from caches of more than 512 rows (one
// workgroup per head streams too few bytes per CU there); head dim 64 only
// past the one-workgroup kernel's score row.
bool attention_split_ok(const AttnArgs& a) {
    if (!(a.d_pos && a.S == 1 && a.causal && a.Hkv > 0 && a.H % a.Hkv == 0)) return false;
    return ((a.D == 80 || a.D == 128) && a.kv_rows > 512) || (a.D == 64 && a.kv_rows > ATT_MAX_J);
}

// One row over J keys known at launch.
bool attention_split_j_ok(const AttnArgs& a, int J) {
    return !a.d_pos && a.S == 1 && J >= 1 && (a.D == 64 || a.D == 80 || a.D == 128) && a.Hkv > 0 &&
           a.H % a.Hkv == 0 && (!a.causal || a.q_pos0 < J);
}

size_t attention_split_scratch(int H, int kv_rows, int D) {
    const size_t nch = (size_t)(kv_rows + AS_CH - 1) / AS_CH;
    return (2 * (size_t)H * nch + (size_t)H * nch * D) * sizeof(float);
}

template <int D, int NT, int CH>
static void launch_split_d(hipStream_t s, const AttnArgs& a, const SplitBufs& b, dim3 grid, bool xch) {
    if constexpr (CH == AS_CH) {
        if (xch) {
            hipLaunchKernelGGL((asplit_kernel<D, NT, true, CH>), grid, dim3(NT), 0, s, a, b);
            return;
        }
    }
    hipLaunchKernelGGL((asplit_kernel<D, NT, false, CH>), grid, dim3(NT), 0, s, a, b);
    hipLaunchKernelGGL((asplit_combine_kernel<D, CH>), dim3((unsigned)a.H), dim3(D), 0, s, a, b);
}
template <int NT, int CH>
static void launch_split_kernel(hipStream_t s, const AttnArgs& a, const SplitBufs& b, dim3 grid, bool xch) {
    if (a.D == 64) launch_split_d<64, NT, CH>(s, a, b, grid, xch);
    else if (a.D == 80) launch_split_d<80, NT, CH>(s, a, b, grid, xch);
    else launch_split_d<128, NT, CH>(s, a, b, grid, xch);
}
// The in-kernel exchange up to AS_XCH_CHUNKS chunks per head, the combine
// kernel beyond: each agent-scope round trip of the exchange (store ack,
// arrival count, the last arriver's loads) costs 1-2 us on MI355X, and the
// more chunks a head has, the later its last one arrives.  Measured on one
// box: Phi-2 decode (7 chunks at 776 cache rows) 800.5 tok/s with the
// exchange vs 774.3 with the combine kernel; one row over 2048 keys at head
// dim 64 in 16 chunks of 128 keys, 10.8 vs 8.4 us per call.
constexpr int AS_XCH_CHUNKS = 8;
constexpr int AS_XCH_ROWS = AS_XCH_CHUNKS * AS_CH;

static tlhip_status launch_split(hipStream_t s, const AttnArgs& a, SplitBufs b, float* scratch) {
    if (!a.head_flags || a.H > ATTN_SPLIT_MAX_HEADS)
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "attention: key-chunked path needs the context's counters and H <= %d",
                    ATTN_SPLIT_MAX_HEADS);
    const bool wide = a.kv_rows > AS_XCH_ROWS && a.kv_rows <= AS_NT_ROWS;   // 2 * AS_CH-key chunks
    const int ch = wide ? 2 * AS_CH : AS_CH;
    b.nch = (a.kv_rows + ch - 1) / ch;
    if (b.nch > AS_MAX_CH) return fail(TLHIP_ERR_INVALID_DIMENSION, "attention: %d key chunks > %d", b.nch, AS_MAX_CH);
    b.mx = scratch;
    b.sum = b.mx + (size_t)a.H * b.nch;
    b.o = b.sum + (size_t)a.H * b.nch;
    b.flags = a.head_flags;
    const dim3 grid((unsigned)b.nch, (unsigned)a.H);
    const bool xch = !wide && b.nch <= AS_XCH_CHUNKS;
    if (wide) launch_split_kernel<512, 2 * AS_CH>(s, a, b, grid, false);
    else if (a.kv_rows <= AS_NT_ROWS) launch_split_kernel<512, AS_CH>(s, a, b, grid, xch);
    else launch_split_kernel<256, AS_CH>(s, a, b, grid, xch);
    return TLHIP_OK;
}

tlhip_status launch_attention_split(hipStream_t s, const AttnArgs& a, float* scratch) {
    if (!attention_split_ok(a) || !scratch)
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "attention: split decode path needs a device position, S = 1, D 64/80/128");
    SplitBufs b = {};
    return launch_split(s, a, b, scratch);
}

// Phi-2 decode: the key-chunked attention (in-kernel exchange) and fc1 in
// one launch.  fc1 reads only the normalised row the QKV launch wrote, so
// the two are independent, and in one grid the attention's chunk
// workgroups -- waiting on their K / V rows and on each other's partials --
// and fc1's weight-streaming workgroups share the device instead of running
// one after the other.  Workgroups [0, nA) are the attention's (chunk slot
// id % nch, head slot id / nch, the order of its own launch, so the same
// XCD placement), the rest fc1's row blocks (8 waves x 4 rows of the flat
// K = 2560 layout).  Same arithmetic as the two launches, so the same bits.
template <int D, int CH, int WT, int NB, int RI, int FN>
__global__ __launch_bounds__(512) void asplit_fc1_kernel(AttnArgs a, SplitBufs b, Gemv1Params p, int nA) {
    const int id = (int)blockIdx.x;
    if (id < nA) asplit_body<D, 512, true, CH>(a, b, id % b.nch, id / b.nch, b.nch);
    else gemv_m1_body<WT, NB, RI, EPI_BIAS_GELU, FN, 8>(p, id - nA);
}

bool launch_attention_split_fc1(hipStream_t s, const AttnArgs& a, float* scratch, tlhip_dtype wt, const GemvArgs& f) {
    if (!attention_split_ok(a) || !scratch || !a.head_flags || a.H > ATTN_SPLIT_MAX_HEADS) return false;
    // the shapes of Phi-2's decode step: head dim 80 over at most
    // AS_XCH_ROWS cache rows (128-key chunks, in-kernel exchange), fc1 a
    // Q8_0 [N >= 8192, 2560] GEMV + bias + GELU on one row
    if (a.D != 80 || a.kv_rows > AS_XCH_ROWS || wt != TLHIP_Q8_0 || f.M != 1 || f.K != 80 * 32 || f.N < 8192 ||
        !f.bias || !f.x || !f.y)
        return false;
    SplitBufs b = {};
    b.nch = (a.kv_rows + AS_CH - 1) / AS_CH;
    b.mx = scratch;
    b.sum = b.mx + (size_t)a.H * b.nch;
    b.o = b.sum + (size_t)a.H * b.nch;
    b.flags = a.head_flags;
    const Gemv1Params p = {f.x, (const uint8_t*)f.wq, f.wd, f.bias, nullptr, f.y, f.N, f.K, EPI_BIAS_GELU};
    const int nA = b.nch * a.H, nF = (f.N + 31) / 32;   // 8 waves x 4 rows per fc1 workgroup
    hipLaunchKernelGGL((asplit_fc1_kernel<80, AS_CH, TLHIP_Q8_0, 2, 4, 80>), dim3((unsigned)(nA + nF)), dim3(512), 0, s,
                       a, b, p, nA);
    return true;
}

// One row over J keys; scratch holds attention_split_scratch(H, J, D) bytes.
tlhip_status launch_attention_split_j(hipStream_t s, const AttnArgs& a, int J, float* scratch) {
    if (!attention_split_j_ok(a, J) || !scratch)
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "attention: split path needs one query row and D 64/80/128");
    AttnArgs r = a;
    r.kv_rows = J;   // rows in k / v
    SplitBufs b = {};
    b.keys = a.causal ? min(J, a.q_pos0 + 1) : J;
    return launch_split(s, r, b, scratch);
}

// ---------------------------------------------------------------------------
// Prefill attention on the matrix cores (S >= 128 query rows, head_dim 64,
// 80 or 128).  The scores keep the reference's rounding points -- f16 dot
// product, f16 product with the f16 scale, masked and non-finite keys
// excluded -- and so do the exponentials, e = f16(exp(s - max)) with the sum
// taken over the unrounded values; the one departure is that P . V is
// accumulated from the f16 e (fp32) and divided by the sum once per output,
// where the reference rounds each P = f16(e / sum) to f16 first (within one
// f16 rounding per term; the layer bars are max-abs 2e-2 and rel-L2 1e-3).
// The contractions run as v_mfma_f32_32x32x16_f16:
//   S^T[key][query] = K . Q^T  (A = 32 keys x 16 dims from K rows, B = 32
//                              queries x 16 dims from Q rows)
//   O[query][d]     = E . V    (A = f16 e straight from S^T's accumulator
//                              layout, B = 16-byte runs of the V^T tiles)
// In S^T's accumulator layout lane l owns query l%32 and keys
// 8(r/4) + 4(l/32) + r%4 (r = 0..15): the row statistics are per lane plus
// one exchange with lane l^32, and registers 8t..8t+7 are exactly the
// A operand of k-step t under the key order 16t + 8(i/4) + 4(l/32) + i%4,
// which the V^T tiles are stored in.
// Pass 1 over the key tiles finds the row max on packed f16 scores; pass 2
// recomputes the scores and accumulates the sum and E . V.  Two waves own
// one head and a 32-row query tile (causal: the pair of tiles t and n-1-t,
// so every workgroup does the same work), each taking half of the key
// tiles; their maxima meet in LDS after pass 1, their sums and the upper
// half's partial O after pass 2.  A workgroup holds four heads (two for
// head_dim 128).  When they share one KV head (GQA groups of a multiple of
// that many heads) the staged kernel copies each 32-key tile of K and V^T
// to LDS once, with DMA loads of whole 1 KiB pieces, and all heads read it
// there; otherwise every wave reads its operands from global memory, where
// each load instruction touches 32 cache lines (the L1 tag rate, not the
// matrix or vector units, then bounds the kernel).
// ---------------------------------------------------------------------------

// V [J, Hkv, D] -> V^T in 32-key tiles [Hkv][Jp/32][4][D][8], zero for
// keys J..Jp-1 (Jp % 32 == 0).  A tile holds row d's 32 keys as four
// 16-byte chunks in the order the E . V operand reads them: chunk
// c = 2t + hh holds keys 16t + 8(i/4) + 4hh + i%4 (i = 0..7), and chunk c
// of every row comes before chunk c + 1, so the 32 lanes reading one chunk
// of 32 rows read 512 contiguous bytes.  A tile is one contiguous
// 64 D-byte block, copied to LDS unchanged.
__global__ __launch_bounds__(256) void vt_transpose_kernel(const uint16_t* __restrict__ v, uint16_t* __restrict__ vt,
                                                         int J, int Jp, int Hkv, int D) {
    __shared__ __attribute__((aligned(16))) uint16_t tile[32 * 128];   // [key][D] of this tile
    const int j0 = blockIdx.x * 32, kvh = blockIdx.y, nc = 4 * D;   // 16-byte units per tile
    const size_t kstride = (size_t)Hkv * D;
    for (int i = threadIdx.x; i < nc; i += 256) {   // 16 bytes of key i / (D/8)
        const int key = i / (D / 8), c = i % (D / 8), j = j0 + key;
        u4 w = {0u, 0u, 0u, 0u};
        if (j < J) w = *(const u4*)(v + (size_t)j * kstride + (size_t)kvh * D + 8 * c);
        *(u4*)(tile + key * D + 8 * c) = w;
    }
    __syncthreads();
    uint16_t* const out = vt + ((size_t)kvh * (Jp / 32) + blockIdx.x) * (size_t)D * 32;
    for (int i = threadIdx.x; i < nc; i += 256) {   // chunk c of row d
        const int c = i / D, d = i % D;
        uint16_t e8[8];
#pragma unroll
        for (int e = 0; e < 8; e++) e8[e] = tile[(16 * (c >> 1) + 8 * (e >> 2) + 4 * (c & 1) + (e & 3)) * D + d];
        u4 w;
#pragma unroll
        for (int q = 0; q < 4; q++) w[q] = (uint32_t)e8[2 * q] | ((uint32_t)e8[2 * q + 1] << 16);
        *(u4*)(out + (size_t)i * 8) = w;
    }
}

// Byte offset, inside a V^T tile, of the 16 bytes lane l reads as the
// E . V operand of output tile n (column d, clamped to D-1: columns past D
// are not stored) and k-step t.
template <int D>
__device__ __forceinline__ int fa_vt_off(int lane, int n, int t) {
    const int d = D % 32 == 0 ? 32 * n + (lane & 31) : min(32 * n + (lane & 31), D - 1);
    return 16 * ((2 * t + (lane >> 5)) * D + d);
}

// Scores of one 32-key tile (jb = first key of this lane's runs) for this
// lane's query as the reference stores them (f16 dot product, then the f16
// product with the f16 scale), as eight f16 pairs; excluded keys (masked,
// non-finite) come back as -inf.  Non-finite scores are found with packed
// f16 arithmetic: x - x is 0 for a finite x and NaN otherwise, x + (x - x)
// keeps x or turns it into NaN, and the IEEE max with -inf maps NaN to -inf.
// FULL: every key of the tile is unmasked for every query of the wave.
// !SAFE: the row is known to hold no +inf score (its largest score is
// finite), so only NaN needs mapping to -inf, and -inf stays.
// fa_round: the f16 dot products; fa_scale: the scores from them, in place.
__device__ __forceinline__ void fa_round(const f16v& acc, h2 (&s2)[8]) {
#pragma unroll
    for (int r = 0; r < 16; r += 2) s2[r >> 1] = h2{(h16)acc[r], (h16)acc[r + 1]};
}
template <bool FULL, bool SAFE = true>
__device__ __forceinline__ void fa_scale(h2 (&s2)[8], int jb, int jlim, float scale_h) {
    const h2 sc2 = {(h16)scale_h, (h16)scale_h};
    const h2 ninf = {(h16)-INFINITY, (h16)-INFINITY};
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
        h2 x = s2[r >> 1] * sc2;
        x = __builtin_elementwise_max(SAFE ? x + (x - x) : x, ninf);
        if (!FULL) {
            if (jb + 8 * (r >> 2) + (r & 3) > jlim) x[0] = (h16)-INFINITY;
            if (jb + 8 * ((r + 1) >> 2) + ((r + 1) & 3) > jlim) x[1] = (h16)-INFINITY;
        }
        s2[r >> 1] = x;
    }
}
template <bool FULL, bool SAFE = true>
__device__ __forceinline__ void fa_scores(const f16v& acc, int jb, int jlim, float scale_h, h2 (&s2)[8]) {
    fa_round(acc, s2);
    fa_scale<FULL, SAFE>(s2, jb, jlim, scale_h);
}

// Pass-2 work of one tile: e = f16(exp(s - m)) as the reference stores it
// (pa, the A operand of E . V) and the fp32 sum of the unrounded
// exponentials; the product of the f16 e with V is divided by the sum at
// the end.  DEG: rows with no finite score (deg) weight every key < J by
// f16(1/J) = uni and keep a sum of 1, as the reference's softmax does.
template <bool DEG>
__device__ __forceinline__ void fa_exp(const h2 (&s2)[8], float m, bool deg, float uni, int jb, int J, h8 (&pa)[2],
                                       float& sum) {
    constexpr float L1 = 1.44269502162933349609375f;   // log2(e)
    // x = s - m in f32 (v_fma_mix_f32 of the f16 s: s * 1 - m, one
    // rounding, as the f32 subtraction); e = 2^(x log2 e) on v_exp_f32,
    // within a few f32 ulps of exp(x) before its f16 rounding; excluded keys
    // (-inf) give exactly 0
    const float nm = -m;
    float e[16];
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
        float x0, x1;
        asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(x0) : "v"(s2[r >> 1]), "v"(nm));
        asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(x1) : "v"(s2[r >> 1]), "v"(nm));
        e[r] = __builtin_amdgcn_exp2f(x0 * L1);
        e[r + 1] = __builtin_amdgcn_exp2f(x1 * L1);
    }
#pragma unroll
    for (int r = 0; r < 16; r++) pa[r >> 3][r & 7] = (h16)e[r];
    // pairwise, so the adds are not one dependent chain
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
        for (int r = 0; r < w; r++) e[r] += e[r + w];
    sum += e[0];
    if (DEG && deg) {
#pragma unroll
        for (int r = 0; r < 16; r++) pa[r >> 3][r & 7] = (h16)(jb + 8 * (r >> 2) + (r & 3) < J ? uni : 0.0f);
    }
}

template <int NT>
__device__ __forceinline__ void fa_pv(const h8 (&pa)[2], const h8 (&vb)[NT][2], f16v (&o)[NT]) {
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int n = 0; n < NT; n++) o[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa[t], vb[n][t], o[n], 0, 0, 0);
}

// pass kinds of the staged kernel
enum { FA_MAX = 0, FA_MAX_EXACT = 1, FA_PV = 2, FA_PV_SAFE = 3, FA_PV_DEG = 4 };

// After pass 2: the row's sum over both lane halves and both key halves in
// a fixed order, the upper half's partial O through LDS (ob: [NT][16][64]),
// and the lower half stores (o + ob) / sum; a degenerate row (no finite
// score in either half's max, stm) divides by 1.  One workgroup barrier,
// reached by every wave.
// Whether p holds for any lane of the workgroup's nw waves: one word per
// wave in slot (LDS), one lds_barrier.  The caller writes the slot again
// only after later barriers.
__device__ __forceinline__ bool wg_any(bool p, int* slot, int nw) {
    const bool wp = __any(p);
    if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = wp;
    lds_barrier();
    int r = 0;
    for (int i = 0; i < nw; i++) r |= slot[i];
    return r != 0;
}

// Row stride (elements) of the f16 output tile staged in LDS by fa_finish.
template <int D>
constexpr int fa_ot_stride() { return D + 8; }

// After pass 2: the row's sum over both lane halves and both key halves in
// a fixed order, the upper half's partial O through LDS (ob: [NT][16][64]),
// and the lower half's f16 (o + ob) / sum, a degenerate row (no finite
// score in either half's max, stm) divided by 1.  The lower half stages
// the tile in ot ([32][fa_ot_stride] f16, LDS) and stores it in 16-byte
// pieces, rows past S left out.  One workgroup barrier, reached by every
// wave.
template <int D>
__device__ __forceinline__ void fa_finish(const AttnArgs& a, int h, int s0, int half, bool store, int os,
                                          const f16v (&o)[(D + 31) / 32], float sum, const float* stm, float* sts,
                                          float* ob, uint16_t* ot) {
    constexpr int NT = (D + 31) / 32, DP = fa_ot_stride<D>();
    // the lane index through an opaque copy: the addresses below are then
    // computed here, not hoisted out of the caller's loops to stay live
    // through them
    int lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));
    const float s1 = sum + __shfl_xor(sum, 32, 64);
    if (lane < 32) sts[half * 32 + lane] = s1;
    if (half) {
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int r = 0; r < 16; r++) ob[(n * 16 + r) * 64 + lane] = o[n][r];
    }
    lds_barrier();
    if (!half) {
        // row q's scale into sts[q] (lane q): a row's sum is at least 1 (its
        // largest score's e), so the f32 reciprocal (v_rcp_f32, 1 ulp) does
        if (lane < 32) {
            const float tot = sts[lane] + sts[32 + lane];
            sts[lane] = fmaxf(stm[lane], stm[32 + lane]) > -INFINITY ? __builtin_amdgcn_rcpf(tot) : 1.0f;
        }
        // O accumulators: column d = 32n + l%32, rows 8(r/4) + 4(l/32) + r%4
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const int d = 32 * n + (lane & 31);
            if (D % 32 == 0 || d < D) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int q = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    ot[q * DP + d] = f2h((o[n][r] + ob[(n * 16 + r) * 64 + lane]) * sts[q]);
                }
            }
        }
        if (store) {
            // the wave's own LDS writes complete before its reads (the
            // compiler waits for them)
            uint16_t* const ob0 = a.out + (size_t)s0 * os + (size_t)h * D;
#pragma unroll
            for (int i = 0; i < (4 * D + 63) / 64; i++) {
                const int c = lane + 64 * i, row = c / (D / 8), c8 = c % (D / 8);
                if (c < 4 * D && s0 + row < a.S)
                    *(u4*)(ob0 + (size_t)row * os + 8 * c8) = *(const u4*)(ot + row * DP + 8 * c8);
            }
        }
    }
}

// The key-tile ranges of one query tile and this lane's query.
struct FaTile {
    int s0, myq, nkt, jlim, nfull, nh;
    __device__ FaTile(const AttnArgs& a, int J, int qt) {
        const int lane = threadIdx.x & 63;
        s0 = qt * 32;
        myq = s0 + (lane & 31);
        const int last = min(s0 + 31, a.S - 1);
        const int kend = a.causal ? min(J, a.q_pos0 + last + 1) : J;
        nkt = (kend + 31) / 32;
        jlim = a.causal ? min(J - 1, a.q_pos0 + myq) : J - 1;
        // tiles below every query's limit need no mask test
        const int lo_lim = a.causal ? min(J - 1, a.q_pos0 + s0) : J - 1;
        nfull = (lo_lim + 1) / 32;
        nh = (nkt + 1) / 2;
    }
};

// Heads per workgroup (each head = two waves, one per key half).
template <int D>
constexpr int fa_heads() { return D > 80 ? 2 : 4; }

// -- operands from global memory (any head grouping) -----------------------
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

    // V^T operands of tile kt
    __device__ __forceinline__ void load_v(int kt, h8 (&vb)[NT][2]) const {
        const uint8_t* tb = (const uint8_t*)(vt + ((size_t)kvh * (Jp / 32) + kt) * (size_t)D * 32);
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int t = 0; t < 2; t++) vb[n][t] = *(const h8*)(tb + fa_vt_off<D>(lane, n, t));
    }

    __device__ __forceinline__ f16v qk(const h8 (&qf)[KS], const h8 (&kf)[KS]) const {
        f16v acc = {};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[ks], qf[ks], acc, 0, 0, 0);
        return acc;
    }

    // pass 1 over tiles [k0, k1): the largest finite score of this lane's
    // keys (-inf if none)
    __device__ __forceinline__ float pass1(const h8 (&qf)[KS], int k0, int k1, int nfull, int jlim) const {
        const h2 ninf = {(h16)-INFINITY, (h16)-INFINITY};
        h2 m2 = ninf;
        if (k0 >= k1) return -INFINITY;
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
            h2 s2[8];
            const int jb = kt * 32 + 4 * (lane >> 5);
            if (kt < nfull) fa_scores<true>(acc, jb, jlim, a.scale_h, s2);
            else fa_scores<false>(acc, jb, jlim, a.scale_h, s2);
            acc = accn;
#pragma unroll
            for (int r = 0; r < 8; r++) m2 = __builtin_elementwise_max(m2, s2[r]);
        }
        return fmaxf((float)m2[0], (float)m2[1]);
    }

    // pass 2 over tiles [k0, k1)
    template <bool DEG>
    __device__ __forceinline__ void pass2(const h8 (&qf)[KS], int k0, int k1, int nfull, int jlim, float m,
                                          bool deg, f16v (&o)[NT], float& sum) const {
        if (k0 >= k1) return;
        const float uni = h2f(f2h(1.0f / (float)J));
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
            h2 s2[8];
            const int jb = kt * 32 + 4 * (lane >> 5);
            if (kt < nfull) fa_scores<true>(acc, jb, jlim, a.scale_h, s2);
            else fa_scores<false>(acc, jb, jlim, a.scale_h, s2);
            acc = accn;
            h8 pa[2];
            fa_exp<DEG>(s2, m, deg, uni, jb, J, pa, sum);
            fa_pv<NT>(pa, vb, o);
        }
    }

    // Query tile qt, key half `half` of its tiles.  stm/sts: this head's
    // [2][32] exchange of row statistics; ob: [NT][16][64] partial O of the
    // upper half.  Two workgroup barriers, reached by every wave.
    __device__ __forceinline__ void run(int qt, int half, bool store, float* stm, float* sts, float* ob,
                                        uint16_t* ot) const {
        const FaTile tl(a, J, qt);
        h8 qf[KS];
        {
            const uint16_t* qr = a.q + (size_t)min(tl.myq, a.S - 1) * qs + (size_t)h * D + 8 * (lane >> 5);
#pragma unroll
            for (int ks = 0; ks < KS; ks++) qf[ks] = *(const h8*)(qr + 16 * ks);
        }

        // the row max: this lane's keys, the other 16 keys of every tile in
        // lane l ^ 32, the other key half in the partner wave
        const float mx = pass1(qf, half ? tl.nh : 0, half ? tl.nkt : tl.nh, tl.nfull, tl.jlim);
        const float m1 = fmaxf(mx, __shfl_xor(mx, 32, 64));
        if (lane < 32) stm[half * 32 + lane] = m1;
        lds_barrier();
        const float m = fmaxf(m1, stm[(half ^ 1) * 32 + (lane & 31)]);
        const bool deg = !(m > -INFINITY) && tl.myq < a.S;   // no finite score in the row

        f16v o[NT];
#pragma unroll
        for (int n = 0; n < NT; n++) o[n] = f16v{};
        float sum = 0.0f;
        if (__any(deg)) {
            const int nk = Jp / 32, nhd = (nk + 1) / 2;
            pass2<true>(qf, half ? nhd : 0, half ? nk : nhd, 0, tl.jlim, deg ? 0.0f : m, deg, o, sum);
        } else {
            pass2<false>(qf, half ? tl.nh : 0, half ? tl.nkt : tl.nh, tl.nfull, tl.jlim, m, false, o, sum);
        }
        fa_finish<D>(a, h, tl.s0, half, store, os, o, sum, stm, sts, ob, ot);
    }
};

// HPW heads per workgroup (two waves each); the heads share no operands
// here, so HPW only sets the launch granularity.
template <int D, int HPW = fa_heads<D>()>
__global__ __launch_bounds__(HPW * 128) void attention_mfma_kernel(AttnArgs a, const uint16_t* __restrict__ vt, int J,
                                                             int Jp, int nqt) {
    constexpr int NT = (D + 31) / 32;
    __shared__ float stm[HPW][64], sts[HPW][64];
    __shared__ float ob[HPW][NT * 16 * 64];
    __shared__ __attribute__((aligned(16))) uint16_t ot[HPW][32 * fa_ot_stride<D>()];
    const int w = threadIdx.x >> 6, hw = w % HPW, half = w / HPW;
    const int hh = blockIdx.y * HPW + hw;
    const FaWave<D> fw(a, vt, J, Jp, min(hh, a.H - 1));
    const bool store = hh < a.H;
    // causal: tiles n-1-x and x (one call site, so run() is inlined)
    const int t0 = a.causal ? nqt - 1 - (int)blockIdx.x : (int)blockIdx.x, t1 = blockIdx.x;
    const int nrun = a.causal && t1 < t0 ? 2 : 1;
    for (int u = 0; u < nrun; u++) fw.run(u ? t1 : t0, half, store, stm[hw], sts[hw], ob[hw], ot[hw]);
}

// -- operands staged in LDS (every head of the workgroup on one KV head) ---
// Ring of ST stages; a stage holds one 32-key tile of K for each key half
// and, in pass 2, one of V^T (64 D bytes each).  Both halves step through
// their tiles in lock step, one workgroup barrier per step: at step i a
// wave waits for its own copies of tile i + 1, the barrier makes every
// wave's copies visible and ends every read of tile i - 1, whose slot then
// receives tile i + ST - 1 -- of the same pass or of the passes that
// follow, so that a pass starts on tiles already in LDS.  A K tile in LDS is chunk-major, [D/8][32][8]:
// 16-byte chunk c of key r at 16 (32 c + r), so a k-step's operand is 16
// contiguous bytes per lane (lane l at 16 l + 1024 ks) and every copy piece
// is two 16-byte chunks of 32 rows.
template <int D>
struct FaStaged {
    static constexpr int HPW = fa_heads<D>();
    static constexpr int KS = D / 16, NT = (D + 31) / 32;
    static constexpr int TB = 64 * D;                   // bytes of a 32-key tile of K or of V^T
    static constexpr int NQ = D / 16;                   // 1 KiB DMA pieces per tile
    static constexpr int CQ = (NQ + HPW - 1) / HPW;     // pieces per wave and tile (the rest copy nothing)
    // LEAD: steps whose copies are in place ahead of the current one (a
    // lead of 2, with tile i+1's K read from LDS a step early, measured
    // slower at head_dim 64: the copies then had one step to land, not two)
    static constexpr int LEAD = 1;
    static constexpr int ST = D > 80 ? 3 : 4;           // ring stages
    static constexpr int STAGE = 4 * TB;                // K half 0, K half 1, V^T half 0, V^T half 1
    static constexpr int RING = ST * STAGE;
    static constexpr uint32_t OOB = 0x80000000u;        // buffer offset past every range: no access, zeros
    static constexpr int G = 2 * CQ;                    // copies per wave and stage

    AttnArgs a;
    int J, Jp, h, lane, hw, half, qs, os;
    uint32_t ring_lds, kstride2, vbase;
    const uint8_t* ring;
    __amdgpu_buffer_rsrc_t rk, rv;
    uint32_t kcol[CQ];     // byte offset, in its key's row of the cache, of this lane's 16 bytes of piece hw + HPW c

    __device__ FaStaged(const AttnArgs& a_, const uint16_t* vt, int J_, int Jp_, int kvh, int h_, int hw_, int half_,
                        const uint8_t* ring_)
        : a(a_), J(J_), Jp(Jp_), h(h_), hw(hw_), half(half_), ring(ring_) {
        lane = threadIdx.x & 63;
        qs = a.q_stride ? a.q_stride : a.H * D;
        os = a.out_stride ? a.out_stride : a.H * D;
        kstride2 = (uint32_t)a.Hkv * D * 2u;
        vbase = (uint32_t)kvh * (uint32_t)(Jp / 32) * TB;
        ring_lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(gl_lds_t)ring);
        rk = sk_rsrc(a.k, (uint32_t)(J - 1) * kstride2 + (uint32_t)a.Hkv * D * 2u);
        rv = sk_rsrc(vt, (uint32_t)a.Hkv * (uint32_t)Jp * D * 2u);
        // piece q = hw + HPW c: LDS 16-byte unit 64 q + lane = chunk 2q + l/32 of key l%32
#pragma unroll
        for (int c = 0; c < CQ; c++) kcol[c] = (uint32_t)kvh * D * 2u + 16u * (2 * (hw + HPW * c) + (lane >> 5));
    }

    // this wave's pieces of tile kt (nothing if !ok; K only if !pv) into
    // ring slot sl: G copies in every case (those of nothing touch no
    // memory), so the wait counts are fixed.  Branch-free (the piece count
    // and its bounds are uniform selects).
    __device__ __forceinline__ void issue(int kt, bool ok, bool pv, int sl) const {
        const uint32_t sb = ring_lds + (uint32_t)(sl * STAGE);
#pragma unroll
        for (int c = 0; c < CQ; c++) {
            const int q = hw + HPW * c;
            const bool real = q < NQ;
            const uint32_t src = ok && real ? (uint32_t)min(kt * 32 + (lane & 31), J - 1) * kstride2 + kcol[c] : OOB;
            sk_dma<16>(rk, real ? sb + (uint32_t)(half * TB + 1024 * q) : ring_lds + RING, src);
        }
#pragma unroll
        for (int c = 0; c < CQ; c++) {
            const int q = hw + HPW * c;
            const bool real = q < NQ;
            const uint32_t src = ok && pv && real ? vbase + (uint32_t)kt * TB + 1024u * q + 16u * lane : OOB;
            sk_dma<16>(rv, real ? sb + (uint32_t)(2 * TB + half * TB + 1024 * q) : ring_lds + RING, src);
        }
    }

    __device__ __forceinline__ void read_k(int sl, h8 (&kf)[KS]) const {
        const uint8_t* kb = ring + sl * STAGE + half * TB + 16 * lane;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) kf[ks] = *(const h8*)(kb + 1024 * ks);
    }
    __device__ __forceinline__ void read_v(int sl, h8 (&vb)[NT][2]) const {
        const uint8_t* vb0 = ring + sl * STAGE + 2 * TB + half * TB;
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int t = 0; t < 2; t++) vb[n][t] = *(const h8*)(vb0 + fa_vt_off<D>(lane, n, t));
    }
    static __device__ __forceinline__ f16v qk(const h8 (&qf)[KS], const h8 (&kf)[KS]) {
        f16v acc = {};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[ks], qf[ks], acc, 0, 0, 0);
        return acc;
    }
    // the largest of mr and 16 raw accumulators (v_max3_f32: a NaN operand
    // is passed over, as IEEE maxNum does)
    static __device__ __forceinline__ float max3(float a, float b, float c) {
        float d;
        asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
        return d;
    }
    static __device__ __forceinline__ void raw_max(const f16v& acc, float& mr) {
        float m0 = max3(mr, acc[0], acc[1]), m1 = max3(acc[2], acc[3], acc[4]);
#pragma unroll
        for (int r = 5; r < 15; r += 4) {
            m0 = max3(m0, acc[r], acc[r + 1]);
            m1 = max3(m1, acc[r + 2], acc[r + 3]);
        }
        mr = max3(m0, m1, acc[15]);
    }

    // Steps i in [0, n) over this half's tiles [k0, k0 + cnt) (n >= cnt,
    // the workgroup's common count).  On entry acc holds the QK^T of tile k0
    // (if cnt > 0) and sl the ring slot of step 0; the copies of steps
    // 0 .. LEAD-1 are in place.  At step i a wave waits for its copies of
    // step i + LEAD, the barrier makes every wave's copies visible and ends
    // every read of step i - 1's slot, and ahead(that slot) issues the
    // copies of step i + ST - 1 (ahead keeps its own position).  On exit sl
    // is the slot of step n; the copies of steps n .. n+LEAD-1 are in
    // place.  MODE:
    //   FA_MAX        the largest raw accumulator (the dot product before
    //                 its f16 roundings) of the unmasked keys into mr;
    //   FA_MAX_EXACT  the largest finite f16 score into m2;
    //   FA_PV         pass 2 for rows whose largest score is finite;
    //   FA_PV_SAFE    pass 2 for any rows;
    //   FA_PV_DEG     pass 2 over every key, degenerate rows uniformly (m,
    //                 deg as in fa_exp).
    // Steps whose tile and next tile are both in range and unmasked run a
    // loop without branches, in which the matrix core takes tile i-1's
    // E . V and tile i+1's QK^T while the vector unit works on tile i.
    template <int MODE, class Ahead>
    __device__ __forceinline__ void loop(const Ahead& ahead, const h8 (&qf)[KS], int k0, int cnt, int n, int nfull,
                                         int jlim, float m, bool deg, float& mr, h2& m2, f16v (&o)[NT], float& sum,
                                         f16v& acc, int& sl) const {
        constexpr bool PV = MODE >= FA_PV, DEG = MODE == FA_PV_DEG, SAFE = MODE != FA_PV;
        const float uni = h2f(f2h(1.0f / (float)J));
        int i = 0;
        if constexpr (MODE != FA_MAX_EXACT && !DEG) {
            const int na = max(0, min(min(cnt - 1, nfull - k0), n));
            h8 pp[2] = {}, vp[NT][2] = {};   // tile i-1's E and V^T (zero before the first step)
            for (; i < na; i++) {
                const int sn = sl + 1 == ST ? 0 : sl + 1;   // tile i + 1
                const int sp = sl == 0 ? ST - 1 : sl - 1;   // tile i - 1, refilled with step i + ST - 1
                sk_wait_vm<(ST - 2 - LEAD) * G>();
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                ahead(sp);
                h8 kf[KS];
                read_k(sn, kf);
                // each register set is read before it is rewritten: the loop
                // carries them without copies
                if constexpr (PV) {
                    fa_pv<NT>(pp, vp, o);   // tile i - 1
                    __builtin_amdgcn_sched_barrier(0);
                    read_v(sl, vp);
                    h2 s2[8];
                    fa_round(acc, s2);
                    __builtin_amdgcn_sched_barrier(0);
                    acc = qk(qf, kf);       // tile i + 1
                    const int jb = (k0 + i) * 32 + 4 * (lane >> 5);
                    fa_scale<true, SAFE>(s2, jb, jlim, a.scale_h);
                    fa_exp<false>(s2, m, false, uni, jb, J, pp, sum);
                } else {
                    raw_max(acc, mr);
                    __builtin_amdgcn_sched_barrier(0);
                    acc = qk(qf, kf);
                }
                sl = sn;
            }
            if constexpr (PV) fa_pv<NT>(pp, vp, o);
        }
        for (; i < n; i++) {
            const int sn = sl + 1 == ST ? 0 : sl + 1;
            const int sp = sl == 0 ? ST - 1 : sl - 1;
            sk_wait_vm<(ST - 2 - LEAD) * G>();
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            ahead(sp);
            f16v accn = acc;
            if (i + 1 < cnt) {   // on the matrix core while the vector unit works on tile i
                h8 kf[KS];
                read_k(sn, kf);
                accn = qk(qf, kf);
            }
            if (i < cnt) {
                const int kt = k0 + i, jb = kt * 32 + 4 * (lane >> 5);
                if constexpr (MODE == FA_MAX) {
                    f16v am = acc;
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        if (jb + 8 * (r >> 2) + (r & 3) > jlim) am[r] = -INFINITY;
                    raw_max(am, mr);
                } else {
                    h2 s2[8];
                    if (kt < nfull) fa_scores<true, SAFE>(acc, jb, jlim, a.scale_h, s2);
                    else fa_scores<false, SAFE>(acc, jb, jlim, a.scale_h, s2);
                    if constexpr (PV) {
                        h8 vb[NT][2], pa[2];
                        read_v(sl, vb);
                        fa_exp<DEG>(s2, m, deg, uni, jb, J, pa, sum);
                        fa_pv<NT>(pa, vb, o);
                    } else {
#pragma unroll
                        for (int r = 0; r < 8; r++) m2 = __builtin_elementwise_max(m2, s2[r]);
                    }
                }
            }
            acc = accn;
            sl = sn;
        }
    }

    // A pass on its own (the rare exact row max and degenerate rows): after
    // every wave is done with the ring, copies of its own from slot 0, and
    // its last copies landed at the end.
    template <int MODE>
    __device__ __forceinline__ void pass(const h8 (&qf)[KS], int k0, int cnt, int n, int nfull, int jlim, float m,
                                         bool deg, float& mr, h2& m2, f16v (&o)[NT], float& sum) const {
        constexpr bool PV = MODE >= FA_PV;
        int pos = 0;
        auto ahead = [&](int s) {
            issue(k0 + pos, pos < cnt, PV, s);
            pos++;
        };
        f16v acc;
        int sl;
        start(ahead, qf, cnt, acc, sl);
        loop<MODE>(ahead, qf, k0, cnt, n, nfull, jlim, m, deg, mr, m2, o, sum, acc, sl);
        sk_wait_vm<0>();
    }

    // Fill the ring from its slot 0 with steps 0 .. ST-2 (ahead), once every
    // wave is done with it (steps 0 .. LEAD-1 in place), and the first
    // tile's QK^T (if cnt > 0).
    template <class Ahead>
    __device__ __forceinline__ void start(const Ahead& ahead, const h8 (&qf)[KS], int cnt, f16v& acc, int& sl) const {
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        sk_wait_vm<0>();
#pragma unroll
        for (int i = 0; i < ST - 1; i++) ahead(i);
        sk_wait_vm<(ST - 1 - LEAD) * G>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        sl = 0;
        acc = f16v{};
        if (cnt > 0) {
            h8 kf[KS];
            read_k(0, kf);
            acc = qk(qf, kf);
        }
    }

    // The workgroup's key tiles as one stream: job j = 2u + p is pass p
    // (0: the row max, 1: the sums and E . V) of query tile u (t0, then
    // t1), job_n steps each over the same tiles; every step copies the step
    // ST - 1 positions ahead, whichever job that is, so only the first job
    // waits for memory.
    struct Stream {
        int nh0, nkt0, nh1, nkt1, nj;   // steps and key tiles of the two query tiles; jobs (2 or 4)
    };
    __device__ __forceinline__ int job_n(const Stream& s, int j) const { return j < 2 ? s.nh0 : s.nh1; }
    __device__ __forceinline__ int job_k0(const Stream& s, int j) const { return half ? job_n(s, j) : 0; }
    __device__ __forceinline__ int job_cnt(const Stream& s, int j) const {
        return half ? (j < 2 ? s.nkt0 : s.nkt1) - job_n(s, j) : job_n(s, j);
    }
    // A position of the stream: step i of job j (past the last job: copies
    // of nothing).
    struct Cursor {
        int j, i;
    };
    // the copies at c into slot sl; c one step on (every job has a step)
    __device__ __forceinline__ void issue_next(const Stream& s, Cursor& c, int sl) const {
        const bool ok = c.j < s.nj && c.i < job_cnt(s, c.j);
        issue(ok ? job_k0(s, c.j) + c.i : 0, ok, (c.j & 1) != 0, sl);
        if (++c.i >= job_n(s, c.j)) {
            c.i = 0;
            c.j++;
        }
    }

    __device__ __forceinline__ void load_q(int myq, h8 (&qf)[KS]) const {
        const uint16_t* qr = a.q + (size_t)min(myq, a.S - 1) * qs + (size_t)h * D + 8 * (lane >> 5);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) qf[ks] = *(const h8*)(qr + 16 * ks);
    }

    // Query tiles t0 and, if nu == 2, t1; stm/sts/ob/ot as in fa_finish,
    // votes 4 HPW words.  Every wave reaches the same barriers.
    __device__ __forceinline__ void run(int t0, int t1, int nu, bool store, float* stm, float* sts, float* ob,
                                        uint16_t* ot, int* votes) const {
        const FaTile T0(a, J, t0), T1(a, J, t1);
        const Stream s{T0.nh, T0.nkt, T1.nh, T1.nkt, 2 * nu};
        // the ring's first copies, then both query tiles' rows: waiting
        // for the rows (the compiler counts only its own loads) waits for
        // the older copies too, one memory latency for both; the rows arrive
        // here, once -- a first use inside the step loops would make the
        // compiler wait there for every load outstanding
        Cursor cur{0, 0};
        auto ahead = [&](int sl_) { issue_next(s, cur, sl_); };
#pragma unroll
        for (int i = 0; i < ST - 1; i++) ahead(i);
        h8 qf[KS], qn[KS];
        load_q(T0.myq, qf);
        load_q(T1.myq, qn);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) asm volatile("" ::"v"(qf[ks]), "v"(qn[ks]));
        sk_wait_vm<0>();
        lds_barrier();
        int sl = 0;
        f16v acc = {};
        if (job_cnt(s, 0) > 0) {
            h8 kf[KS];
            read_k(0, kf);
            acc = qk(qf, kf);
        }
        for (int u = 0; u < nu; u++) {
            const FaTile& T = u ? T1 : T0;
            const int j = 2 * u, k0 = job_k0(s, j), cnt = job_cnt(s, j), n = job_n(s, j);
            f16v o[NT];
#pragma unroll
            for (int nn = 0; nn < NT; nn++) o[nn] = f16v{};
            float sum = 0.0f, mr = -INFINITY;
            h2 m2 = {(h16)-INFINITY, (h16)-INFINITY};
            // The row max from the raw accumulators: rounding to f16 and the
            // product with the positive f16 scale never reverse an order, so
            // the largest score is g(M) = f16(f16(M) * scale) of the largest
            // accumulator M whenever g(M) is finite (M itself a finite
            // score).  Otherwise (a score overflowing f16, no finite score)
            // the workgroup takes the exact pass over the f16 scores.
            loop<FA_MAX>(ahead, qf, k0, cnt, n, T.nfull, T.jlim, 0.0f, false, mr, m2, o, sum, acc, sl);
            if (cnt > 0) {   // pass 2's first QK^T: the same tile, in place
                h8 kf[KS];
                read_k(sl, kf);
                acc = qk(qf, kf);
            }
            float m1 = fmaxf(mr, __shfl_xor(mr, 32, 64));
            if (lane < 32) stm[half * 32 + lane] = m1;
            lds_barrier();
            float m = (float)((h16)fmaxf(m1, stm[(half ^ 1) * 32 + (lane & 31)]) * (h16)a.scale_h);
            const bool exact = wg_any(!(__builtin_fabsf(m) < INFINITY) && T.myq < a.S, votes, 2 * HPW);
            if (exact) {
                pass<FA_MAX_EXACT>(qf, k0, cnt, n, T.nfull, T.jlim, 0.0f, false, mr, m2, o, sum);
                m1 = fmaxf((float)m2[0], (float)m2[1]);
                m1 = fmaxf(m1, __shfl_xor(m1, 32, 64));
                if (lane < 32) stm[half * 32 + lane] = m1;
                lds_barrier();
                m = fmaxf(m1, stm[(half ^ 1) * 32 + (lane & 31)]);
            }
            const bool deg = !(m > -INFINITY) && T.myq < a.S;   // no finite score in the row
            const bool anydeg = wg_any(deg, votes + 2 * HPW, 2 * HPW);
            if (anydeg) {
                // every key of the cache, the degenerate rows uniformly
                const int nk = Jp / 32, nhd = (nk + 1) / 2;
                pass<FA_PV_DEG>(qf, half ? nhd : 0, half ? nk - nhd : nhd, nhd, 0, T.jlim, deg ? 0.0f : m, deg, mr, m2,
                                o, sum);
            } else {
                if (exact) {   // the ring refilled from pass 2's first step
                    cur = Cursor{j + 1, 0};
                    start(ahead, qf, cnt, acc, sl);
                    loop<FA_PV_SAFE>(ahead, qf, k0, cnt, n, T.nfull, T.jlim, m, false, mr, m2, o, sum, acc, sl);
                } else {
                    loop<FA_PV>(ahead, qf, k0, cnt, n, T.nfull, T.jlim, m, false, mr, m2, o, sum, acc, sl);
                }
            }
            fa_finish<D>(a, h, T.s0, half, store, os, o, sum, stm, sts, ob, ot);
            if (u + 1 < nu) {   // query tile t1: its q rows, its first tile in place (or the ring refilled)
#pragma unroll
                for (int ks = 0; ks < KS; ks++) qf[ks] = qn[ks];
                if (anydeg) {
                    cur = Cursor{j + 2, 0};
                    start(ahead, qf, job_cnt(s, j + 2), acc, sl);
                } else {
                    acc = f16v{};
                    if (job_cnt(s, j + 2) > 0) {
                        h8 kf[KS];
                        read_k(sl, kf);
                        acc = qk(qf, kf);
                    }
                }
            }
        }
        sk_wait_vm<0>();   // no copy into LDS outstanding when the workgroup ends
    }
};

template <int D>
__global__ __launch_bounds__(fa_heads<D>() * 128) void attention_mfma_staged_kernel(AttnArgs a,
                                                                    const uint16_t* __restrict__ vt, int J,
                                                                    int Jp, int nqt) {
    using L = FaStaged<D>;
    constexpr int HPW = L::HPW, NT = L::NT;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[L::RING + 1024];   // + the pieces that copy nothing
    __shared__ float stm[HPW][64], sts[HPW][64];
    __shared__ float ob[HPW][NT * 16 * 64];
    __shared__ __attribute__((aligned(16))) uint16_t ot[HPW][32 * fa_ot_stride<D>()];
    __shared__ int votes[4 * HPW];
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), hw = w % HPW, half = w / HPW;
    const int hh = blockIdx.y * HPW + hw;
    const int kvh = (int)(blockIdx.y * HPW) / (a.H / a.Hkv);
    const L fs(a, vt, J, Jp, kvh, min(hh, a.H - 1), hw, half, ring);
    // causal: tiles n-1-x and x
    const int t0 = a.causal ? nqt - 1 - (int)blockIdx.x : (int)blockIdx.x, t1 = blockIdx.x;
    fs.run(t0, t1, a.causal && t1 < t0 ? 2 : 1, hh < a.H, stm[hw], sts[hw], ob[hw], ot[hw], votes);
}

// S >= 128 query rows; fewer take the matrix cores only past the
// one-workgroup kernels' score row (more than ATT_MAX_J keys), where those
// kernels cannot run.
bool attention_mfma_ok(const AttnArgs& a, int J) {
    const int qs = a.q_stride ? a.q_stride : a.H * a.D;
    const int os = a.out_stride ? a.out_stride : a.H * a.D;
    return (a.S >= 128 || (a.S >= 2 && J > ATT_MAX_J)) && J >= 1 && (a.D == 64 || a.D == 80 || a.D == 128) &&
           !a.d_pos && qs % 8 == 0 &&
           os % 8 == 0 && ((uintptr_t)a.q % 16) == 0 && ((uintptr_t)a.k % 16) == 0 && ((uintptr_t)a.v % 16) == 0 &&
           ((uintptr_t)a.out % 16) == 0;
}

size_t attention_mfma_scratch(int J, int Hkv, int D) {
    return (size_t)Hkv * D * (size_t)((J + 31) / 32 * 32) * sizeof(uint16_t);
}

// The staged kernel: every workgroup's heads on one KV head, and the K and
// V^T byte ranges within its 32-bit buffer offsets.
static bool attention_staged_ok(const AttnArgs& a, int J) {
    const int hpw = a.D > 80 ? 2 : 4;
    const size_t jp = (size_t)(J + 31) / 32 * 32;
    return (a.H / a.Hkv) % hpw == 0 && (size_t)J * a.Hkv * a.D * 2 < 0x80000000u &&
           jp * a.Hkv * a.D * 2 < 0x80000000u;
}

// Heads per workgroup of the operands-from-memory kernel without GQA: one,
// so a prefill fills the device (Phi-2, 32 heads at S = 512: 256 workgroups
// instead of 64; measured on MI355X, 512-token prefill 7.97 -> 7.52 ms, 7.60
// with two heads per workgroup, same tokens).
constexpr int FA_HPW_NOGQA = 1;
template <int D>
static void launch_fa(hipStream_t s, const AttnArgs& a, const uint16_t* vt, int J, int Jp, int nqt, int gx, bool staged) {
    constexpr int HPW = fa_heads<D>();
    const dim3 grid(gx, (a.H + HPW - 1) / HPW), block(HPW * 128);
    if (staged) {
        hipLaunchKernelGGL(attention_mfma_staged_kernel<D>, grid, block, 0, s, a, vt, J, Jp, nqt);
    } else if (a.H == a.Hkv) {
        constexpr int H1 = FA_HPW_NOGQA;
        hipLaunchKernelGGL((attention_mfma_kernel<D, H1>), dim3(gx, (a.H + H1 - 1) / H1), dim3(H1 * 128), 0, s, a, vt, J, Jp, nqt);
    } else {
        hipLaunchKernelGGL(attention_mfma_kernel<D>, grid, block, 0, s, a, vt, J, Jp, nqt);
    }
}

// Prefill over J keys through the matrix cores; vt holds
// attention_mfma_scratch(J, Hkv, D) bytes.
tlhip_status launch_attention_mfma(hipStream_t s, const AttnArgs& a, int J, uint16_t* vt) {
    if (!attention_mfma_ok(a, J) || !vt)
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "attention: shape not on the matrix-core path");
    if (a.Hkv <= 0 || a.H % a.Hkv) return fail(TLHIP_ERR_INVALID_DIMENSION, "attention: heads %d/%d", a.H, a.Hkv);
    const int Jp = (J + 31) / 32 * 32;
    hipLaunchKernelGGL(vt_transpose_kernel, dim3(Jp / 32, a.Hkv), dim3(256), 0, s, a.v, vt, J, Jp, a.Hkv, a.D);
    const int nqt = (a.S + 31) / 32;
    const int gx = a.causal ? (nqt + 1) / 2 : nqt;
    const bool staged = attention_staged_ok(a, J);
    if (a.D == 64) launch_fa<64>(s, a, vt, J, Jp, nqt, gx, staged);
    else if (a.D == 80) launch_fa<80>(s, a, vt, J, Jp, nqt, gx, staged);
    else launch_fa<128>(s, a, vt, J, Jp, nqt, gx, staged);
    return TLHIP_OK;
}

static void launch_attn_any(hipStream_t s, const AttnArgs& a, int J) {
    // a key count known at launch above one 256-key pass takes the 512-thread
    // variant (512 keys per pass); decode (J read on the device) keeps 256.
    // A key count known at launch of at most 512 takes a 2 KiB score row
    // instead of the 32 KiB one, so more workgroups share a CU.
    const bool small = !a.d_pos && J <= 512;
    const dim3 g(a.S, a.H);
    if (a.D == 64 && !a.d_pos && J > 256) {
        if (small) hipLaunchKernelGGL((attention64_kernel<512, 512>), g, dim3(512), 0, s, a, J);
        else hipLaunchKernelGGL(attention64_kernel<512>, g, dim3(512), 0, s, a, J);
    } else if (a.D == 64) {
        // decode: 512 threads, 4 K / V rows per key group and pass (256 keys
        // per pass as with 256 x 8, half the loads per lane before the first
        // dot product; config-4 decode 1951.6 -> 1971 tok/s on MI355X)
        if (a.d_pos && a.S == 1 && a.causal && !a.q_stride && !a.out_stride && a.kv_rows > 0)
            hipLaunchKernelGGL((attention64_kernel<512, ATT_MAX_J, 4, true>), g, dim3(512), 0, s, a, J);
        else if (small && J <= 64) hipLaunchKernelGGL((attention64_kernel<256, 64, 2>), g, dim3(256), 0, s, a, J);
        else if (small) hipLaunchKernelGGL((attention64_kernel<256, 512>), g, dim3(256), 0, s, a, J);
        else hipLaunchKernelGGL(attention64_kernel<256>, g, dim3(256), 0, s, a, J);
    } else if (a.D == 80) {
        if (small) hipLaunchKernelGGL((attention_dk_kernel<80, 512>), g, dim3(ADK_THREADS), 0, s, a, J);
        else hipLaunchKernelGGL(attention_dk_kernel<80>, g, dim3(ADK_THREADS), 0, s, a, J);
    } else if (a.D == 128) {
        if (small) hipLaunchKernelGGL((attention_dk_kernel<128, 512>), g, dim3(ADK_THREADS), 0, s, a, J);
        else hipLaunchKernelGGL(attention_dk_kernel<128>, g, dim3(ADK_THREADS), 0, s, a, J);
    } else {
        hipLaunchKernelGGL(attention_kernel, g, dim3(256), 0, s, a, J);
    }
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

// The two einsums for head dims 64 / 80 / 128, laid out for the memory
// system as the fused attention kernels are: a K / V row is read by 8 lanes
// (lane c holds dims EPL*c .. EPL*c + EPL - 1, EPL = D / 8) with 16-byte
// loads where the row allows, instead of one lane walking a row serially.
// scores: 8 lanes per output (i, h, j), 32 outputs per workgroup, the 8
// partial dot products combined with an xor tree.
template <int D>
__global__ __launch_bounds__(256) void scores8_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                      uint16_t* __restrict__ out, int I, int J, int H, int Hkv) {
    constexpr int EPL = D / 8, NW = EPL / 2;
    const int c = threadIdx.x & 7;
    const int64_t n = (int64_t)I * H * J;
    const int64_t o = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    const int64_t oc = o < n ? o : n - 1;   // (clamped: every load stays inside the tensors)
    const int j = (int)(oc % J), h = (int)((oc / J) % H), i = (int)(oc / ((int64_t)J * H));
    const int kvh = h / (H / Hkv);
    uint32_t qw[NW], kw[NW];
    load_row_words<NW>((const uint32_t*)(q + ((size_t)i * H + h) * D + EPL * c), qw);
    load_row_words<NW>((const uint32_t*)(k + ((size_t)j * Hkv + kvh) * D + EPL * c), kw);
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < NW; t++) {
        const h2 a2 = as_h2(qw[t]), b2 = as_h2(kw[t]);
        acc += (float)a2[0] * (float)b2[0];
        acc += (float)a2[1] * (float)b2[1];
    }
    acc = group8_sum(acc);
    if (c == 0 && o < n) out[o] = f2h(acc);
}

// context: one 256-thread workgroup per row (i, h); 32 key groups of 8
// lanes, each holding keys g, g + 32, ... (8 rows' loads in flight per
// pass); the key groups' partial rows summed within each wave, then over the
// waves, in a fixed order.
template <int D>
__global__ __launch_bounds__(256) void context8_kernel(const uint16_t* __restrict__ p, const uint16_t* __restrict__ v,
                                                       uint16_t* __restrict__ out, int J, int H, int Hkv) {
    constexpr int EPL = D / 8, NW = EPL / 2, NG = 32, UNR = 8;
    __shared__ float part[4][D];
    const int row = blockIdx.x, h = row % H, tid = threadIdx.x, c = tid & 7, g = tid >> 3;
    const int kvh = h / (H / Hkv);
    const uint16_t* pr = p + (size_t)row * J;
    const uint32_t* vb = (const uint32_t*)(v + (size_t)kvh * D + EPL * c);
    const size_t wstride = (size_t)Hkv * D / 2;
    float o[EPL];
#pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = 0.0f;
    for (int j0 = g; j0 < J; j0 += NG * UNR) {
        uint32_t vw[UNR][NW];
        float pj[UNR];
#pragma unroll
        for (int u = 0; u < UNR; u++) {   // (unconditional, clamped rows)
            const int jc = min(j0 + NG * u, J - 1);
            load_row_words<NW>(vb + (size_t)jc * wstride, vw[u]);
            pj[u] = h2f(pr[jc]);
        }
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            if (j0 + NG * u < J) {
#pragma unroll
                for (int t = 0; t < NW; t++) {
                    const h2 v2 = as_h2(vw[u][t]);
                    o[2 * t] += pj[u] * (float)v2[0];
                    o[2 * t + 1] += pj[u] * (float)v2[1];
                }
            }
        }
    }
#pragma unroll
    for (int e = 0; e < EPL; e++) o[e] = stride8_sum(o[e]);
    if ((tid & 63) < 8)
#pragma unroll
        for (int e = 0; e < EPL; e++) part[tid >> 6][EPL * c + e] = o[e];
    lds_barrier();
    if (tid < D) out[(size_t)row * D + tid] = f2h(((part[0][tid] + part[1][tid]) + part[2][tid]) + part[3][tid]);
}

// The 8-lane kernels for D = 64 / 80 / 128 on 4-byte aligned tensors, the
// one-output-per-thread kernels otherwise.
static bool einsum8_ok(const void* a, const void* b, int D) {
    return (D == 64 || D == 80 || D == 128) && ((uintptr_t)a & 3) == 0 && ((uintptr_t)b & 3) == 0;
}

tlhip_status launch_scores(hipStream_t s, const uint16_t* q, const uint16_t* k, uint16_t* sc, int I,
                           int J, int H, int Hkv, int D) {
    int64_t n = (int64_t)I * H * J;
    if (n <= 0) return TLHIP_OK;
    if (einsum8_ok(q, k, D)) {
        const dim3 grid((unsigned)((n + 31) / 32));
        if (D == 64) hipLaunchKernelGGL(scores8_kernel<64>, grid, dim3(256), 0, s, q, k, sc, I, J, H, Hkv);
        else if (D == 80) hipLaunchKernelGGL(scores8_kernel<80>, grid, dim3(256), 0, s, q, k, sc, I, J, H, Hkv);
        else hipLaunchKernelGGL(scores8_kernel<128>, grid, dim3(256), 0, s, q, k, sc, I, J, H, Hkv);
        return TLHIP_OK;
    }
    hipLaunchKernelGGL(scores_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, q, k, sc, I, J, H,
                       Hkv, D);
    return TLHIP_OK;
}

tlhip_status launch_context(hipStream_t s, const uint16_t* p, const uint16_t* v, uint16_t* out, int I,
                            int J, int H, int Hkv, int D) {
    int64_t n = (int64_t)I * H * D;
    if (n <= 0) return TLHIP_OK;
    if (J > 0 && einsum8_ok(p, v, D) && (int64_t)I * H <= 0x7fffffff) {
        const dim3 grid((unsigned)(I * H));
        if (D == 64) hipLaunchKernelGGL(context8_kernel<64>, grid, dim3(256), 0, s, p, v, out, J, H, Hkv);
        else if (D == 80) hipLaunchKernelGGL(context8_kernel<80>, grid, dim3(256), 0, s, p, v, out, J, H, Hkv);
        else hipLaunchKernelGGL(context8_kernel<128>, grid, dim3(256), 0, s, p, v, out, J, H, Hkv);
        return TLHIP_OK;
    }
    hipLaunchKernelGGL(context_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, v, out, I, J,
                       H, Hkv, D);
    return TLHIP_OK;
}

// einsum_ihd_jhd_ihj_f32 / einsum_ihj_jhd_ihd_f32 (unified.metal:2702-2768,
// einsum.rs:740-886): one thread per output, the sum over d (scores) or j
// (context) in index order, each term one fused multiply-add (the
// contraction of `sum += A * B` under Metal's default fast math, assumed as
// for the f32 linear).  Query head h reads KV head h / (H / Hkv); the
// reference's kernels take equal head counts, which is Hkv == H.
__global__ void scores_f32_kernel(const float* __restrict__ q, const float* __restrict__ k, float* __restrict__ sc,
                                  int I, int J, int H, int Hkv, int D) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)I * H * J) return;
    const int j = (int)(idx % J);
    const int64_t ih = idx / J;
    const int h = (int)(ih % H);
    const float* qr = q + (size_t)ih * D;
    const float* kr = k + ((size_t)j * Hkv + h / (H / Hkv)) * D;
    float sum = 0.0f;
    for (int d = 0; d < D; d++) sum = fmaf(qr[d], kr[d], sum);
    sc[idx] = sum;
}

__global__ void context_f32_kernel(const float* __restrict__ p, const float* __restrict__ v, float* __restrict__ out,
                                   int I, int J, int H, int Hkv, int D) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)I * H * D) return;
    const int d = (int)(idx % D);
    const int64_t ih = idx / D;
    const int h = (int)(ih % H);
    const float* pr = p + (size_t)ih * J;
    const float* vc = v + (size_t)(h / (H / Hkv)) * D + d;
    const size_t vstride = (size_t)Hkv * D;
    float sum = 0.0f;
    for (int j = 0; j < J; j++) sum = fmaf(pr[j], vc[(size_t)j * vstride], sum);
    out[idx] = sum;
}

tlhip_status launch_scores_f32(hipStream_t s, const float* q, const float* k, float* sc, int I, int J, int H, int Hkv,
                               int D) {
    const int64_t n = (int64_t)I * H * J;
    if (n <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(scores_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, q, k, sc, I, J, H, Hkv,
                       D);
    return TLHIP_OK;
}

tlhip_status launch_context_f32(hipStream_t s, const float* p, const float* v, float* out, int I, int J, int H, int Hkv,
                                int D) {
    const int64_t n = (int64_t)I * H * D;
    if (n <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(context_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, v, out, I, J, H,
                       Hkv, D);
    return TLHIP_OK;
}

}  // namespace tlhip
