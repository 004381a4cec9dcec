// kernels_elem.hip -- bandwidth-bound kernels of the hot path, gfx950:
// RMSNorm, LayerNorm, RoPE (+ fused KV-cache write), softmax, elementwise
// activations, attention mask, embedding gather and greedy argmax.
//
// Each kernel stores f16 exactly where the reference stores f16 and computes
// in f32 in between, following the reference op named beside it.
#include <algorithm>

#include "device_common.hpp"
#include "internal.hpp"

namespace tlhip {

// Block-wide sum / max over 256 threads in a fixed order (wave xor tree,
// then the 4 wave partials in order): deterministic for a given launch.
__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = wave_sum<64>(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float block_max256(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// ---------------------------------------------------------------------------
// RMSNorm  (rms_norm_cpu normalization.rs:199-250, rms_norm_f16
// unified.metal:1785-1831): y = f16((x * (1/sqrt(mean(x^2) + eps))) * w)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rms_norm_kernel(const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ w,
                                                       uint16_t* __restrict__ y, int n, float eps) {
    __shared__ float red[4];
    const uint16_t* xr = x + (size_t)blockIdx.x * n;
    uint16_t* yr = y + (size_t)blockIdx.x * n;
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        float v = h2f(xr[i]);
        s += v * v;
    }
    s = block_sum256(s, red);
    const float mean_sq = s / (float)n;
    const float rms = sqrtf(mean_sq + eps);
    const float inv = 1.0f / rms;
    for (int i = threadIdx.x; i < n; i += 256) {
        float nv = h2f(xr[i]) * inv;
        yr[i] = f2h(nv * h2f(w[i]));
    }
}

// The same with 16-byte accesses for n % 8 == 0, n <= 8 * 256 * NC: thread t
// holds the 8-element chunks t, t+256, ... of its row in registers, so x and
// w are read once, with every load issued before the reduction.
template <int NC>
__global__ __launch_bounds__(256) void rms_norm_vec_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w,
                                                           uint16_t* __restrict__ y, int n, float eps) {
    __shared__ float red[4];
    const u4* xr = (const u4*)(x + (size_t)blockIdx.x * n);
    const u4* wr = (const u4*)w;
    u4* yr = (u4*)(y + (size_t)blockIdx.x * n);
    const int nch = n >> 3;
    u4 xv[NC], wv[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int i = threadIdx.x + 256 * c;
        xv[c] = i < nch ? xr[i] : u4{0u, 0u, 0u, 0u};
        wv[c] = i < nch ? wr[i] : u4{0u, 0u, 0u, 0u};
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const h2 v = as_h2(xv[c][k]);
            s += (float)v[0] * (float)v[0];
            s += (float)v[1] * (float)v[1];
        }
    s = block_sum256(s, red);
    const float inv = 1.0f / sqrtf(s / (float)n + eps);
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int i = threadIdx.x + 256 * c;
        if (i < nch) {
            u4 o;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const h2 v = as_h2(xv[c][k]), g = as_h2(wv[c][k]);
                o[k] = (uint32_t)f2h(((float)v[0] * inv) * (float)g[0]) | ((uint32_t)f2h(((float)v[1] * inv) * (float)g[1]) << 16);
            }
            yr[i] = o;
        }
    }
}

tlhip_status launch_rms_norm(hipStream_t s, const uint16_t* x, const uint16_t* w, uint16_t* y,
                             int rows, int n, float eps) {
    if (rows <= 0 || n <= 0) return TLHIP_OK;
    const bool vec = n % 8 == 0 && ((uintptr_t)x | (uintptr_t)w | (uintptr_t)y) % 16 == 0;
    if (vec && n <= 2048) hipLaunchKernelGGL(rms_norm_vec_kernel<1>, dim3(rows), dim3(256), 0, s, x, w, y, n, eps);
    else if (vec && n <= 4096) hipLaunchKernelGGL(rms_norm_vec_kernel<2>, dim3(rows), dim3(256), 0, s, x, w, y, n, eps);
    else if (vec && n <= 8192) hipLaunchKernelGGL(rms_norm_vec_kernel<4>, dim3(rows), dim3(256), 0, s, x, w, y, n, eps);
    else hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(256), 0, s, x, w, y, n, eps);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// LayerNorm (layer_norm_f16 unified.metal:1620-1697): two-pass mean and
// biased variance in f32, y = f16(((x - mean) * inv_std) * w + b)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void layer_norm_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ w,
                                                         const uint16_t* __restrict__ b,
                                                         uint16_t* __restrict__ y, int n, float eps) {
    __shared__ float red[4];
    const uint16_t* xr = x + (size_t)blockIdx.x * n;
    uint16_t* yr = y + (size_t)blockIdx.x * n;
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) s += h2f(xr[i]);
    s = block_sum256(s, red);
    const float mean = s / (float)n;
    float q = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        float d = h2f(xr[i]) - mean;
        q += d * d;
    }
    q = block_sum256(q, red);
    const float var = q / (float)n;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (int i = threadIdx.x; i < n; i += 256) {
        float v = (h2f(xr[i]) - mean) * inv_std;
        if (w) v = v * h2f(w[i]);
        if (b) v = v + h2f(b[i]);
        yr[i] = f2h(v);
    }
}

// The same with 16-byte accesses (n % 8 == 0, n <= 8 * 256 * NC), the row
// held in registers between the two reductions.
template <int NC>
__global__ __launch_bounds__(256) void layer_norm_vec_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ w,
                                                             const uint16_t* __restrict__ b,
                                                             uint16_t* __restrict__ y, int n, float eps) {
    __shared__ float red[4];
    const u4* xr = (const u4*)(x + (size_t)blockIdx.x * n);
    u4* yr = (u4*)(y + (size_t)blockIdx.x * n);
    const int nch = n >> 3;
    u4 xv[NC], wv[NC], bv[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int i = threadIdx.x + 256 * c;
        const bool in = i < nch;
        xv[c] = in ? xr[i] : u4{0u, 0u, 0u, 0u};
        wv[c] = in && w ? ((const u4*)w)[i] : u4{0u, 0u, 0u, 0u};
        bv[c] = in && b ? ((const u4*)b)[i] : u4{0u, 0u, 0u, 0u};
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const h2 v = as_h2(xv[c][k]);
            s += (float)v[0];
            s += (float)v[1];
        }
    s = block_sum256(s, red);
    const float mean = s / (float)n;
    float q = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; c++)
        if (threadIdx.x + 256 * c < nch)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const h2 v = as_h2(xv[c][k]);
                const float d0 = (float)v[0] - mean, d1 = (float)v[1] - mean;
                q += d0 * d0;
                q += d1 * d1;
            }
    q = block_sum256(q, red);
    const float inv_std = 1.0f / sqrtf(q / (float)n + eps);
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int i = threadIdx.x + 256 * c;
        if (i < nch) {
            u4 o;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const h2 v = as_h2(xv[c][k]), g = as_h2(wv[c][k]), bb = as_h2(bv[c][k]);
                float r[2];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    float t = ((float)v[e] - mean) * inv_std;
                    if (w) t = t * (float)g[e];
                    if (b) t = t + (float)bb[e];
                    r[e] = t;
                }
                o[k] = (uint32_t)f2h(r[0]) | ((uint32_t)f2h(r[1]) << 16);
            }
            yr[i] = o;
        }
    }
}

tlhip_status launch_layer_norm(hipStream_t s, const uint16_t* x, const uint16_t* w,
                               const uint16_t* b, uint16_t* y, int rows, int n, float eps) {
    if (rows <= 0 || n <= 0) return TLHIP_OK;
    const bool vec = n % 8 == 0 && ((uintptr_t)x | (uintptr_t)w | (uintptr_t)b | (uintptr_t)y) % 16 == 0;
    if (vec && n <= 2048) hipLaunchKernelGGL(layer_norm_vec_kernel<1>, dim3(rows), dim3(256), 0, s, x, w, b, y, n, eps);
    else if (vec && n <= 4096) hipLaunchKernelGGL(layer_norm_vec_kernel<2>, dim3(rows), dim3(256), 0, s, x, w, b, y, n, eps);
    else if (vec && n <= 8192) hipLaunchKernelGGL(layer_norm_vec_kernel<4>, dim3(rows), dim3(256), 0, s, x, w, b, y, n, eps);
    else hipLaunchKernelGGL(layer_norm_kernel, dim3(rows), dim3(256), 0, s, x, w, b, y, n, eps);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// RoPE (rope_f16 unified.metal:2355-2418): rotate pairs by the angle of
// position pos = offset + s, cos/sin from the precomputed table.
//   out0 = f16(x0*c - x1*s), out1 = f16(x0*s + x1*c) -- products rounded
//   separately (no fused multiply-add), as the f32 scalar code rounds.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, float& r0, float& r1) {
    float a = __fmul_rn(x0, c), b = __fmul_rn(x1, s);
    r0 = __fsub_rn(a, b);
    float e = __fmul_rn(x0, s), f = __fmul_rn(x1, c);
    r1 = __fadd_rn(e, f);
}

__device__ __forceinline__ void rope_indices(int layout, int i, int half, int& i0, int& i1) {
    if (layout == 0) { i0 = 2 * i; i1 = 2 * i + 1; }
    else { i0 = i; i1 = i + half; }
}

// x, y: [batch][S][H][D] with row (per s) strides in elements.
__global__ void rope_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y, int S, int H,
                            int D, int64_t batch, int offset, const int32_t* d_pos, int layout,
                            int rot, const float* __restrict__ table, int xs, int ys) {
    const int half = rot / 2;
    const int64_t per_row = (int64_t)H * (D - half);   // pairs + pass-through elements
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = batch * S * per_row;
    if (idx >= total) return;
    const int64_t row = idx / per_row;        // batch*S index
    const int64_t rem = idx % per_row;
    const int h = (int)(rem / (D - half)), e = (int)(rem % (D - half));
    const int s = (int)(row % S);
    const int pos = offset + s + (d_pos ? *d_pos : 0);
    const uint16_t* xr = x + (size_t)row * xs + (size_t)h * D;
    uint16_t* yr = y + (size_t)row * ys + (size_t)h * D;
    if (e < half) {
        int i0, i1;
        rope_indices(layout, e, half, i0, i1);
        const float c = table[2 * ((size_t)pos * half + e)], sn = table[2 * ((size_t)pos * half + e) + 1];
        float r0, r1;
        rope_pair(h2f(xr[i0]), h2f(xr[i1]), c, sn, r0, r1);
        yr[i0] = f2h(r0);
        yr[i1] = f2h(r1);
    } else {
        const int d = rot + (e - half);   // pass-through dims >= rot
        yr[d] = xr[d];
    }
}

// The interleaved layout with every dim rotated and dense rows: each thread
// rotates 8 consecutive elements (4 adjacent pairs) of a head row with one
// 16-byte load and store, and reads the 4 pairs' (cos, sin) as two 16-byte
// loads of the table -- consecutive threads on consecutive 16 bytes.  The
// arithmetic is rope_kernel's (rope_pair), bit for bit.
__global__ void rope_vec8_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y, int S, int H, int D,
                                 int64_t groups, int offset, const int32_t* d_pos, const float* __restrict__ table) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    const int gpr = H * D / 8;   // 8-element groups per sequence row
    const int s = (int)((g / gpr) % S);
    const int e0 = (int)(g % (D / 8)) * 8;
    const int pos = offset + s + (d_pos ? *d_pos : 0);
    const u4 v = ((const u4*)x)[g];
    const float4* tp = (const float4*)(table + 2 * ((size_t)pos * (D / 2) + e0 / 2));
    const float4 t0 = tp[0], t1 = tp[1];
    const float c[4] = {t0.x, t0.z, t1.x, t1.z}, sn[4] = {t0.y, t0.w, t1.y, t1.w};
    u4 o;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const h2 p2 = as_h2(v[k]);
        float r0, r1;
        rope_pair((float)p2[0], (float)p2[1], c[k], sn[k], r0, r1);
        o[k] = (uint32_t)f2h(r0) | ((uint32_t)f2h(r1) << 16);
    }
    ((u4*)y)[g] = o;
}

tlhip_status launch_rope(hipStream_t s, const uint16_t* x, uint16_t* y, int S, int H, int D,
                         int64_t batch, int offset, const int32_t* d_pos, int layout, int rot_dims,
                         const float* table, int x_row_stride, int y_row_stride) {
    const int half = rot_dims / 2;
    int64_t total = batch * S * (int64_t)H * (D - half);
    if (total <= 0) return TLHIP_OK;
    const bool dense = (x_row_stride == 0 || x_row_stride == H * D) && (y_row_stride == 0 || y_row_stride == H * D);
    if (layout == 0 && rot_dims == D && D % 8 == 0 && dense && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0 &&
        ((uintptr_t)table & 15) == 0) {
        const int64_t groups = batch * S * (int64_t)H * D / 8;
        hipLaunchKernelGGL(rope_vec8_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, s, x, y, S, H, D,
                           groups, offset, d_pos, table);
        return TLHIP_OK;
    }
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x, y, S,
                       H, D, batch, offset, d_pos, layout, rot_dims, table,
                       x_row_stride ? x_row_stride : H * D, y_row_stride ? y_row_stride : H * D);
    return TLHIP_OK;
}

// Decoder glue: from a fused projection row [q (H*D) | k (Hkv*D) | v (Hkv*D)]
// write RoPE(q) to q_out, RoPE(k) and v into the KV cache rows at pos0 + s
// (model::llama::Cache stores K after RoPE, llama.rs:78-114).
__global__ void rope_kv_kernel(const uint16_t* __restrict__ qkv, int qkv_stride, int S, int H,
                               int Hkv, int D, int layout, int rot, const float* __restrict__ table,
                               int pos0, const int32_t* d_pos, uint16_t* __restrict__ q_out,
                               uint16_t* __restrict__ kc, uint16_t* __restrict__ vc) {
    const int half = rot / 2;
    const int per_head = D - half;               // pairs + pass-through
    const int nq = H * per_head, nk = Hkv * per_head, nv = Hkv * D;
    const int per_row = nq + nk + nv;
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)S * per_row) return;
    const int s = (int)(idx / per_row);
    int e = (int)(idx % per_row);
    const int base = pos0 + (d_pos ? *d_pos : 0);
    const int pos = base + s;
    const uint16_t* row = qkv + (size_t)s * qkv_stride;
    if (e >= nq + nk) {   // V: copy into the cache
        e -= nq + nk;
        vc[(size_t)pos * nv + e] = row[(size_t)(H + Hkv) * D + e];
        return;
    }
    const bool is_k = e >= nq;
    if (is_k) e -= nq;
    const int h = e / per_head, pe = e % per_head;
    const uint16_t* xr = row + (size_t)(is_k ? H + h : h) * D;
    uint16_t* yr = is_k ? kc + (size_t)pos * Hkv * D + (size_t)h * D : q_out + (size_t)s * H * D + (size_t)h * D;
    if (pe < half) {
        // layout 2: a pair-permuted projection (pair i in rows 2i, 2i+1)
        // rotated into the half-rotation output positions (i, i + half)
        int i0, i1, o0, o1;
        if (layout == 2) {
            i0 = 2 * pe;
            i1 = 2 * pe + 1;
            o0 = pe;
            o1 = pe + half;
        } else {
            rope_indices(layout, pe, half, i0, i1);
            o0 = i0;
            o1 = i1;
        }
        const float c = table[2 * ((size_t)pos * half + pe)], sn = table[2 * ((size_t)pos * half + pe) + 1];
        float r0, r1;
        rope_pair(h2f(xr[i0]), h2f(xr[i1]), c, sn, r0, r1);
        yr[o0] = f2h(r0);
        yr[o1] = f2h(r1);
    } else {
        const int d = rot + (pe - half);
        yr[d] = xr[d];
    }
}

// rope_kv_kernel with 8 output elements per thread and 16-byte accesses,
// for the model's two layouts: 0 (interleaved pairs (2i, 2i+1) rotated in
// place, every dim rotated: rot == D) and 2 (pair-permuted rows, pair i at
// (2i, 2i+1), rotated into (i, i + half); dims >= rot pass through).  The
// per-pair arithmetic is rope_kv_kernel's (rope_pair, the same table
// entries).  Item e of a row: q heads, then k heads, each head
// rope8_items(layout, D, rot) items (layout 2: half / 8 items of 8 pairs,
// each writing 16 outputs (i, i + half), then (D - rot) / 8 items copying
// the pass-through dims; layout 0: D / 8 items of 4 pairs), then V, D / 8
// 16-byte copies per KV head.
__host__ __device__ __forceinline__ int rope8_items(int layout, int D, int rot) {
    return layout == 2 ? rot / 16 + (D - rot) / 8 : D / 8;
}

__global__ void rope_kv8_kernel(const uint16_t* __restrict__ qkv, int qkv_stride, int S, int H, int Hkv, int D,
                                int layout, int rot, const float* __restrict__ table, int pos0,
                                const int32_t* d_pos, uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
                                uint16_t* __restrict__ vc) {
    const int half = rot / 2, per_head = rope8_items(layout, D, rot);
    const int nq = H * per_head, nk = Hkv * per_head, per_row = nq + nk + Hkv * (D / 8);
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)S * per_row) return;
    const int s = (int)(idx / per_row);
    int e = (int)(idx % per_row);
    const int pos = pos0 + (d_pos ? *d_pos : 0) + s;
    const uint16_t* row = qkv + (size_t)s * qkv_stride;
    if (e >= nq + nk) {   // V: copy into the cache
        e -= nq + nk;
        *(u4*)(vc + (size_t)pos * Hkv * D + 8 * e) = *(const u4*)(row + (size_t)(H + Hkv) * D + 8 * e);
        return;
    }
    const bool is_k = e >= nq;
    if (is_k) e -= nq;
    const int h = e / per_head, pe = e % per_head;
    const uint16_t* xr = row + (size_t)(is_k ? H + h : h) * D;
    uint16_t* yr = is_k ? kc + (size_t)pos * Hkv * D + (size_t)h * D : q_out + (size_t)s * H * D + (size_t)h * D;
    const float* tp = table + 2 * (size_t)pos * half;
    if (layout == 0) {   // pairs 4 pe .. 4 pe + 3 in place
        const u4 x = *(const u4*)(xr + 8 * pe);
        u4 y;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const h2 v = as_h2(x[k]);
            const int i = 4 * pe + k;
            float r0, r1;
            rope_pair((float)v[0], (float)v[1], tp[2 * i], tp[2 * i + 1], r0, r1);
            h2 o;
            o[0] = (h16)r0;
            o[1] = (h16)r1;
            y[k] = as_u32(o);
        }
        *(u4*)(yr + 8 * pe) = y;
        return;
    }
    const int hr = half / 8;
    if (pe >= hr) {   // pass-through dims rot + 8 (pe - hr) ..
        const int d = rot + 8 * (pe - hr);
        *(u4*)(yr + d) = *(const u4*)(xr + d);
        return;
    }
    // pairs 8 pe .. 8 pe + 7 (input elements 16 pe .. 16 pe + 15)
    const u4 xa = *(const u4*)(xr + 16 * pe), xb = *(const u4*)(xr + 16 * pe + 8);
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
        float r[2][2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const h2 v = as_h2(k + u < 4 ? xa[k + u] : xb[k + u - 4]);
            const int i = 8 * pe + k + u;
            rope_pair((float)v[0], (float)v[1], tp[2 * i], tp[2 * i + 1], r[u][0], r[u][1]);
        }
        h2 o0, o1;
        o0[0] = (h16)r[0][0];
        o0[1] = (h16)r[1][0];
        o1[0] = (h16)r[0][1];
        o1[1] = (h16)r[1][1];
        lo[k / 2] = as_u32(o0);
        hi[k / 2] = as_u32(o1);
    }
    *(u4*)(yr + 8 * pe) = u4{lo[0], lo[1], lo[2], lo[3]};
    *(u4*)(yr + half + 8 * pe) = u4{hi[0], hi[1], hi[2], hi[3]};
}

tlhip_status launch_rope_kv(hipStream_t s, const uint16_t* qkv, int qkv_stride, int S, int H,
                            int Hkv, int D, int layout, int rot_dims, const float* table, int pos0,
                            const int32_t* d_pos, uint16_t* q_out, uint16_t* kcache,
                            uint16_t* vcache) {
    const bool vec = D % 8 == 0 && qkv_stride % 8 == 0 && ((layout == 0 && rot_dims == D) || (layout == 2 && rot_dims % 16 == 0)) &&
                     ((uintptr_t)qkv | (uintptr_t)q_out | (uintptr_t)kcache | (uintptr_t)vcache | (uintptr_t)table) % 16 == 0;
    if (vec) {
        const int64_t total = (int64_t)S * ((H + Hkv) * rope8_items(layout, D, rot_dims) + Hkv * (D / 8));
        if (total <= 0) return TLHIP_OK;
        hipLaunchKernelGGL(rope_kv8_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, qkv, qkv_stride, S,
                           H, Hkv, D, layout, rot_dims, table, pos0, d_pos, q_out, kcache, vcache);
        return TLHIP_OK;
    }
    const int per_head = D - rot_dims / 2;
    int64_t total = (int64_t)S * ((H + Hkv) * per_head + Hkv * D);
    if (total <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(rope_kv_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, qkv,
                       qkv_stride, S, H, Hkv, D, layout, rot_dims, table, pos0, d_pos, q_out, kcache,
                       vcache);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// softmax over the last dim (softmax_f16 unified.metal:2057-2148 as
// dispatched one thread per row, activations.rs:204-209):
//   max over finite values (0 if none); e = exp(x - max) or 0 for
//   non-finite x; y = f16(e); sum += e (f32); y = f16(f32(y) / sum);
//   a zero / non-finite sum gives f16(1/n) everywhere.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void softmax_kernel(const uint16_t* __restrict__ x,
                                                      uint16_t* __restrict__ y, int n) {
    __shared__ float red[4];
    const uint16_t* xr = x + (size_t)blockIdx.x * n;
    uint16_t* yr = y + (size_t)blockIdx.x * n;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < n; i += 256) {
        float v = h2f(xr[i]);
        if (isfinite(v)) mx = fmaxf(mx, v);
    }
    mx = block_max256(mx, red);
    if (!isfinite(mx)) mx = 0.0f;
    float sum = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        float v = h2f(xr[i]);
        float e = isfinite(v) ? expf(v - mx) : 0.0f;
        yr[i] = f2h(e);
        sum += e;
    }
    sum = block_sum256(sum, red);
    if (sum > 0.0f && isfinite(sum)) {
        for (int i = threadIdx.x; i < n; i += 256) yr[i] = f2h(h2f(yr[i]) / sum);
    } else {
        const uint16_t u = f2h(1.0f / (float)n);
        for (int i = threadIdx.x; i < n; i += 256) yr[i] = u;
    }
}

tlhip_status launch_softmax(hipStream_t s, const uint16_t* x, uint16_t* y, int64_t rows, int n) {
    if (rows <= 0 || n <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(softmax_kernel, dim3((unsigned)rows), dim3(256), 0, s, x, y, n);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// elementwise (f16 in/out, f32 math, one rounding per reference op)
// ---------------------------------------------------------------------------
__global__ void elementwise_kernel(int op, const uint16_t* __restrict__ a,
                                   const uint16_t* __restrict__ b, uint16_t* __restrict__ y,
                                   int64_t n, int64_t bp, float sc) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint16_t av = a[i];
    uint16_t r;
    switch (op) {
        case EW_SIGMOID: r = sigmoid_h(av); break;
        case EW_SILU: r = f2h(h2f(av) * h2f(sigmoid_h(av))); break;
        case EW_GELU: r = gelu_h(av); break;
        case EW_ADD: r = f2h(h2f(av) + h2f(b[bp ? i % bp : i])); break;
        case EW_MUL: r = f2h(h2f(av) * h2f(b[bp ? i % bp : i])); break;
        case EW_MUL_SCALAR: r = f2h(h2f(av) * sc); break;
        case EW_SILU_MUL: r = swiglu_h(av, b[i]); break;
        default: r = av;
    }
    y[i] = r;
}

tlhip_status launch_elementwise(hipStream_t s, int op, const uint16_t* a, const uint16_t* b,
                                uint16_t* y, int64_t n, int64_t b_period, float scalar) {
    if (n <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(elementwise_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, op, a,
                       b, y, n, b_period, scalar);
    return TLHIP_OK;
}

// apply_attention_mask (masking.rs:147-165, unified.metal:4474-4489):
// y = mask == 0 ? -10000 : score.  Either the mask repeats every `period`
// elements of the scores, or scores are [I, H, J] and the mask is [I, J]
// (the TL pattern reshape(mask, [S,1,S]) + broadcast_to [S,H,S]).
__global__ void mask_kernel(const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mask,
                            uint16_t* __restrict__ y, int64_t n, int64_t period, int64_t inner,
                            int64_t heads) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t mi;
    if (heads > 1) {   // scores [I, H, J], mask [I, J]
        const int64_t j = i % inner, ih = i / inner, row = ih / heads;
        mi = row * inner + j;
    } else {
        mi = i % period;
    }
    const uint16_t m = mask[mi];
    y[i] = ((m & 0x7fffu) == 0) ? f2h(-10000.0f) : sc[i];
}

tlhip_status launch_mask(hipStream_t s, const uint16_t* sc, const uint16_t* mask, uint16_t* y,
                         int64_t n, int64_t mask_period) {
    // mask_period > 0: elementwise repeat; mask_period < 0 encodes (-J, H)
    // packed as -(J * 65536 + H) for scores [I, H, J] with mask [I, J].
    if (n <= 0) return TLHIP_OK;
    int64_t period = mask_period, inner = 1, heads = 1;
    if (mask_period < 0) {
        int64_t enc = -mask_period;
        inner = enc >> 16;
        heads = enc & 0xffff;
        period = 0;
    }
    hipLaunchKernelGGL(mask_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, sc, mask, y, n,
                       period, inner, heads);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// causal_mask(n) (builtin_nn.rs:423-460, Tensor::causal_mask masking.rs:
// 192-207): [n, n] f16, 1 where j <= i.  Eight elements per thread, one
// 16-byte store where the group lies inside the matrix.
// ---------------------------------------------------------------------------
__global__ void causal_mask_kernel(uint16_t* __restrict__ out, int64_t n) {
    const int64_t total = n * n;
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i0 >= total) return;
    uint16_t v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const int64_t i = i0 + e;
        v[e] = (i < total && i % n <= i / n) ? (uint16_t)0x3C00u : (uint16_t)0u;
    }
    if (i0 + 8 <= total && (i0 & 7) == 0) {
        *(u4*)(out + i0) = u4{(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16),
                              (uint32_t)v[4] | ((uint32_t)v[5] << 16), (uint32_t)v[6] | ((uint32_t)v[7] << 16)};
    } else {
        for (int e = 0; e < 8 && i0 + e < total; e++) out[i0 + e] = v[e];
    }
}

tlhip_status launch_causal_mask(hipStream_t s, uint16_t* out, int64_t n) {
    const int64_t groups = (n * n + 7) / 8;
    if (groups <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(causal_mask_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, s, out, n);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// Tensor::argmax(dim, keepdim) (reduce.rs:585-668, the argmax() builtin):
// one workgroup per output element.  The reference scans its line in order
// with a strict '>' (from element 0's value for the whole tensor, from -inf
// along a dim), so the result is the first index of the line's largest
// value, a NaN never wins, and along a dim neither does -inf (index 0 when
// nothing beats the start; for the whole tensor, also when element 0 is
// NaN).  Here every thread scans a strided part of the line and keeps the
// largest key (order-preserving image of the value << 32 | ~index: larger
// value first, then smaller index), -0 counted as +0; the keys meet in a
// workgroup maximum, which no scan order changes.  Line o starts at the
// coordinates the reference derives from o (first kept dim least
// significant, reduce.rs:649-657).  The index is stored as T::from_f64(i)
// in the input's type (f16: rounded to nearest even above 2048).
// ---------------------------------------------------------------------------
struct ArgmaxDims {
    int64_t shape[8];
    int64_t stride[8];
    int nd, dim;          // dim < 0: the whole tensor
    int64_t line, lstride;
};

__device__ __forceinline__ unsigned long long argmax_key(float v, int64_t i) {
    if (!(v > -INFINITY)) return 0ull;   // NaN and -inf never win a '>' against -inf
    if (v == 0.0f) v = 0.0f;             // -0 == +0
    const uint32_t b = __float_as_uint(v);
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)ord << 32) | (0xffffffffu - (uint32_t)i);
}

template <typename T>
__global__ __launch_bounds__(256) void tensor_argmax_kernel(const T* __restrict__ x, T* __restrict__ y, ArgmaxDims d) {
    __shared__ unsigned long long wk[4];
    int64_t base = 0;
    if (d.dim >= 0) {
        int64_t rem = blockIdx.x;
        for (int i = 0; i < d.nd; i++)
            if (i != d.dim) {
                base += (rem % d.shape[i]) * d.stride[i];
                rem /= d.shape[i];
            }
    }
    auto val = [&](int64_t i) -> float {
        if constexpr (sizeof(T) == 2) return h2f(x[base + i * d.lstride]);
        else return x[base + i * d.lstride];
    };
    unsigned long long best = 0ull;
    for (int64_t i = threadIdx.x; i < d.line; i += 256) {
        const unsigned long long k = argmax_key(val(i), i);
        best = k > best ? k : best;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)best, off), hi = __shfl_xor((uint32_t)(best >> 32), off);
        const unsigned long long o = ((unsigned long long)hi << 32) | lo;
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = wk[0];
        for (int w = 1; w < 4; w++) b = wk[w] > b ? wk[w] : b;
        int64_t idx = b ? (int64_t)(0xffffffffu - (uint32_t)b) : 0;
        if (d.dim < 0 && !(val(0) == val(0))) idx = 0;   // a NaN start is never beaten
        const float f = (float)idx;                        // exact below 2^24
        if constexpr (sizeof(T) == 2) y[blockIdx.x] = f2h(f);
        else y[blockIdx.x] = f;
    }
}

tlhip_status launch_tensor_argmax(hipStream_t s, tlhip_dtype dt, const void* x, void* y, const int64_t* shape, int nd,
                                  int dim) {
    if (nd > 8) return fail(TLHIP_ERR_INVALID_DIMENSION, "argmax: rank %d > 8", nd);
    ArgmaxDims d = {};
    d.nd = nd;
    d.dim = dim;
    int64_t total = 1, st = 1;
    for (int i = nd - 1; i >= 0; i--) {
        d.shape[i] = shape[i];
        d.stride[i] = st;
        st *= shape[i];
    }
    total = st;
    int64_t outs = 1;
    if (dim < 0) {
        d.line = total;
        d.lstride = 1;
    } else {
        d.line = shape[dim];
        d.lstride = d.stride[dim];
        outs = total / (shape[dim] ? shape[dim] : 1);
        if (shape[dim] == 0) {   // every line is empty: all outputs index 0
            outs = 1;
            for (int i = 0; i < nd; i++)
                if (i != dim) outs *= shape[i];
        }
    }
    if (d.line >= 0xffffffffll) return fail(TLHIP_ERR_INVALID_DIMENSION, "argmax: line of %lld elements", (long long)d.line);
    if (outs <= 0) return TLHIP_OK;
    if (outs > 0x7fffffffll) return fail(TLHIP_ERR_INVALID_DIMENSION, "argmax: %lld outputs", (long long)outs);
    if (dt == TLHIP_F16)
        hipLaunchKernelGGL(tensor_argmax_kernel<uint16_t>, dim3((unsigned)outs), dim3(256), 0, s, (const uint16_t*)x, (uint16_t*)y, d);
    else
        hipLaunchKernelGGL(tensor_argmax_kernel<float>, dim3((unsigned)outs), dim3(256), 0, s, (const float*)x, (float*)y, d);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// broadcast_to (broadcast.rs:11-120, broadcast_f16 unified.metal:3769-3815):
// target element g reads the input element whose coordinates are g's,
// aligned from the right, with coordinate 0 on the input's size-1 dims
// (stride 0 below).  One thread per output element, 2- or 4-byte elements.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void broadcast_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t total, BcastDims b) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= total) return;
    int64_t rem = g, src = 0;
    for (int i = b.nd - 1; i >= 0; i--) {
        const int64_t c = rem % b.shape[i];
        rem /= b.shape[i];
        src += c * b.xstride[i];
    }
    y[g] = x[src];
}

tlhip_status launch_broadcast(hipStream_t s, const void* x, void* y, int elem, const BcastDims& b) {
    int64_t total = 1;
    for (int i = 0; i < b.nd; i++) total *= b.shape[i];
    if (total <= 0) return TLHIP_OK;
    const dim3 grid((unsigned)((total + 255) / 256));
    if (elem == 2) hipLaunchKernelGGL(broadcast_kernel<uint16_t>, grid, dim3(256), 0, s, (const uint16_t*)x, (uint16_t*)y, total, b);
    else hipLaunchKernelGGL(broadcast_kernel<uint32_t>, grid, dim3(256), 0, s, (const uint32_t*)x, (uint32_t*)y, total, b);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// rope(x, cos, sin) = Tensor::rope_candle (rope.rs:18-65, rope_candle_f16
// unified.metal:5122-5185): x [S, H, D], tables [L >= S, D]; pair i of row
// s is rotated by cos[s, i] / sin[s, i] (column i, as the Metal kernel
// indexes the table), f32 products each rounded, f16 stores.  One thread
// per pair, both elements written by it.
// ---------------------------------------------------------------------------
__global__ void rope_cs_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ ct,
                               const uint16_t* __restrict__ st, uint16_t* __restrict__ y, int S, int H, int D) {
    const int64_t half = D / 2;
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= (int64_t)S * H * half) return;
    const int64_t i = p % half, sh = p / half, s = sh / H;
    const float c = h2f(ct[s * D + i]), sn = h2f(st[s * D + i]);
    const uint32_t xw = *(const uint32_t*)(x + sh * D + 2 * i);
    const float x0 = h2f((uint16_t)(xw & 0xffffu)), x1 = h2f((uint16_t)(xw >> 16));
    const float r0 = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, sn));
    const float r1 = __fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, c));
    *(uint32_t*)(y + sh * D + 2 * i) = (uint32_t)f2h(r0) | ((uint32_t)f2h(r1) << 16);
}

tlhip_status launch_rope_cs(hipStream_t s, const uint16_t* x, const uint16_t* ct, const uint16_t* st, uint16_t* y,
                            int S, int H, int D) {
    const int64_t pairs = (int64_t)S * H * (D / 2);
    if (pairs <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(rope_cs_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, s, x, ct, st, y, S, H, D);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// embedding (builtin_nn.rs:627-812, embedding_lookup_f16 unified.metal:
// 658-676): out[s, :] = table[id_s, :]; quantized tables are dequantised
// row by row (bit-exact with gguf.rs).  ids come from a device array, or in
// graph-replay decode from the device token slot.
// ---------------------------------------------------------------------------
__global__ void embedding_kernel(int tt, const uint8_t* __restrict__ tq, const uint16_t* __restrict__ td,
                                 const int32_t* __restrict__ ids, const int32_t* d_token,
                                 uint16_t* __restrict__ out, int n, int hidden, int rows) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)n * hidden) return;
    const int s = (int)(i / hidden), c = (int)(i % hidden);
    const int id = d_token ? d_token[0] : ids[s];
    if (tt == TLHIP_F16) {
        out[i] = ((const uint16_t*)tq)[(size_t)id * hidden + c];
        return;
    }
    if (tt == TLHIP_Q6_K) {
        // planes of the packed Q6_K layout (see internal.hpp)
        const int b = c / 32, e = c % 32;
        const uint8_t* q2 = tq + q6k_q2_offset(rows, hidden);
        const int8_t* sc = (const int8_t*)(tq + q6k_sc_offset(rows, hidden));
        const uint8_t byte = tq[(size_t)id * (hidden / 2) + 16 * b + (e & 15)];
        const int lo = e < 16 ? (byte & 15) : (byte >> 4);
        const int hb = (q2[(size_t)id * (hidden / 4) + 8 * b + 4 * (e / 16) + (e % 4)] >> (2 * ((e % 16) / 4))) & 3;
        const float ds = h2f(td[(size_t)id * (hidden / 256) + c / 256]) * (float)sc[(size_t)id * (hidden / 16) + c / 16];
        out[i] = f2h(ds * (float)((lo | (hb << 4)) - 32));
        return;
    }
    const int nbr = hidden / 32, b = c / 32, e = c % 32;
    const float d = h2f(td[(size_t)id * nbr + b]);
    float q;
    if (tt == TLHIP_Q4_0) {
        const uint8_t byte = tq[(size_t)id * (hidden / 2) + 16 * b + (e & 15)];
        q = (float)((e < 16 ? (byte & 15) : (byte >> 4)) - 8);
    } else {
        q = (float)(int8_t)tq[(size_t)id * hidden + c];
    }
    out[i] = f2h(q * d);
}

tlhip_status launch_embedding(hipStream_t s, tlhip_dtype tt, const void* tq, const uint16_t* td,
                              const int32_t* ids, const int32_t* d_token, uint16_t* out, int n,
                              int hidden, int rows) {
    int64_t total = (int64_t)n * hidden;
    if (total <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(embedding_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, (int)tt,
                       (const uint8_t*)tq, td, ids, d_token, out, n, hidden, rows);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// greedy argmax (temperature_sample with T <= 1e-4, builtin_sampling.rs:
// 170-176): Iterator::max_by keeps the LAST of equal maxima.  Optionally
// logs the token and advances the device decode state
// d_state = {token, pos, step}: token <- argmax, pos += 1, step += 1.
// ---------------------------------------------------------------------------
// (value, index) order of the reduction: larger value wins, equal values
// go to the larger index (the last maximum); index -1 means "none".
__device__ __forceinline__ void amax_merge(float& bv, int& bi, float v, int i) {
    if (i >= 0 && (bi < 0 || v > bv || (v == bv && i > bi))) {
        bv = v;
        bi = i;
    }
}

__global__ __launch_bounds__(1024) void argmax_kernel(const uint16_t* __restrict__ x, int n,
                                                      int32_t* out, int32_t* token_log,
                                                      int32_t* d_state) {
    __shared__ float sv[16];
    __shared__ int si[16];
    float best = -INFINITY;
    int bi = -1;
    // 8 elements per 16-byte load over the aligned body, scalar tail
    const int n8 = ((uintptr_t)x % 16 == 0) ? n / 8 : 0;
    for (int c = threadIdx.x; c < n8; c += 1024) {
        const u4 v4 = *(const u4*)(x + (size_t)c * 8);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const h2 p2 = as_h2(v4[t]);
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const float v = (float)p2[e];
                if (!isnan(v) && (bi < 0 || v >= best)) { best = v; bi = 8 * c + 2 * t + e; }
            }
        }
    }
    for (int i = 8 * n8 + threadIdx.x; i < n; i += 1024) {
        const float v = h2f(x[i]);
        if (!isnan(v) && (bi < 0 || v >= best)) { best = v; bi = i; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float v2 = __shfl_xor(best, off, 64);
        const int i2 = __shfl_xor(bi, off, 64);
        amax_merge(best, bi, v2, i2);
    }
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) {
        sv[w] = best;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = sv[0];
        int ib = si[0];
        for (int k = 1; k < 16; k++) amax_merge(b, ib, sv[k], si[k]);
        const int tok = ib < 0 ? 0 : ib;
        if (out) out[0] = tok;
        if (d_state) {
            if (token_log) token_log[d_state[2]] = tok;
            d_state[0] = tok;
            d_state[1] += 1;
            d_state[2] += 1;
        }
    }
}

tlhip_status launch_argmax(hipStream_t s, const uint16_t* x, int n, int32_t* out, int32_t* token_log,
                           int32_t* d_state) {
    if (n <= 0) return fail(TLHIP_ERR_INVALID_DIMENSION, "argmax of an empty tensor");
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, x, n, out, token_log, d_state);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// temperature_sample with T > 1e-4 (builtin_sampling.rs:178-215): s = x / T,
// e = exp(s - max), p = e / sum(e), then the first index whose running sum
// of p exceeds the draw r, else n - 1.  Two kernels:
//   sample_stats: workgroup w owns the 1024-logit slice w and records its
//     (max, sum of exp(s - slice max));
//   sample_pick: one workgroup combines the slice statistics into the row
//     max and sum, locates the slice whose probability mass holds r (slice
//     masses in slice order), then forms p for that slice with the row max
//     and sum and finds the first crossing with a workgroup scan in index
//     order.
// The draw is splitmix64(seed + (counter + 1) * golden)'s top 24 bits *
// 2^-24, with counter += d_state[2] (the decode step) when the decode state
// is given, so a replayed graph draws a fresh value per step.  Running sums
// are f32 as in the reference, summed in slice order.
// ---------------------------------------------------------------------------
constexpr int SMP_SLICE = 1024;   // logits per slice
constexpr int SMP_MAXW = 1024;    // slices: rows up to 1M logits

__device__ __forceinline__ float sample_uniform(uint64_t seed, uint64_t counter) {
    uint64_t z = seed + (counter + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)(z >> 40) * 0x1p-24f;
}

// max / sum over a workgroup of NW waves (partials in w_part[NW])
template <int NW>
__device__ __forceinline__ float wg_max(float v, float* w_part) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) w_part[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = w_part[0];
    for (int k = 1; k < NW; k++) m = fmaxf(m, w_part[k]);
    __syncthreads();
    return m;
}

template <int NW>
__device__ __forceinline__ float wg_sum(float v, float* w_part) {
    v = wave_sum<64>(v);
    if ((threadIdx.x & 63) == 0) w_part[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = w_part[0];
    for (int k = 1; k < NW; k++) t += w_part[k];
    __syncthreads();
    return t;
}

// exclusive scan over a 1024-thread workgroup in thread order (wave scans,
// then the wave totals in order); `total` = the sum of all
__device__ __forceinline__ float wg_excl_scan(float v, float* wtot, float& total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    float inc = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float u = __shfl_up(inc, off, 64);
        if (lane >= off) inc += u;
    }
    if (lane == 63) wtot[w] = inc;
    __syncthreads();
    float before = 0.0f, t = 0.0f;
    for (int k = 0; k < 16; k++) {
        if (k < w) before += wtot[k];
        t += wtot[k];
    }
    total = t;
    __syncthreads();
    return before + (inc - v);
}

__global__ __launch_bounds__(256) void sample_stats_kernel(const uint16_t* __restrict__ x, int n, float temperature,
                                                           float2* __restrict__ stats) {
    __shared__ float part[4];
    const int i0 = blockIdx.x * SMP_SLICE;
    float s[SMP_SLICE / 256];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < SMP_SLICE / 256; k++) {
        const int i = i0 + threadIdx.x + 256 * k;
        s[k] = i < n ? h2f(x[i]) / temperature : -INFINITY;
        mx = fmaxf(mx, s[k]);   // as f32::max: a NaN operand loses
    }
    mx = wg_max<4>(mx, part);
    float es = 0.0f;
#pragma unroll
    for (int k = 0; k < SMP_SLICE / 256; k++)
        if (i0 + (int)threadIdx.x + 256 * k < n) es += expf(s[k] - mx);
    es = wg_sum<4>(es, part);
    if (threadIdx.x == 0) stats[blockIdx.x] = make_float2(mx, es);
}

__global__ __launch_bounds__(1024) void sample_pick_kernel(const uint16_t* __restrict__ x, int n, float temperature,
                                                           uint64_t seed, uint64_t counter,
                                                           const float2* __restrict__ stats, int32_t* out,
                                                           int32_t* token_log, int32_t* d_state) {
    __shared__ float wpart[16];
    __shared__ int wmin[16];
    __shared__ float sh_off;
    __shared__ int sh_slice;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nw = (n + SMP_SLICE - 1) / SMP_SLICE;
    const float2 st = tid < nw ? stats[tid] : make_float2(-INFINITY, 0.0f);
    const float m = wg_max<16>(st.x, wpart);
    const float rs = (tid < nw && st.x > -INFINITY) ? st.y * expf(st.x - m) : 0.0f;
    float sum;
    const float r = sample_uniform(seed, counter + (d_state ? (uint64_t)d_state[2] : 0ull));
    // slice masses rs / sum in slice order: the slice whose running mass
    // first exceeds r
    const float mass = rs;   // scaled by 1/sum below, after the total is known
    float before = wg_excl_scan(mass, wpart, sum);
    int cand = 0x7fffffff;
    if (tid < nw && r < (before + mass) / sum) cand = tid;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) cand = min(cand, __shfl_xor(cand, off, 64));
    if (lane == 0) wmin[w] = cand;
    __syncthreads();
    if (tid == 0) {
        int c = wmin[0];
        for (int k = 1; k < 16; k++) c = min(c, wmin[k]);
        sh_slice = c == 0x7fffffff ? nw - 1 : c;
    }
    __syncthreads();
    const int sl = sh_slice;
    if (tid == sl) sh_off = before / sum;
    __syncthreads();
    // p for the slice with the row max and sum, running sum in index order
    const int i = sl * SMP_SLICE + tid;
    const float p = i < n ? expf(h2f(x[i]) / temperature - m) / sum : 0.0f;
    float tot;
    const float cum = sh_off + wg_excl_scan(p, wpart, tot) + p;
    int found = (i < n && r < cum) ? i : 0x7fffffff;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) found = min(found, __shfl_xor(found, off, 64));
    if (lane == 0) wmin[w] = found;
    __syncthreads();
    if (tid == 0) {
        int f = wmin[0];
        for (int k = 1; k < 16; k++) f = min(f, wmin[k]);
        // past the slice's last logit by rounding: its last index (n - 1 at
        // the row's end, as the reference's default)
        const int tok = f == 0x7fffffff ? min(n, (sl + 1) * SMP_SLICE) - 1 : f;
        if (out) out[0] = tok;
        if (d_state) {
            if (token_log) token_log[d_state[2]] = tok;
            d_state[0] = tok;
            d_state[1] += 1;
            d_state[2] += 1;
        }
    }
}

size_t sample_scratch_bytes(int n) { return sizeof(float2) * (size_t)((n + SMP_SLICE - 1) / SMP_SLICE); }

tlhip_status launch_sample(hipStream_t s, const uint16_t* x, int n, float temperature, uint64_t seed,
                           uint64_t counter, void* scratch, int32_t* out, int32_t* token_log, int32_t* d_state) {
    if (n <= 0) return fail(TLHIP_ERR_INVALID_DIMENSION, "temperature_sample of an empty tensor");
    if (n > SMP_SLICE * SMP_MAXW) return fail(TLHIP_ERR_INVALID_DIMENSION, "temperature_sample: %d logits", n);
    if (!(temperature > 0.0f)) return fail(TLHIP_ERR_INVALID_ARGUMENT, "temperature_sample: temperature %g", temperature);
    const int nw = (n + SMP_SLICE - 1) / SMP_SLICE;
    hipLaunchKernelGGL(sample_stats_kernel, dim3(nw), dim3(256), 0, s, x, n, temperature, (float2*)scratch);
    hipLaunchKernelGGL(sample_pick_kernel, dim3(1), dim3(1024), 0, s, x, n, temperature, seed, counter,
                       (const float2*)scratch, out, token_log, d_state);
    return TLHIP_OK;
}

// Copies rows (e.g. KV-cache set/append): dst row (dst_row0 + *d_pos + r).
__global__ void copy_rows_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                 int rows, int row_elems, int ss, int ds, const int32_t* d_pos,
                                 int dst_row0) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * row_elems) return;
    const int r = (int)(i / row_elems), c = (int)(i % row_elems);
    const int dr = dst_row0 + r + (d_pos ? *d_pos : 0);
    dst[(size_t)dr * ds + c] = src[(size_t)r * ss + c];
}

tlhip_status launch_copy_rows(hipStream_t s, const uint16_t* src, uint16_t* dst, int rows,
                              int row_elems, int src_stride, int dst_stride, const int32_t* d_pos,
                              int dst_row0) {
    int64_t total = (int64_t)rows * row_elems;
    if (total <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(copy_rows_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src,
                       dst, rows, row_elems, src_stride, dst_stride, d_pos, dst_row0);
    return TLHIP_OK;
}

// Plain 16-byte-per-lane copy (measurement reference: the bandwidth a
// streaming kernel reaches on this device, and the scale of the profiler's
// FETCH_SIZE / WRITE_SIZE counters for a known byte count).
__global__ void stream_copy_kernel(const u4* __restrict__ src, u4* __restrict__ dst, size_t n) {
    const size_t step = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) dst[i] = src[i];
}

tlhip_status launch_stream_copy(hipStream_t s, const void* src, void* dst, size_t bytes) {
    const size_t n = bytes / 16;
    if (n == 0) return TLHIP_OK;
    const unsigned grid = (unsigned)std::min<size_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(stream_copy_kernel, dim3(grid), dim3(256), 0, s, (const u4*)src, (u4*)dst, n);
    return TLHIP_OK;
}

// dst[c, r] = src[r, c] for a row-major [rows, cols] f16 matrix.
template <typename T>
__global__ void transpose_kernel(const T* __restrict__ src, T* __restrict__ dst, int rows, int cols) {
    __shared__ T tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 256 threads: 32 x 8
    for (int i = ty; i < 32; i += 8) {
        const int r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) tile[i][tx] = src[(size_t)r * cols + c];
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const int c = c0 + i, r = r0 + tx;
        if (r < rows && c < cols) dst[(size_t)c * rows + r] = tile[tx][i];
    }
}

template <typename T>
static tlhip_status launch_transpose_t(hipStream_t s, const T* src, T* dst, int rows, int cols) {
    if (rows <= 0 || cols <= 0) return TLHIP_OK;
    const unsigned gy = (unsigned)((rows + 31) / 32);
    if (gy > 65535u) return fail(TLHIP_ERR_INVALID_DIMENSION, "transpose: %d rows exceed the launch grid", rows);
    hipLaunchKernelGGL(transpose_kernel<T>, dim3((cols + 31) / 32, gy), dim3(256), 0, s, src, dst, rows, cols);
    return TLHIP_OK;
}

tlhip_status launch_transpose(hipStream_t s, const uint16_t* src, uint16_t* dst, int rows, int cols) {
    return launch_transpose_t(s, src, dst, rows, cols);
}

tlhip_status launch_transpose_f32(hipStream_t s, const float* src, float* dst, int rows, int cols) {
    return launch_transpose_t(s, src, dst, rows, cols);
}

// ---------------------------------------------------------------------------
// general einsum (general_einsum_cpu / sum_over_indices, einsum.rs:207-333)
// on f16 tensors, one thread per output element: the product of the
// operands' elements starts at f16 one and multiplies them in operand order,
// each product rounded to f16; the summed indices nest outermost first, and
// every level keeps its own f16 running sum from +0 of the completed inner
// level's sums (the innermost of the products), each addition rounded to
// f16 -- the reference's recursion.  With no summed index the output is the
// product itself.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint16_t einsum_product(const EinsumPlan& p, const int64_t* off) {
    uint16_t prod = 0x3C00u;
    for (int k = 0; k < p.n_ops; k++) prod = f2h(h2f(prod) * h2f(p.op[k][off[k]]));
    return prod;
}

__global__ __launch_bounds__(256) void einsum_general_kernel(EinsumPlan p, uint16_t* __restrict__ out, int64_t n_out,
                                                             int64_t n_sum) {
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < n_out; o += (int64_t)gridDim.x * 256) {
        int64_t off[EINSUM_MAX_OPS] = {};
        int64_t rem = o;
        for (int d = p.n_out - 1; d >= 0; d--) {
            const int64_t c = rem % p.out_dim[d];
            rem /= p.out_dim[d];
            for (int k = 0; k < p.n_ops; k++) off[k] += c * p.out_stride[k][d];
        }
        uint16_t r;
        if (p.n_sum == 0) {
            r = einsum_product(p, off);
        } else {
            uint16_t acc[EINSUM_MAX_SUM];
            int64_t idx[EINSUM_MAX_SUM];
            for (int d = 0; d < EINSUM_MAX_SUM; d++) {
                acc[d] = 0;
                idx[d] = 0;
            }
            const int last = p.n_sum - 1;
            for (int64_t s = 0; s < n_sum; s++) {
                acc[last] = f2h(h2f(acc[last]) + h2f(einsum_product(p, off)));
                // advance the innermost index; a level that wraps hands its
                // sum to the level outside it
                for (int d = last; d >= 0; d--) {
                    idx[d]++;
                    for (int k = 0; k < p.n_ops; k++) off[k] += p.sum_stride[k][d];
                    if (idx[d] < p.sum_dim[d]) break;
                    for (int k = 0; k < p.n_ops; k++) off[k] -= p.sum_stride[k][d] * p.sum_dim[d];
                    idx[d] = 0;
                    if (d > 0) {
                        acc[d - 1] = f2h(h2f(acc[d - 1]) + h2f(acc[d]));
                        acc[d] = 0;
                    }
                }
            }
            r = acc[0];
        }
        out[o] = r;
    }
}

tlhip_status launch_einsum_general(hipStream_t s, const EinsumPlan& p, uint16_t* out, int64_t n_out, int64_t n_sum) {
    if (n_out <= 0) return TLHIP_OK;
    const int64_t blocks = std::min<int64_t>((n_out + 255) / 256, 65536);
    hipLaunchKernelGGL(einsum_general_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p, out, n_out, n_sum);
    return TLHIP_OK;
}

// ---------------------------------------------------------------------------
// The TensorF32 arms of rms_norm, softmax, rope and sigmoid (f32 in, f32
// out, f32 arithmetic).

// rms_norm_simple_f32 / rms_norm_f32 (unified.metal:1961-2036, dispatched by
// normalization.rs:139-177): the sum of squares in the reference's order --
// rows of n <= 256 by one thread in element order; longer rows as 256
// partial sums (thread t: elements t, t + 256, ...) and then a halving tree,
// partial t adding partial t + stride for stride = 128, 64, ..., 1.  Each
// square joins its partial sum as one fused multiply-add, the contraction
// Metal's default fast math makes of `sum += v * v` (assumed, as for the f32
// linear).  Then rms = sqrt(sum / n + eps) and y = (x * (1 / rms)) * w.
__global__ __launch_bounds__(256) void rms_norm_f32_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           float* __restrict__ y, int n, float eps) {
    __shared__ float part[256];
    const float* xr = x + (size_t)blockIdx.x * n;
    float* yr = y + (size_t)blockIdx.x * n;
    const int t = threadIdx.x;
    if (n <= 256) {
        if (t == 0) {
            float s = 0.0f;
            for (int i = 0; i < n; i++) s = fmaf(xr[i], xr[i], s);
            part[0] = s;
        }
        __syncthreads();
    } else {
        float s = 0.0f;
        for (int i = t; i < n; i += 256) s = fmaf(xr[i], xr[i], s);
        part[t] = s;
        __syncthreads();
        for (int st = 128; st > 0; st >>= 1) {
            if (t < st) part[t] = part[t] + part[t + st];
            __syncthreads();
        }
    }
    const float mean_sq = part[0] / (float)n;
    const float rms = sqrtf(mean_sq + eps);
    const float inv = 1.0f / rms;
    for (int i = t; i < n; i += 256) yr[i] = (xr[i] * inv) * w[i];
}

tlhip_status launch_rms_norm_f32(hipStream_t s, const float* x, const float* w, float* y, int rows, int n, float eps) {
    if (rows <= 0 || n <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(rms_norm_f32_kernel, dim3((unsigned)rows), dim3(256), 0, s, x, w, y, n, eps);
    return TLHIP_OK;
}

// softmax_simple_f32 / softmax_f32 (unified.metal:2202-2340; both run one
// thread per row, activations.rs:155-209): max over the finite values (0 if
// none), e = exp(x - max) (0 for a non-finite x), y = e / sum, or 1/n
// everywhere when the sum is not a positive finite number.  The max and the
// exponentials are spread over the workgroup; the sum is taken in element
// order by one thread, as the reference's: a tree sum drifts from that
// running f32 sum by ~20 ulps at 1000 elements.
__global__ __launch_bounds__(256) void softmax_f32_kernel(const float* __restrict__ x, float* __restrict__ y, int n) {
    __shared__ float red[4];
    __shared__ float total;
    const float* xr = x + (size_t)blockIdx.x * n;
    float* yr = y + (size_t)blockIdx.x * n;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = xr[i];
        if (isfinite(v)) mx = fmaxf(mx, v);
    }
    mx = block_max256(mx, red);
    if (!isfinite(mx)) mx = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = xr[i];
        yr[i] = isfinite(v) ? expf(v - mx) : 0.0f;
    }
    __syncthreads();   // (the block's global writes are visible to thread 0 after it)
    if (threadIdx.x == 0) {
        float s = 0.0f;
        for (int i = 0; i < n; i++) s += yr[i];
        total = s;
    }
    __syncthreads();
    const float sum = total;
    if (sum > 0.0f && isfinite(sum)) {
        for (int i = threadIdx.x; i < n; i += 256) yr[i] = yr[i] / sum;
    } else {
        const float u = 1.0f / (float)n;
        for (int i = threadIdx.x; i < n; i += 256) yr[i] = u;
    }
}

tlhip_status launch_softmax_f32(hipStream_t s, const float* x, float* y, int64_t rows, int n) {
    if (rows <= 0 || n <= 0) return TLHIP_OK;
    if (rows > 0x7fffffff) return fail(TLHIP_ERR_INVALID_DIMENSION, "softmax: %lld rows", (long long)rows);
    hipLaunchKernelGGL(softmax_f32_kernel, dim3((unsigned)rows), dim3(256), 0, s, x, y, n);
    return TLHIP_OK;
}

// rope_f32 (unified.metal:2420-2482): rope_kernel's indexing, table and
// rotation (rope_pair, separately rounded products) with f32 rows in and
// out.
__global__ void rope_f32_kernel(const float* __restrict__ x, float* __restrict__ y, int S, int H, int D, int64_t batch,
                                int offset, int layout, int rot, const float* __restrict__ table) {
    const int half = rot / 2;
    const int64_t per_row = (int64_t)H * (D - half);
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= batch * S * per_row) return;
    const int64_t row = idx / per_row, rem = idx % per_row;
    const int h = (int)(rem / (D - half)), e = (int)(rem % (D - half));
    const int pos = offset + (int)(row % S);
    const float* xr = x + ((size_t)row * H + h) * D;
    float* yr = y + ((size_t)row * H + h) * D;
    if (e < half) {
        int i0, i1;
        rope_indices(layout, e, half, i0, i1);
        const float c = table[2 * ((size_t)pos * half + e)], sn = table[2 * ((size_t)pos * half + e) + 1];
        float r0, r1;
        rope_pair(xr[i0], xr[i1], c, sn, r0, r1);
        yr[i0] = r0;
        yr[i1] = r1;
    } else {
        const int d = rot + (e - half);
        yr[d] = xr[d];
    }
}

tlhip_status launch_rope_f32(hipStream_t s, const float* x, float* y, int S, int H, int D, int64_t batch, int offset,
                             int layout, int rot_dims, const float* table) {
    const int64_t total = batch * S * (int64_t)H * (D - rot_dims / 2);
    if (total <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(rope_f32_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x, y, S, H, D, batch,
                       offset, layout, rot_dims, table);
    return TLHIP_OK;
}

// sigmoid_f32 (unified.metal:1129-1135): 1 / (1 + exp(-x)).
__global__ void sigmoid_f32_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = 1.0f / (1.0f + expf(-x[i]));
}

tlhip_status launch_sigmoid_f32(hipStream_t s, const float* x, float* y, int64_t n) {
    if (n <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(sigmoid_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
    return TLHIP_OK;
}

// The TensorF32 elementwise ops: add_f32 / mul_f32 / mul_scalar_f32
// (unified.metal:934-992, one IEEE f32 operation each; b may repeat every
// bp elements as in the f16 kernel), silu = x * sigmoid_f32(x) and
// silu(g) * u with every step rounded to f32 (the TL functions, as the
// f16 kernel), and gelu_f32 (unified.metal:1051-1062): x3 = x * x * x,
// inner = sqrt(2/pi) * (x + 0.044715 * x3) with the multiply-add fused (the
// contraction assumed for the reference's f32 kernels), 0.5 * x * (1 +
// tanh(inner)).
__device__ __forceinline__ float sigmoid_f(float v) { return 1.0f / (1.0f + expf(-v)); }
__device__ __forceinline__ float gelu_f(float x) {
    const float x3 = __fmul_rn(__fmul_rn(x, x), x);
    const float inner = __fmul_rn(0.7978845608f, fmaf(0.044715f, x3, x));
    return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, tanhf(inner)));
}

__global__ void elementwise_f32_kernel(int op, const float* __restrict__ a, const float* __restrict__ b,
                                       float* __restrict__ y, int64_t n, int64_t bp, float sc) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float av = a[i];
    float r;
    switch (op) {
        case EW_SIGMOID: r = sigmoid_f(av); break;
        case EW_SILU: r = __fmul_rn(av, sigmoid_f(av)); break;
        case EW_GELU: r = gelu_f(av); break;
        case EW_ADD: r = __fadd_rn(av, b[bp ? i % bp : i]); break;
        case EW_MUL: r = __fmul_rn(av, b[bp ? i % bp : i]); break;
        case EW_MUL_SCALAR: r = __fmul_rn(av, sc); break;
        case EW_SILU_MUL: r = __fmul_rn(__fmul_rn(av, sigmoid_f(av)), b[i]); break;
        default: r = av;
    }
    y[i] = r;
}

tlhip_status launch_elementwise_f32(hipStream_t s, int op, const float* a, const float* b, float* y, int64_t n,
                                    int64_t b_period, float scalar) {
    if (n <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(elementwise_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, op, a, b, y, n,
                       b_period, scalar);
    return TLHIP_OK;
}

// layer_norm_f32 / layer_norm_simple_f32 (unified.metal:1833-1958,
// dispatched by normalization.rs:396-441) per row: sum in element order,
// mean = sum / n; the squared deviations summed in element order, each as
// one fused multiply-add (the contraction assumed for `sq_sum += diff *
// diff`); inv_std = 1 / sqrt(sq_sum / n + eps); y = (x - mean) * inv_std,
// then * w and + b (fused into one multiply-add when both are given).
// Element order is what the reference's dispatch computes for a single row
// (one thread) and for rows of at most 256 (the simple kernel); its
// multi-row dispatch of the long-row kernel shares one threadgroup between
// rows, which this restates per row.  Thread 0 takes both sums; every
// thread normalises.
__global__ __launch_bounds__(256) void layer_norm_f32_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                             const float* __restrict__ b, float* __restrict__ y,
                                                             int n, float eps) {
    __shared__ float stat[2];
    const float* xr = x + (size_t)blockIdx.x * n;
    float* yr = y + (size_t)blockIdx.x * n;
    if (threadIdx.x == 0) {
        float s = 0.0f;
        for (int i = 0; i < n; i++) s = __fadd_rn(s, xr[i]);
        const float mean = s / (float)n;
        float q = 0.0f;
        for (int i = 0; i < n; i++) {
            const float d = __fsub_rn(xr[i], mean);
            q = fmaf(d, d, q);
        }
        stat[0] = mean;
        stat[1] = 1.0f / sqrtf(__fadd_rn(q / (float)n, eps));
    }
    __syncthreads();
    const float mean = stat[0], inv_std = stat[1];
    for (int i = threadIdx.x; i < n; i += 256) {
        const float t = __fmul_rn(__fsub_rn(xr[i], mean), inv_std);
        float v;
        if (w && b) v = fmaf(t, w[i], b[i]);
        else if (w) v = __fmul_rn(t, w[i]);
        else if (b) v = __fadd_rn(t, b[i]);
        else v = t;
        yr[i] = v;
    }
}

tlhip_status launch_layer_norm_f32(hipStream_t s, const float* x, const float* w, const float* b, float* y, int rows,
                                   int n, float eps) {
    if (rows <= 0 || n <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(layer_norm_f32_kernel, dim3((unsigned)rows), dim3(256), 0, s, x, w, b, y, n, eps);
    return TLHIP_OK;
}

// apply_attention_mask_f32 (unified.metal:4491-4503): y = mask == 0 ?
// -10000 : score (-0 counts as 0, NaN keeps the score), with mask_kernel's
// two mask layouts.
__global__ void mask_f32_kernel(const float* __restrict__ sc, const float* __restrict__ mask, float* __restrict__ y,
                                int64_t n, int64_t period, int64_t inner, int64_t heads) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t mi;
    if (heads > 1) {
        const int64_t j = i % inner, row = (i / inner) / heads;
        mi = row * inner + j;
    } else {
        mi = i % period;
    }
    y[i] = mask[mi] == 0.0f ? -10000.0f : sc[i];
}

tlhip_status launch_mask_f32(hipStream_t s, const float* sc, const float* mask, float* y, int64_t n,
                             int64_t mask_period) {
    if (n <= 0) return TLHIP_OK;
    int64_t period = mask_period, inner = 1, heads = 1;
    if (mask_period < 0) {
        const int64_t enc = -mask_period;
        inner = enc >> 16;
        heads = enc & 0xffff;
        period = 0;
    }
    hipLaunchKernelGGL(mask_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, sc, mask, y, n, period,
                       inner, heads);
    return TLHIP_OK;
}

// embedding_lookup_f32 (unified.metal:678-694): out[s, :] = table[id_s, :]
// for an f32 table, four floats per thread where the rows allow.
__global__ void embedding_f32_kernel(const float* __restrict__ table, const int32_t* __restrict__ ids,
                                     float* __restrict__ out, int n, int hidden, int vec) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec) {
        const int q = hidden / 4;
        if (i >= (int64_t)n * q) return;
        const int s = (int)(i / q), c = (int)(i % q);
        ((float4*)out)[i] = ((const float4*)table)[(size_t)ids[s] * q + c];
    } else {
        if (i >= (int64_t)n * hidden) return;
        const int s = (int)(i / hidden), c = (int)(i % hidden);
        out[i] = table[(size_t)ids[s] * hidden + c];
    }
}

tlhip_status launch_embedding_f32(hipStream_t s, const float* table, const int32_t* ids, float* out, int n,
                                  int hidden) {
    const bool vec = hidden % 4 == 0 && ((uintptr_t)table | (uintptr_t)out) % 16 == 0;
    const int64_t total = (int64_t)n * (vec ? hidden / 4 : hidden);
    if (total <= 0) return TLHIP_OK;
    hipLaunchKernelGGL(embedding_f32_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, table, ids, out,
                       n, hidden, vec ? 1 : 0);
    return TLHIP_OK;
}

}  // namespace tlhip
