/*
 * tl_oracle.c -- CPU restatement of TensorLogic's quantized-LLM hot path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and timed CPU baseline); the
 * product never links or calls this file.  Declarations and the reference
 * file:line each function follows are in tl_oracle.h.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).  Floating
 * point contraction is off so every multiply and add rounds exactly where
 * the reference's scalar code rounds.
 */
#define _GNU_SOURCE
#include "tl_oracle.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ======================================================================== */
/* binary16 <-> binary32                                                    */
/* ======================================================================== */

static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float tlo_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return bits_f(sign);
        /* subnormal: value = m * 2^-24, renormalise */
        uint32_t ee = 113;            /* exponent of 2^-14 in f32 bias */
        while (!(m & 0x400u)) { m <<= 1; ee--; }
        m &= 0x3ffu;
        return bits_f(sign | (ee << 23) | (m << 13));
    }
    if (e == 31) return bits_f(sign | 0x7f800000u | (m << 13));
    return bits_f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t tlo_f2h(float f) {
    uint32_t x = f_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                      /* below 2^-14 */
        if (ax < 0x33000000u) return sign;                       /* below 2^-25 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;                               /* 14..24 */
        uint32_t r = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ax - 0x38000000u;
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

void tlo_h2f_array(const uint16_t* h, float* f, size_t n) {
    for (size_t i = 0; i < n; i++) f[i] = tlo_h2f(h[i]);
}
void tlo_f2h_array(const float* f, uint16_t* h, size_t n) {
    for (size_t i = 0; i < n; i++) h[i] = tlo_f2h(f[i]);
}

/* f16 -> f32 lookup table for the hot loops (exactly tlo_h2f). */
static float g_h2f_lut[65536];
static int g_lut_ready = 0;
static void lut_init(void) {
    if (g_lut_ready) return;
    for (uint32_t i = 0; i < 65536u; i++) g_h2f_lut[i] = tlo_h2f((uint16_t)i);
    g_lut_ready = 1;
}
#define H2F(h) (g_h2f_lut[(uint16_t)(h)])

/* ======================================================================== */
/* GGUF block dequantisation  (gguf.rs:22-112, mmap_gguf.rs:383-439)        */
/* ======================================================================== */

void tlo_dequant_q4_0(const uint8_t* blocks, size_t nblocks, uint16_t* out) {
    lut_init();
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = blocks + b * 18;
        float d = H2F((uint16_t)(blk[0] | (blk[1] << 8)));
        uint16_t* o = out + b * 32;
        for (int j = 0; j < 16; j++) {
            uint8_t byte = blk[2 + j];
            float x0 = (float)((int)(byte & 0x0f) - 8);
            float x1 = (float)((int)(byte >> 4) - 8);
            o[j] = tlo_f2h(x0 * d);
            o[j + 16] = tlo_f2h(x1 * d);
        }
    }
}

void tlo_dequant_q8_0(const uint8_t* blocks, size_t nblocks, uint16_t* out) {
    lut_init();
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = blocks + b * 34;
        float d = H2F((uint16_t)(blk[0] | (blk[1] << 8)));
        uint16_t* o = out + b * 32;
        for (int j = 0; j < 32; j++) {
            float q = (float)(int8_t)blk[2 + j];   /* exact in f16 */
            o[j] = tlo_f2h(q * d);
        }
    }
}

/* Q6_K: 256-element super-blocks of 210 bytes, ql[128] qh[64] sc[16] d, as
 * gguf.rs:128-212 / mmap_gguf.rs:457-545 walk them: for each 128-element
 * half n and l < 32 the four values
 *   q1 = ql[l]    low  | qh[l] bits 0-1 << 4   -> y[l]       scale sc[is]
 *   q2 = ql[l+32] low  | qh[l] bits 2-3 << 4   -> y[l + 32]  scale sc[is + 2]
 *   q3 = ql[l]    high | qh[l] bits 4-5 << 4   -> y[l + 64]  scale sc[is + 4]
 *   q4 = ql[l+32] high | qh[l] bits 6-7 << 4   -> y[l + 96]  scale sc[is + 6]
 * with is = l / 16, each value f16(d * sc * (q - 32)) in f32 (d * sc first),
 * and ql += 64, qh += 32, sc += 8 per half.                                */
void tlo_dequant_q6_k(const uint8_t* blocks, size_t nblocks, uint16_t* out) {
    lut_init();
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = blocks + b * 210;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        const float d = H2F((uint16_t)(blk[208] | (blk[209] << 8)));
        uint16_t* y = out + b * 256;
        for (int n = 0; n < 2; n++) {
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l] = tlo_f2h(d * (float)sc[is + 0] * (float)q1);
                y[l + 32] = tlo_f2h(d * (float)sc[is + 2] * (float)q2);
                y[l + 64] = tlo_f2h(d * (float)sc[is + 4] * (float)q3);
                y[l + 96] = tlo_f2h(d * (float)sc[is + 6] * (float)q4);
            }
            y += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

/* ======================================================================== */
/* linear (matmul_transposed_b)                                             */
/* ======================================================================== */

/* fp32 accumulation in k order: matmul_transposed_b_tiled_32x32_f16
 * (unified.metal:4291-4348) sums float(a)*float(b) tile by tile in k order. */
static float dot_f32acc(const float* a, const float* b, int K) {
    float s = 0.0f;
    for (int k = 0; k < K; k++) s += a[k] * b[k];
    return s;
}

/* TLO_ACC_F32_REV: the same sum in descending k -- a second fp32 order */
static float dot_f32acc_rev(const float* a, const float* b, int K) {
    float s = 0.0f;
    for (int k = K - 1; k >= 0; k--) s += a[k] * b[k];
    return s;
}

/* f16 accumulation: matmul_cpu (matmul.rs:201-228), `sum += a * b` on
 * half::f16 -- the product is rounded to f16, then the sum is.             */
static uint16_t dot_f16acc(const float* a, const float* b, int K) {
    uint16_t s = 0;
    for (int k = 0; k < K; k++) {
        uint16_t p = tlo_f2h(a[k] * b[k]);
        s = tlo_f2h(H2F(s) + H2F(p));
    }
    return s;
}

static void linear_rows_f32w(const float* xf, const float* wf, const uint16_t* bias,
                             int M, int N, int K, int acc_mode, uint16_t* y) {
    #pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        const float* wr = wf + (size_t)n * K;
        for (int m = 0; m < M; m++) {
            uint16_t r = (acc_mode == TLO_ACC_F16)       ? dot_f16acc(xf + (size_t)m * K, wr, K)
                         : (acc_mode == TLO_ACC_F32_REV) ? tlo_f2h(dot_f32acc_rev(xf + (size_t)m * K, wr, K))
                                                         : tlo_f2h(dot_f32acc(xf + (size_t)m * K, wr, K));
            if (bias) r = tlo_f2h(H2F(r) + H2F(bias[n]));
            y[(size_t)m * N + n] = r;
        }
    }
}

void tlo_linear_f32(const float* x, const float* w, const float* bias, int M, int N, int K, float* y) {
    const int kp = (K + 31) / 32 * 32;   /* the kernel's 32-wide tiles, zero-padded */
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float sum = 0.0f;
            for (int k = 0; k < kp; k++) {
                const float a = k < K ? x[(size_t)m * K + k] : 0.0f;
                const float b = k < K ? w[(size_t)n * K + k] : 0.0f;
                sum = fmaf(a, b, sum);
            }
            y[(size_t)m * N + n] = bias ? sum + bias[n] : sum;
        }
}

void tlo_linear_f16(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                    int M, int N, int K, int acc_mode, uint16_t* y) {
    lut_init();
    float* xf = (float*)malloc(sizeof(float) * (size_t)M * K);
    float* wf = (float*)malloc(sizeof(float) * (size_t)N * K);
    for (size_t i = 0; i < (size_t)M * K; i++) xf[i] = H2F(x[i]);
    for (size_t i = 0; i < (size_t)N * K; i++) wf[i] = H2F(w[i]);
    linear_rows_f32w(xf, wf, bias, M, N, K, acc_mode, y);
    free(xf);
    free(wf);
}

/* nblocks counts 32-element units (Q6_K: eight per 210-byte super-block) */
static void dequant_any(const uint8_t* blocks, int wtype, size_t nblocks, uint16_t* out) {
    if (wtype == 2) tlo_dequant_q4_0(blocks, nblocks, out);
    else if (wtype == 14) tlo_dequant_q6_k(blocks, nblocks / 8, out);
    else tlo_dequant_q8_0(blocks, nblocks, out);
}

void tlo_linear_q(const uint16_t* x, const uint8_t* wblocks, int wtype,
                  const uint16_t* bias, int M, int N, int K, int acc_mode,
                  uint16_t* y) {
    lut_init();
    size_t nblk = (size_t)N * K / 32;
    uint16_t* wh = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)N * K);
    dequant_any(wblocks, wtype, nblk, wh);
    tlo_linear_f16(x, wh, bias, M, N, K, acc_mode, y);
    free(wh);
}

/* ======================================================================== */
/* normalisation                                                            */
/* ======================================================================== */

void tlo_rms_norm(const uint16_t* x, const uint16_t* w, int rows, int n,
                  float eps, uint16_t* y) {
    lut_init();
    for (int r = 0; r < rows; r++) {
        const uint16_t* xr = x + (size_t)r * n;
        float sq = 0.0f;
        for (int i = 0; i < n; i++) { float v = H2F(xr[i]); sq += v * v; }
        float mean_sq = sq / (float)n;
        float rms = sqrtf(mean_sq + eps);
        float inv = 1.0f / rms;
        for (int i = 0; i < n; i++) {
            float nv = H2F(xr[i]) * inv;
            float sv = nv * H2F(w[i]);
            y[(size_t)r * n + i] = tlo_f2h(sv);
        }
    }
}

void tlo_layer_norm(const uint16_t* x, const uint16_t* w, const uint16_t* b,
                    int rows, int n, float eps, uint16_t* y) {
    lut_init();
    for (int r = 0; r < rows; r++) {
        const uint16_t* xr = x + (size_t)r * n;
        float s = 0.0f;
        for (int i = 0; i < n; i++) s += H2F(xr[i]);
        float mean = s / (float)n;
        float sq = 0.0f;
        for (int i = 0; i < n; i++) { float d = H2F(xr[i]) - mean; sq += d * d; }
        float var = sq / (float)n;
        float inv_std = 1.0f / sqrtf(var + eps);
        for (int i = 0; i < n; i++) {
            float v = (H2F(xr[i]) - mean) * inv_std;
            if (w) v = v * H2F(w[i]);
            if (b) v = v + H2F(b[i]);
            y[(size_t)r * n + i] = tlo_f2h(v);
        }
    }
}

/* ======================================================================== */
/* RoPE                                                                     */
/* ======================================================================== */

void tlo_rope_table(int max_pos, int rot_dims, float theta, float* cs) {
    int half = rot_dims / 2;
    for (int i = 0; i < half; i++) {
        float expo = (float)(2 * i) / (float)rot_dims;
        float freq = 1.0f / powf(theta, expo);
        for (int p = 0; p < max_pos; p++) {
            float ang = (float)p * freq;
            cs[2 * ((size_t)p * half + i) + 0] = (float)cos((double)ang);
            cs[2 * ((size_t)p * half + i) + 1] = (float)sin((double)ang);
        }
    }
}

void tlo_rope(const uint16_t* x, int S, int H, int D, int offset, float theta,
              int layout, int rot_dims, uint16_t* y) {
    lut_init();
    if (rot_dims <= 0 || rot_dims > D) rot_dims = D;
    int half = rot_dims / 2;
    float* cs = (float*)malloc(sizeof(float) * 2 * (size_t)half);
    for (int s = 0; s < S; s++) {
        int pos = offset + s;
        for (int i = 0; i < half; i++) {
            float expo = (float)(2 * i) / (float)rot_dims;
            float freq = 1.0f / powf(theta, expo);
            float ang = (float)pos * freq;
            cs[2 * i + 0] = (float)cos((double)ang);
            cs[2 * i + 1] = (float)sin((double)ang);
        }
        for (int h = 0; h < H; h++) {
            const uint16_t* xr = x + ((size_t)s * H + h) * D;
            uint16_t* yr = y + ((size_t)s * H + h) * D;
            for (int d = rot_dims; d < D; d++) yr[d] = xr[d];
            for (int i = 0; i < half; i++) {
                int i0, i1;
                if (layout == TLO_ROPE_INTERLEAVED) { i0 = 2 * i; i1 = 2 * i + 1; }
                else { i0 = i; i1 = i + half; }
                float c = cs[2 * i], sn = cs[2 * i + 1];
                float x0 = H2F(xr[i0]), x1 = H2F(xr[i1]);
                float a = x0 * c, bb = x1 * sn;
                float r0 = a - bb;
                float e = x0 * sn, f = x1 * c;
                float r1 = e + f;
                yr[i0] = tlo_f2h(r0);
                yr[i1] = tlo_f2h(r1);
            }
        }
    }
    free(cs);
}

/* ======================================================================== */
/* softmax / elementwise                                                    */
/* ======================================================================== */

static void softmax_row(const uint16_t* x, int n, uint16_t* y) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) { float v = H2F(x[i]); if (isfinite(v)) mx = fmaxf(mx, v); }
    if (!isfinite(mx)) mx = 0.0f;
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        float v = H2F(x[i]);
        float e = isfinite(v) ? expf(v - mx) : 0.0f;
        y[i] = tlo_f2h(e);
        sum += e;
    }
    if (sum > 0.0f && isfinite(sum)) {
        for (int i = 0; i < n; i++) y[i] = tlo_f2h(H2F(y[i]) / sum);
    } else {
        uint16_t u = tlo_f2h(1.0f / (float)n);
        for (int i = 0; i < n; i++) y[i] = u;
    }
}

void tlo_softmax(const uint16_t* x, int rows, int n, uint16_t* y) {
    lut_init();
    for (int r = 0; r < rows; r++) softmax_row(x + (size_t)r * n, n, y + (size_t)r * n);
}

static inline uint16_t sigmoid_h(uint16_t x) {
    float v = H2F(x);
    return tlo_f2h(1.0f / (1.0f + expf(-v)));
}

void tlo_sigmoid(const uint16_t* x, size_t n, uint16_t* y) {
    lut_init();
    for (size_t i = 0; i < n; i++) y[i] = sigmoid_h(x[i]);
}

/* ======================================================================== */
/* the TensorF32 arms: f32 in, f32 out, f32 arithmetic                      */
/* ======================================================================== */

/* rms_norm_simple_f32 / rms_norm_f32 (unified.metal:1961-2036; dispatch
   normalization.rs:139-177): rows of n <= 256 summed by one thread in
   element order, longer rows as 256 partial sums (thread t: elements t,
   t + 256, ...) reduced by a halving tree (partial t += partial t + stride,
   stride 128 .. 1).  Each square joins its sum as one fused multiply-add,
   the contraction Metal's default fast math makes of `sum += v * v`
   (assumed, as in tlo_linear_f32).  rms = sqrt(sum / n + eps),
   y = (x * (1 / rms)) * w. */
void tlo_rms_norm_f32(const float* x, const float* w, int rows, int n, float eps, float* y) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * n;
        float sq;
        if (n <= 256) {
            sq = 0.0f;
            for (int i = 0; i < n; i++) sq = fmaf(xr[i], xr[i], sq);
        } else {
            float part[256];
            for (int t = 0; t < 256; t++) {
                float s = 0.0f;
                for (int i = t; i < n; i += 256) s = fmaf(xr[i], xr[i], s);
                part[t] = s;
            }
            for (int st = 128; st > 0; st >>= 1)
                for (int t = 0; t < st; t++) part[t] = part[t] + part[t + st];
            sq = part[0];
        }
        const float mean_sq = sq / (float)n;
        const float rms = sqrtf(mean_sq + eps);
        const float inv = 1.0f / rms;
        for (int i = 0; i < n; i++) {
            const float nv = xr[i] * inv;
            y[(size_t)r * n + i] = nv * w[i];
        }
    }
}

/* softmax_simple_f32 / softmax_f32 (unified.metal:2202-2340; both run as
   one thread per row, activations.rs:155-209): max over the finite values
   (0 if none), e = exp(x - max) (0 for a non-finite x), sum in element
   order, y = e / sum, or 1/n everywhere when the sum is not a positive
   finite number. */
void tlo_softmax_f32(const float* x, int rows, int n, float* y) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * n;
        float* yr = y + (size_t)r * n;
        float mx = -INFINITY;
        for (int i = 0; i < n; i++) if (isfinite(xr[i])) mx = fmaxf(mx, xr[i]);
        if (!isfinite(mx)) mx = 0.0f;
        float sum = 0.0f;
        for (int i = 0; i < n; i++) {
            const float e = isfinite(xr[i]) ? expf(xr[i] - mx) : 0.0f;
            yr[i] = e;
            sum += e;
        }
        if (sum > 0.0f && isfinite(sum)) {
            for (int i = 0; i < n; i++) yr[i] = yr[i] / sum;
        } else {
            const float u = 1.0f / (float)n;
            for (int i = 0; i < n; i++) yr[i] = u;
        }
    }
}

/* rope_f32 (unified.metal:2420-2482): tlo_rope's angles and rotation with
   f32 rows in and out. */
void tlo_rope_f32(const float* x, int S, int H, int D, int offset, float theta, int layout, int rot_dims, float* y) {
    if (rot_dims <= 0 || rot_dims > D) rot_dims = D;
    const int half = rot_dims / 2;
    float* cs = (float*)malloc(sizeof(float) * 2 * (size_t)(half > 0 ? half : 1));
    for (int s = 0; s < S; s++) {
        const int pos = offset + s;
        for (int i = 0; i < half; i++) {
            const float expo = (float)(2 * i) / (float)rot_dims;
            const float freq = 1.0f / powf(theta, expo);
            const float ang = (float)pos * freq;
            cs[2 * i + 0] = (float)cos((double)ang);
            cs[2 * i + 1] = (float)sin((double)ang);
        }
        for (int h = 0; h < H; h++) {
            const float* xr = x + ((size_t)s * H + h) * D;
            float* yr = y + ((size_t)s * H + h) * D;
            for (int d = rot_dims; d < D; d++) yr[d] = xr[d];
            for (int i = 0; i < half; i++) {
                int i0, i1;
                if (layout == TLO_ROPE_INTERLEAVED) { i0 = 2 * i; i1 = 2 * i + 1; }
                else { i0 = i; i1 = i + half; }
                const float c = cs[2 * i], sn = cs[2 * i + 1];
                const float x0 = xr[i0], x1 = xr[i1];
                const float a = x0 * c, bb = x1 * sn, e = x0 * sn, f = x1 * c;
                yr[i0] = a - bb;
                yr[i1] = e + f;
            }
        }
    }
    free(cs);
}

/* sigmoid_f32 (unified.metal:1129-1135) */
void tlo_sigmoid_f32(const float* x, size_t n, float* y) {
    for (size_t i = 0; i < n; i++) y[i] = 1.0f / (1.0f + expf(-x[i]));
}

/* layer_norm_f32 / layer_norm_simple_f32 (unified.metal:1833-1958;
   dispatch normalization.rs:396-441), per row: sum in element order, mean =
   sum / n; squared deviations summed in element order, each as one fused
   multiply-add (the contraction assumed for `sq_sum += diff * diff`, as in
   tlo_rms_norm_f32); inv_std = 1 / sqrt(sq_sum / n + eps); y = (x - mean) *
   inv_std, then * w and + b, fused into one multiply-add when both are
   given.  Element order is what the reference computes for one row (its
   long-row kernel then runs as one thread) and for rows of <= 256 (the
   simple kernel). */
void tlo_layer_norm_f32(const float* x, const float* w, const float* b, int rows, int n, float eps, float* y) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * n;
        float* yr = y + (size_t)r * n;
        float s = 0.0f;
        for (int i = 0; i < n; i++) s += xr[i];
        const float mean = s / (float)n;
        float q = 0.0f;
        for (int i = 0; i < n; i++) {
            const float d = xr[i] - mean;
            q = fmaf(d, d, q);
        }
        const float inv_std = 1.0f / sqrtf(q / (float)n + eps);
        for (int i = 0; i < n; i++) {
            const float t = (xr[i] - mean) * inv_std;
            if (w && b) yr[i] = fmaf(t, w[i], b[i]);
            else if (w) yr[i] = t * w[i];
            else if (b) yr[i] = t + b[i];
            else yr[i] = t;
        }
    }
}

/* gelu_f32 (unified.metal:1051-1062): x3 = (x * x) * x, inner = sqrt(2/pi)
   * (x + 0.044715 * x3) with the multiply-add fused (assumed contraction),
   y = (0.5 * x) * (1 + tanh(inner)). */
void tlo_gelu_f32(const float* x, size_t n, float* y) {
    for (size_t i = 0; i < n; i++) {
        const float v = x[i];
        const float x3 = (v * v) * v;
        const float inner = 0.7978845608f * fmaf(0.044715f, x3, v);
        y[i] = (0.5f * v) * (1.0f + tanhf(inner));
    }
}

/* TL silu(x) = x * sigmoid(x) and swiglu(g, u) = silu(g) * u on f32
   tensors: sigmoid_f32, then mul_f32 (each step rounded to f32). */
void tlo_silu_f32(const float* x, size_t n, float* y) {
    for (size_t i = 0; i < n; i++) {
        const float s = 1.0f / (1.0f + expf(-x[i]));
        y[i] = x[i] * s;
    }
}

void tlo_swiglu_f32(const float* g, const float* u, size_t n, float* y) {
    for (size_t i = 0; i < n; i++) {
        const float s = 1.0f / (1.0f + expf(-g[i]));
        const float a = g[i] * s;
        y[i] = a * u[i];
    }
}

/* einsum_ihd_jhd_ihj_f32 / einsum_ihj_jhd_ihd_f32 (unified.metal:2702-2768):
   the sum over d (scores) or j (context) in index order, one fused
   multiply-add per term; query head h reads KV head h / (H / Hkv). */
void tlo_einsum_scores_f32(const float* q, const float* k, int I, int J, int H, int Hkv, int D, float* out) {
    const int group = H / Hkv;
    for (int i = 0; i < I; i++)
        for (int h = 0; h < H; h++) {
            const float* qr = q + ((size_t)i * H + h) * D;
            for (int j = 0; j < J; j++) {
                const float* kr = k + ((size_t)j * Hkv + h / group) * D;
                float sum = 0.0f;
                for (int d = 0; d < D; d++) sum = fmaf(qr[d], kr[d], sum);
                out[((size_t)i * H + h) * J + j] = sum;
            }
        }
}

void tlo_einsum_context_f32(const float* p, const float* v, int I, int J, int H, int Hkv, int D, float* out) {
    const int group = H / Hkv;
    for (int i = 0; i < I; i++)
        for (int h = 0; h < H; h++) {
            const float* pr = p + ((size_t)i * H + h) * J;
            for (int d = 0; d < D; d++) {
                float sum = 0.0f;
                for (int j = 0; j < J; j++) sum = fmaf(pr[j], v[((size_t)j * Hkv + h / group) * D + d], sum);
                out[((size_t)i * H + h) * D + d] = sum;
            }
        }
}

void tlo_silu(const uint16_t* x, size_t n, uint16_t* y) {
    lut_init();
    for (size_t i = 0; i < n; i++) {
        uint16_t s = sigmoid_h(x[i]);
        y[i] = tlo_f2h(H2F(x[i]) * H2F(s));
    }
}

void tlo_add(const uint16_t* a, const uint16_t* b, size_t n, uint16_t* y) {
    lut_init();
    for (size_t i = 0; i < n; i++) y[i] = tlo_f2h(H2F(a[i]) + H2F(b[i]));
}

void tlo_mul(const uint16_t* a, const uint16_t* b, size_t n, uint16_t* y) {
    lut_init();
    for (size_t i = 0; i < n; i++) y[i] = tlo_f2h(H2F(a[i]) * H2F(b[i]));
}

void tlo_mul_scalar(const uint16_t* a, float s, size_t n, uint16_t* y) {
    lut_init();
    float sh = H2F(tlo_f2h(s));   /* the scalar is an f16 operand */
    for (size_t i = 0; i < n; i++) y[i] = tlo_f2h(H2F(a[i]) * sh);
}

void tlo_swiglu(const uint16_t* g, const uint16_t* u, size_t n, uint16_t* y) {
    lut_init();
    for (size_t i = 0; i < n; i++) {
        uint16_t s = sigmoid_h(g[i]);
        uint16_t a = tlo_f2h(H2F(g[i]) * H2F(s));
        y[i] = tlo_f2h(H2F(a) * H2F(u[i]));
    }
}

void tlo_gelu(const uint16_t* x, size_t n, uint16_t* y) {
    lut_init();
    const float c0 = 0.7978845608f, c1 = 0.044715f;
    for (size_t i = 0; i < n; i++) {
        float v = H2F(x[i]);
        float x3 = (v * v) * v;
        float inner = c0 * (v + c1 * x3);
        float r = (0.5f * v) * (1.0f + tanhf(inner));
        y[i] = tlo_f2h(r);
    }
}

/* ======================================================================== */
/* attention                                                                */
/* ======================================================================== */

void tlo_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                   int S, int J, int H, int Hkv, int D, int q_pos0,
                   float scale, int causal, int acc_mode, uint16_t* out) {
    lut_init();
    int group = H / Hkv;
    float scale_h = H2F(tlo_f2h(scale));
    #pragma omp parallel
    {
        uint16_t* sc = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)J);
        uint16_t* p = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)J);
        float* qf = (float*)malloc(sizeof(float) * (size_t)D);
        #pragma omp for schedule(static) collapse(2)
        for (int s = 0; s < S; s++) {
            for (int h = 0; h < H; h++) {
                int kvh = h / group;
                const uint16_t* qr = q + ((size_t)s * H + h) * D;
                for (int d = 0; d < D; d++) qf[d] = H2F(qr[d]);
                int qpos = q_pos0 + s;
                for (int j = 0; j < J; j++) {
                    const uint16_t* kr = k + ((size_t)j * Hkv + kvh) * D;
                    float acc = 0.0f;
                    if (acc_mode == TLO_ACC_F32_REV)
                        for (int d = D - 1; d >= 0; d--) acc += qf[d] * H2F(kr[d]);
                    else
                        for (int d = 0; d < D; d++) acc += qf[d] * H2F(kr[d]);
                    uint16_t sv = tlo_f2h(acc);                 /* einsum store  */
                    sv = tlo_f2h(H2F(sv) * scale_h);            /* scores * c    */
                    if (causal && j > qpos) sv = tlo_f2h(-10000.0f);  /* mask */
                    sc[j] = sv;
                }
                softmax_row(sc, J, p);
                uint16_t* orow = out + ((size_t)s * H + h) * D;
                for (int d = 0; d < D; d++) {
                    if (acc_mode == TLO_ACC_F16) {
                        uint16_t a = 0;
                        for (int j = 0; j < J; j++) {
                            uint16_t pr = tlo_f2h(H2F(p[j]) * H2F(v[((size_t)j * Hkv + kvh) * D + d]));
                            a = tlo_f2h(H2F(a) + H2F(pr));
                        }
                        orow[d] = a;
                    } else if (acc_mode == TLO_ACC_F32_REV) {
                        float a = 0.0f;
                        for (int j = J - 1; j >= 0; j--)
                            a += H2F(p[j]) * H2F(v[((size_t)j * Hkv + kvh) * D + d]);
                        orow[d] = tlo_f2h(a);
                    } else {
                        float a = 0.0f;
                        for (int j = 0; j < J; j++)
                            a += H2F(p[j]) * H2F(v[((size_t)j * Hkv + kvh) * D + d]);
                        orow[d] = tlo_f2h(a);
                    }
                }
            }
        }
        free(sc);
        free(p);
        free(qf);
    }
}

void tlo_einsum_scores(const uint16_t* q, const uint16_t* k, int I, int J, int H, int Hkv, int D,
                       uint16_t* out) {
    lut_init();
    const int group = H / Hkv;
    #pragma omp parallel for schedule(static) collapse(2)
    for (int i = 0; i < I; i++) {
        for (int h = 0; h < H; h++) {
            const uint16_t* qr = q + ((size_t)i * H + h) * D;
            for (int j = 0; j < J; j++) {
                const uint16_t* kr = k + ((size_t)j * Hkv + h / group) * D;
                float acc = 0.0f;
                for (int d = 0; d < D; d++) acc += H2F(qr[d]) * H2F(kr[d]);
                out[((size_t)i * H + h) * J + j] = tlo_f2h(acc);
            }
        }
    }
}

void tlo_einsum_context(const uint16_t* p, const uint16_t* v, int I, int J, int H, int Hkv, int D,
                        int acc_mode, uint16_t* out) {
    lut_init();
    const int group = H / Hkv;
    #pragma omp parallel for schedule(static) collapse(2)
    for (int i = 0; i < I; i++) {
        for (int h = 0; h < H; h++) {
            const uint16_t* pr = p + ((size_t)i * H + h) * J;
            for (int d = 0; d < D; d++) {
                float a = 0.0f;
                uint16_t ah = 0;
                for (int j = 0; j < J; j++) {
                    const float vv = H2F(v[((size_t)j * Hkv + h / group) * D + d]);
                    if (acc_mode == TLO_ACC_F16) ah = tlo_f2h(H2F(ah) + H2F(tlo_f2h(H2F(pr[j]) * vv)));
                    else a += H2F(pr[j]) * vv;
                }
                out[((size_t)i * H + h) * D + d] = acc_mode == TLO_ACC_F16 ? ah : tlo_f2h(a);
            }
        }
    }
}

void tlo_apply_attention_mask(const uint16_t* scores, const uint16_t* mask, size_t n, uint16_t* out) {
    lut_init();
    const uint16_t masked = tlo_f2h(-10000.0f);
    for (size_t i = 0; i < n; i++) out[i] = H2F(mask[i]) == 0.0f ? masked : scores[i];
}

/* ======================================================================== */
/* masks, slicing, broadcasting, table RoPE                                 */
/* ======================================================================== */

void tlo_causal_mask(int n, uint16_t* out) {
    /* builtin_nn.rs:445-455: f16::ONE where j <= i, f16::ZERO otherwise */
    for (int i = 0; i < n; i++)
        for (int j = 0; j < n; j++) out[(size_t)i * n + j] = j <= i ? 0x3C00u : 0u;
}

int tlo_slice_last(const void* x, const int64_t* shape, int ndim, int axis, int elem, void* y) {
    /* slice.rs:29-40: axis must exist and be 0 */
    if (axis < 0 || axis >= ndim || axis != 0) return -1;
    size_t inner = 1;
    for (int i = 1; i < ndim; i++) inner *= (size_t)shape[i];
    if (shape[0] <= 0) return -1;
    memcpy(y, (const uint8_t*)x + (size_t)(shape[0] - 1) * inner * (size_t)elem, inner * (size_t)elem);
    return 0;
}

int64_t tlo_tensor_argmax(const double* x, const int64_t* shape, int ndim, int dim, int64_t* idx) {
    size_t total = 1;
    for (int i = 0; i < ndim; i++) total *= (size_t)shape[i];
    if (dim < 0) {
        /* reduce.rs:589-598 */
        if (total == 0) return -1;
        int64_t best = 0;
        double mv = x[0];
        for (size_t i = 1; i < total; i++)
            if (x[i] > mv) {
                mv = x[i];
                best = (int64_t)i;
            }
        idx[0] = best;
        return 1;
    }
    if (dim >= ndim || ndim > 8) return -1;
    /* reduce.rs:621-668 */
    int64_t strides[8];
    strides[ndim - 1] = 1;
    for (int i = ndim - 2; i >= 0; i--) strides[i] = strides[i + 1] * shape[i + 1];
    size_t out_n = 1;
    for (int i = 0; i < ndim; i++)
        if (i != dim) out_n *= (size_t)shape[i];
    for (size_t o = 0; o < out_n; o++) {
        int64_t coords[8] = {0};
        size_t rem = o;
        for (int i = 0; i < ndim; i++)
            if (i != dim) {
                coords[i] = (int64_t)(rem % (size_t)shape[i]);
                rem /= (size_t)shape[i];
            }
        int64_t best = 0;
        double mv = -INFINITY;
        for (int64_t d = 0; d < shape[dim]; d++) {
            coords[dim] = d;
            int64_t lin = 0;
            for (int i = 0; i < ndim; i++) lin += coords[i] * strides[i];
            if (x[lin] > mv) {
                mv = x[lin];
                best = d;
            }
        }
        idx[o] = best;
    }
    return (int64_t)out_n;
}

int tlo_broadcast_to(const void* x, const int64_t* xshape, int xnd, const int64_t* tshape,
                     int tnd, int elem, void* y) {
    /* shape.rs:37-49: rank may not shrink; aligned from the right each input
     * dim equals the target's or is 1 */
    if (xnd > tnd || tnd > 8) return -1;
    for (int k = 1; k <= xnd; k++) {
        const int64_t a = xshape[xnd - k], b = tshape[tnd - k];
        if (a != b && a != 1) return -1;
    }
    size_t total = 1;
    for (int i = 0; i < tnd; i++) total *= (size_t)tshape[i];
    int64_t xstride[8];
    int64_t st = 1;
    for (int i = xnd - 1; i >= 0; i--) { xstride[i] = st; st *= xshape[i]; }
    const int rd = tnd - xnd;
    for (size_t g = 0; g < total; g++) {
        /* unified.metal:3788-3812: target multi-index, then each input dim of
         * size 1 reads coordinate 0 */
        size_t rem = g, src = 0;
        for (int i = tnd - 1; i >= 0; i--) {
            const size_t c = rem % (size_t)tshape[i];
            rem /= (size_t)tshape[i];
            if (i >= rd) {
                const int xi = i - rd;
                if (xshape[xi] != 1) src += c * (size_t)xstride[xi];
            }
        }
        memcpy((uint8_t*)y + g * (size_t)elem, (const uint8_t*)x + src * (size_t)elem, (size_t)elem);
    }
    return 0;
}

int tlo_rope_cos_sin(const uint16_t* x, int S, int H, int D, const uint16_t* cos_t,
                     const uint16_t* sin_t, int L, uint16_t* y) {
    lut_init();
    /* rope.rs:22-55: [S, H, D] input, [L >= S, D] tables */
    if (S < 0 || H < 0 || D <= 0 || D % 2 || L < S) return -1;
    for (int s = 0; s < S; s++)
        for (int h = 0; h < H; h++) {
            const uint16_t* xr = x + ((size_t)s * H + h) * D;
            uint16_t* yr = y + ((size_t)s * H + h) * D;
            for (int i = 0; i < D / 2; i++) {
                /* unified.metal:5161-5178: cos_sin_idx = seq_idx * head_dim + pair */
                const float c = H2F(cos_t[(size_t)s * D + i]), sn = H2F(sin_t[(size_t)s * D + i]);
                const float x0 = H2F(xr[2 * i]), x1 = H2F(xr[2 * i + 1]);
                const float a = x0 * c, b = x1 * sn;
                const float e = x0 * sn, f = x1 * c;
                yr[2 * i] = tlo_f2h(a - b);
                yr[2 * i + 1] = tlo_f2h(e + f);
            }
        }
    return 0;
}

void tlo_precompute_rope(int D, int L, float base, int want_sin, uint16_t* out) {
    for (int pos = 0; pos < L; pos++)
        for (int i = 0; i < D / 2; i++) {
            /* builtin_tensor.rs:664-682 */
            const float theta = 1.0f / powf(base, (float)(2 * i) / (float)D);
            const float ang = (float)pos * theta;
            const uint16_t v = tlo_f2h(want_sin ? sinf(ang) : cosf(ang));
            out[(size_t)pos * D + 2 * i] = v;
            out[(size_t)pos * D + 2 * i + 1] = v;
        }
}

/* ======================================================================== */
/* gather / sampling                                                        */
/* ======================================================================== */

int tlo_embedding(const uint16_t* table, int vocab, int hidden,
                  const int32_t* ids, int n, uint16_t* out) {
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= vocab) return -1;
    for (int i = 0; i < n; i++)
        memcpy(out + (size_t)i * hidden, table + (size_t)ids[i] * hidden,
               sizeof(uint16_t) * (size_t)hidden);
    return 0;
}

int tlo_sample_temperature(const uint16_t* logits, int n, float temperature, float r) {
    lut_init();
    float* p = (float*)malloc(sizeof(float) * (size_t)n);
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) {
        p[i] = H2F(logits[i]) / temperature;
        mx = fmaxf(mx, p[i]);   /* f32::max: a NaN operand loses */
    }
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        p[i] = expf(p[i] - mx);
        sum += p[i];
    }
    for (int i = 0; i < n; i++) p[i] /= sum;
    float cum = 0.0f;
    int idx = n - 1;
    for (int i = 0; i < n; i++) {
        cum += p[i];
        if (r < cum) { idx = i; break; }
    }
    free(p);
    return idx;
}

float tlo_sample_uniform(uint64_t seed, uint64_t counter) {
    uint64_t z = seed + (counter + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)(z >> 40) * 0x1p-24f;
}

int tlo_argmax_last(const uint16_t* logits, int n) {
    lut_init();
    int best = 0;
    float bv = H2F(logits[0]);
    for (int i = 1; i < n; i++) {
        float v = H2F(logits[i]);
        if (v >= bv) { bv = v; best = i; }
    }
    return best;
}

/* ======================================================================== */
/* GGUF reader: magic, version 2/3, KV section (every value type sized per
 * the GGUF spec, unlike mmap_gguf.rs:329-336 which reads 4 bytes for the
 * 1- and 2-byte types), tensor infos (dims reversed, mmap_gguf.rs:220-231),
 * data section aligned to general.alignment (default 32, :256-257).       */
/* ======================================================================== */

typedef struct {
    char* name;
    int type;
    int ndim;
    int64_t dims[4];
    uint64_t offset;
    size_t nbytes;
} tlo_ginfo;

typedef struct {
    char* key;
    int type;
    uint64_t u;     /* integer payload */
    double f;       /* float payload */
} tlo_gkv;

struct tlo_gguf {
    uint8_t* map;
    size_t size;
    int n_tensors;
    tlo_ginfo* infos;
    int n_kv;
    tlo_gkv* kvs;
    size_t data_off;
};

typedef struct { const uint8_t* p; size_t n; size_t off; int err; } rd_t;

static uint64_t rd_uint(rd_t* r, int bytes) {
    if (r->off + (size_t)bytes > r->n) { r->err = 1; return 0; }
    uint64_t v = 0;
    for (int i = 0; i < bytes; i++) v |= (uint64_t)r->p[r->off + i] << (8 * i);
    r->off += (size_t)bytes;
    return v;
}

static char* rd_str(rd_t* r) {
    uint64_t len = rd_uint(r, 8);
    if (r->err || r->off + len > r->n) { r->err = 1; return NULL; }
    char* s = (char*)malloc(len + 1);
    memcpy(s, r->p + r->off, len);
    s[len] = 0;
    r->off += len;
    return s;
}

static int gguf_scalar_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;   /* u8 i8 bool */
        case 2: case 3: return 2;           /* u16 i16 */
        case 4: case 5: case 6: return 4;   /* u32 i32 f32 */
        case 10: case 11: case 12: return 8;/* u64 i64 f64 */
        default: return -1;
    }
}

static int rd_skip_value(rd_t* r, uint32_t t, uint64_t* u, double* f) {
    if (t == 8) { char* s = rd_str(r); free(s); return r->err ? -1 : 0; }
    if (t == 9) {
        uint32_t at = (uint32_t)rd_uint(r, 4);
        uint64_t n = rd_uint(r, 8);
        if (r->err) return -1;
        for (uint64_t i = 0; i < n; i++)
            if (rd_skip_value(r, at, NULL, NULL)) return -1;
        return 0;
    }
    int sz = gguf_scalar_size(t);
    if (sz < 0) return -1;
    uint64_t v = rd_uint(r, sz);
    if (r->err) return -1;
    if (u) *u = v;
    if (f) {
        if (t == 6) { uint32_t b = (uint32_t)v; float ff; memcpy(&ff, &b, 4); *f = ff; }
        else if (t == 12) { double dd; memcpy(&dd, &v, 8); *f = dd; }
        else *f = (double)v;
    }
    return 0;
}

static size_t gguf_type_bytes(int type, uint64_t nelem) {
    switch (type) {
        case 0: return nelem * 4;
        case 1: return nelem * 2;
        case 2: return nelem / 32 * 18;
        case 8: return nelem / 32 * 34;
        case 14: return nelem / 256 * 210;
        default: return 0;
    }
}

tlo_gguf* tlo_gguf_open(const char* path) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) return NULL;
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); return NULL; }
    size_t size = (size_t)st.st_size;
    void* m = mmap(NULL, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return NULL;
    tlo_gguf* g = (tlo_gguf*)calloc(1, sizeof(tlo_gguf));
    g->map = (uint8_t*)m;
    g->size = size;
    rd_t r = { g->map, size, 0, 0 };
    uint32_t magic = (uint32_t)rd_uint(&r, 4);
    uint32_t version = (uint32_t)rd_uint(&r, 4);
    if (r.err || magic != 0x46554747u || version < 2 || version > 3) goto fail;
    uint64_t nt = rd_uint(&r, 8), nkv = rd_uint(&r, 8);
    if (r.err || nt > (1u << 20) || nkv > (1u << 20)) goto fail;
    g->n_kv = (int)nkv;
    g->kvs = (tlo_gkv*)calloc(nkv ? nkv : 1, sizeof(tlo_gkv));
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < nkv; i++) {
        g->kvs[i].key = rd_str(&r);
        uint32_t t = (uint32_t)rd_uint(&r, 4);
        if (r.err) goto fail;
        g->kvs[i].type = (int)t;
        if (rd_skip_value(&r, t, &g->kvs[i].u, &g->kvs[i].f)) goto fail;
        if (!strcmp(g->kvs[i].key, "general.alignment") && t == 4) alignment = g->kvs[i].u;
    }
    g->n_tensors = (int)nt;
    g->infos = (tlo_ginfo*)calloc(nt ? nt : 1, sizeof(tlo_ginfo));
    for (uint64_t i = 0; i < nt; i++) {
        tlo_ginfo* ti = &g->infos[i];
        ti->name = rd_str(&r);
        uint32_t nd = (uint32_t)rd_uint(&r, 4);
        if (r.err || nd < 1 || nd > 4) goto fail;
        int64_t raw[4];
        uint64_t nelem = 1;
        for (uint32_t d = 0; d < nd; d++) {
            raw[d] = (int64_t)rd_uint(&r, 8);
            /* element counts past 2^48 fit no mappable file; the bound keeps
             * gguf_type_bytes' products in range */
            if (raw[d] < 0 || __builtin_mul_overflow(nelem, (uint64_t)raw[d], &nelem) ||
                nelem > ((uint64_t)1 << 48)) goto fail;
        }
        ti->ndim = (int)nd;
        for (uint32_t d = 0; d < nd; d++) ti->dims[d] = raw[nd - 1 - d];
        ti->type = (int)rd_uint(&r, 4);
        ti->offset = rd_uint(&r, 8);
        if (r.err) goto fail;
        ti->nbytes = gguf_type_bytes(ti->type, nelem);
        /* quantized tensors hold whole blocks (Q4_0 / Q8_0: 32, Q6_K: 256) */
        if ((ti->type == 2 || ti->type == 8) && nelem % 32) goto fail;
        if (ti->type == 14 && nelem % 256) goto fail;
    }
    if (alignment == 0) alignment = 32;
    g->data_off = (r.off + alignment - 1) / alignment * alignment;
    if (g->data_off > size) goto fail;
    for (int i = 0; i < g->n_tensors; i++) {
        /* [offset, offset + nbytes) inside the data section, compared as
         * differences so that no sum wraps */
        const size_t avail = size - g->data_off;
        if (g->infos[i].offset > avail || g->infos[i].nbytes > avail - g->infos[i].offset) goto fail;
    }
    return g;
fail:
    tlo_gguf_close(g);
    return NULL;
}

void tlo_gguf_close(tlo_gguf* g) {
    if (!g) return;
    if (g->infos) { for (int i = 0; i < g->n_tensors; i++) free(g->infos[i].name); free(g->infos); }
    if (g->kvs) { for (int i = 0; i < g->n_kv; i++) free(g->kvs[i].key); free(g->kvs); }
    if (g->map) munmap(g->map, g->size);
    free(g);
}

int tlo_gguf_n_tensors(const tlo_gguf* g) { return g ? g->n_tensors : 0; }

const char* tlo_gguf_tensor_name(const tlo_gguf* g, int i) {
    return (g && i >= 0 && i < g->n_tensors) ? g->infos[i].name : NULL;
}

const void* tlo_gguf_tensor(const tlo_gguf* g, const char* name, int* gguf_type,
                            int* ndim, int64_t dims[4], size_t* nbytes) {
    if (!g) return NULL;
    for (int i = 0; i < g->n_tensors; i++) {
        const tlo_ginfo* ti = &g->infos[i];
        if (ti->name && !strcmp(ti->name, name)) {
            if (gguf_type) *gguf_type = ti->type;
            if (ndim) *ndim = ti->ndim;
            if (dims) for (int d = 0; d < 4; d++) dims[d] = d < ti->ndim ? ti->dims[d] : 1;
            if (nbytes) *nbytes = ti->nbytes;
            return g->map + g->data_off + ti->offset;
        }
    }
    return NULL;
}

static const tlo_gkv* find_kv(const tlo_gguf* g, const char* key) {
    for (int i = 0; i < g->n_kv; i++)
        if (g->kvs[i].key && !strcmp(g->kvs[i].key, key)) return &g->kvs[i];
    return NULL;
}

int tlo_gguf_kv_u32(const tlo_gguf* g, const char* key, uint32_t* v) {
    const tlo_gkv* kv = g ? find_kv(g, key) : NULL;
    if (!kv) return -1;
    *v = (uint32_t)kv->u;
    return 0;
}

int tlo_gguf_kv_f32(const tlo_gguf* g, const char* key, float* v) {
    const tlo_gkv* kv = g ? find_kv(g, key) : NULL;
    if (!kv) return -1;
    *v = (float)kv->f;
    return 0;
}

/* ======================================================================== */
/* decoder driver                                                           */
/* ======================================================================== */

typedef struct {
    float* w;        /* dequantised weight, as f32 (exactly the f16 values) */
    uint16_t* b;     /* optional bias (f16) */
    int n, k;
} lin_t;

typedef struct {
    uint16_t *norm_w, *norm_b, *ffn_norm_w;
    lin_t q, k, v, qkv, o, gate, up, down;
    uint16_t *kc, *vc;   /* [max_ctx, Hkv, D] */
} layer_t;

struct tlo_model {
    int arch, n_layers, hidden, inter, n_heads, n_kv, head_dim, vocab, rot_dims, max_ctx;
    float eps, theta;
    int acc_mode;
    int literal;             /* tlo_model_set_program_semantics */
    float gguf_eps;          /* eps read from the file */
    int pos;                 /* tokens already in the cache */
    uint16_t* embd;          /* [vocab, hidden] f16 */
    uint16_t *out_norm_w, *out_norm_b;
    lin_t out;
    layer_t* layers;
};

static uint16_t* load_f16_vec(const tlo_gguf* g, const char* name, int64_t expect) {
    int type, nd; int64_t dims[4]; size_t nb;
    const void* p = tlo_gguf_tensor(g, name, &type, &nd, dims, &nb);
    if (!p) return NULL;
    int64_t n = 1;
    for (int i = 0; i < nd; i++) n *= dims[i];
    if (expect >= 0 && n != expect) return NULL;
    uint16_t* out = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n);
    if (type == 1) memcpy(out, p, sizeof(uint16_t) * (size_t)n);
    else if (type == 0) { const float* f = (const float*)p; for (int64_t i = 0; i < n; i++) out[i] = tlo_f2h(f[i]); }
    else if (type == 2 || type == 8) dequant_any((const uint8_t*)p, type, (size_t)n / 32, out);
    else if (type == 14 && n % 256 == 0) dequant_any((const uint8_t*)p, type, (size_t)n / 32, out);
    else { free(out); return NULL; }
    return out;
}

static int load_lin(const tlo_gguf* g, const char* name, const char* bname, int n, int k, lin_t* l) {
    uint16_t* h = load_f16_vec(g, name, (int64_t)n * k);
    if (!h) return -1;
    l->n = n; l->k = k;
    l->w = (float*)malloc(sizeof(float) * (size_t)n * k);
    for (size_t i = 0; i < (size_t)n * k; i++) l->w[i] = H2F(h[i]);
    free(h);
    l->b = bname ? load_f16_vec(g, bname, n) : NULL;
    return 0;
}

static void free_lin(lin_t* l) { free(l->w); free(l->b); }

int tlo_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

tlo_model* tlo_model_load(const char* path, int arch, int max_ctx, int acc_mode, int n_threads) {
    lut_init();
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#else
    (void)n_threads;
#endif
    tlo_gguf* g = tlo_gguf_open(path);
    if (!g) return NULL;
    tlo_model* m = (tlo_model*)calloc(1, sizeof(tlo_model));
    m->arch = arch;
    m->acc_mode = acc_mode;
    m->max_ctx = max_ctx;
    const char* a = arch == 0 ? "llama" : "phi2";
    char key[128];
    uint32_t u;
    float f;
    {
        const char* keys[5] = { "block_count", "embedding_length", "feed_forward_length",
                                "attention.head_count", "attention.head_count_kv" };
        int* fields[5] = { &m->n_layers, &m->hidden, &m->inter, &m->n_heads, &m->n_kv };
        for (int i = 0; i < 5; i++) {
            snprintf(key, sizeof key, "%s.%s", a, keys[i]);
            if (tlo_gguf_kv_u32(g, key, &u)) goto fail;
            *fields[i] = (int)u;
        }
    }
    m->head_dim = m->hidden / m->n_heads;
    snprintf(key, sizeof key, "%s.%s", a, arch == 0 ? "attention.layer_norm_rms_epsilon" : "attention.layer_norm_epsilon");
    m->eps = tlo_gguf_kv_f32(g, key, &f) ? 1e-5f : f;
    m->gguf_eps = m->eps;
    snprintf(key, sizeof key, "%s.rope.freq_base", a);
    m->theta = tlo_gguf_kv_f32(g, key, &f) ? 10000.0f : f;
    snprintf(key, sizeof key, "%s.rope.dimension_count", a);
    m->rot_dims = tlo_gguf_kv_u32(g, key, &u) ? m->head_dim : (int)u;
    {
        int type, nd; int64_t dims[4];
        if (!tlo_gguf_tensor(g, "token_embd.weight", &type, &nd, dims, NULL)) goto fail;
        m->vocab = (int)dims[0];
    }
    m->embd = load_f16_vec(g, "token_embd.weight", (int64_t)m->vocab * m->hidden);
    if (!m->embd) goto fail;
    int H = m->hidden, kvd = m->n_kv * m->head_dim;
    m->out_norm_w = load_f16_vec(g, "output_norm.weight", H);
    if (!m->out_norm_w) goto fail;
    if (arch == 1) m->out_norm_b = load_f16_vec(g, "output_norm.bias", H);
    if (load_lin(g, "output.weight", arch == 1 ? "output.bias" : NULL, m->vocab, H, &m->out)) goto fail;
    m->layers = (layer_t*)calloc((size_t)m->n_layers, sizeof(layer_t));
    for (int i = 0; i < m->n_layers; i++) {
        layer_t* L = &m->layers[i];
        char n1[96], n2[96];
#define NM(buf, s) snprintf(buf, sizeof buf, "blk.%d.%s", i, s)
        NM(n1, "attn_norm.weight");
        if (!(L->norm_w = load_f16_vec(g, n1, H))) goto fail;
        if (arch == 0) {
            NM(n1, "ffn_norm.weight");
            if (!(L->ffn_norm_w = load_f16_vec(g, n1, H))) goto fail;
            NM(n1, "attn_q.weight"); if (load_lin(g, n1, NULL, H, H, &L->q)) goto fail;
            NM(n1, "attn_k.weight"); if (load_lin(g, n1, NULL, kvd, H, &L->k)) goto fail;
            NM(n1, "attn_v.weight"); if (load_lin(g, n1, NULL, kvd, H, &L->v)) goto fail;
            NM(n1, "attn_output.weight"); if (load_lin(g, n1, NULL, H, H, &L->o)) goto fail;
            NM(n1, "ffn_gate.weight"); if (load_lin(g, n1, NULL, m->inter, H, &L->gate)) goto fail;
            NM(n1, "ffn_up.weight"); if (load_lin(g, n1, NULL, m->inter, H, &L->up)) goto fail;
            NM(n1, "ffn_down.weight"); if (load_lin(g, n1, NULL, H, m->inter, &L->down)) goto fail;
        } else {
            NM(n1, "attn_norm.bias");
            if (!(L->norm_b = load_f16_vec(g, n1, H))) goto fail;
            NM(n1, "attn_qkv.weight"); NM(n2, "attn_qkv.bias");
            if (load_lin(g, n1, n2, H + 2 * kvd, H, &L->qkv)) goto fail;
            NM(n1, "attn_output.weight"); NM(n2, "attn_output.bias");
            if (load_lin(g, n1, n2, H, H, &L->o)) goto fail;
            NM(n1, "ffn_up.weight"); NM(n2, "ffn_up.bias");
            if (load_lin(g, n1, n2, m->inter, H, &L->up)) goto fail;
            NM(n1, "ffn_down.weight"); NM(n2, "ffn_down.bias");
            if (load_lin(g, n1, n2, H, m->inter, &L->down)) goto fail;
        }
#undef NM
        L->kc = (uint16_t*)calloc((size_t)max_ctx * kvd, sizeof(uint16_t));
        L->vc = (uint16_t*)calloc((size_t)max_ctx * kvd, sizeof(uint16_t));
    }
    tlo_gguf_close(g);
    return m;
fail:
    tlo_gguf_close(g);
    tlo_model_free(m);
    return NULL;
}

void tlo_model_free(tlo_model* m) {
    if (!m) return;
    free(m->embd); free(m->out_norm_w); free(m->out_norm_b);
    free_lin(&m->out);
    if (m->layers) {
        for (int i = 0; i < m->n_layers; i++) {
            layer_t* L = &m->layers[i];
            free(L->norm_w); free(L->norm_b); free(L->ffn_norm_w);
            free_lin(&L->q); free_lin(&L->k); free_lin(&L->v); free_lin(&L->qkv);
            free_lin(&L->o); free_lin(&L->gate); free_lin(&L->up); free_lin(&L->down);
            free(L->kc); free(L->vc);
        }
        free(m->layers);
    }
    free(m);
}

void tlo_model_reset(tlo_model* m) { if (m) m->pos = 0; }
int tlo_model_vocab(const tlo_model* m) { return m ? m->vocab : 0; }
int tlo_model_hidden(const tlo_model* m) { return m ? m->hidden : 0; }

/* y[M, l->n] = linear(x[M, l->k]) with the model's accumulation mode. */
static void run_lin(const tlo_model* m, const lin_t* l, const uint16_t* x, int M, uint16_t* y) {
    float* xf = (float*)malloc(sizeof(float) * (size_t)M * l->k);
    for (size_t i = 0; i < (size_t)M * l->k; i++) xf[i] = H2F(x[i]);
    linear_rows_f32w(xf, l->w, l->b, M, l->n, l->k, m->acc_mode, y);
    free(xf);
}

int tlo_model_forward(tlo_model* m, const int32_t* ids, int n, int pos0,
                      uint16_t* hidden_out, uint16_t* logits_out) {
    if (!m || n <= 0 || pos0 < 0 || pos0 + n > m->max_ctx) return -1;
    int H = m->hidden, D = m->head_dim, NH = m->n_heads, NKV = m->n_kv, kvd = NKV * D, I = m->inter;
    size_t SH = (size_t)n * H;
    uint16_t* x = (uint16_t*)malloc(sizeof(uint16_t) * SH);
    uint16_t* xn = (uint16_t*)malloc(sizeof(uint16_t) * SH);
    uint16_t* q = (uint16_t*)malloc(sizeof(uint16_t) * SH);
    uint16_t* qr = (uint16_t*)malloc(sizeof(uint16_t) * SH);
    uint16_t* kk = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n * kvd);
    uint16_t* vv = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n * kvd);
    uint16_t* att = (uint16_t*)malloc(sizeof(uint16_t) * SH);
    uint16_t* ao = (uint16_t*)malloc(sizeof(uint16_t) * SH);
    uint16_t* x1 = (uint16_t*)malloc(sizeof(uint16_t) * SH);
    uint16_t* g = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n * I);
    uint16_t* u = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n * I);
    uint16_t* qkv = m->arch == 1 ? (uint16_t*)malloc(sizeof(uint16_t) * (size_t)n * (H + 2 * kvd)) : NULL;
    int rc = tlo_embedding(m->embd, m->vocab, H, ids, n, x);
    if (rc) goto done;
    float scale = 1.0f / sqrtf((float)D);
    /* rotation offset: literal program semantics rotate a decode row (one
     * token after the prompt) at position 0, prompt rows at pos0 + s */
    const int rope_off = (m->literal && n == 1 && pos0 > 0) ? 0 : pos0;
    for (int li = 0; li < m->n_layers; li++) {
        layer_t* L = &m->layers[li];
        uint16_t* kdst = L->kc + (size_t)pos0 * kvd;
        uint16_t* vdst = L->vc + (size_t)pos0 * kvd;
        if (m->arch == 0) {
            tlo_rms_norm(x, L->norm_w, n, H, m->eps, xn);
            run_lin(m, &L->q, xn, n, q);
            run_lin(m, &L->k, xn, n, kk);
            run_lin(m, &L->v, xn, n, vv);
            tlo_rope(q, n, NH, D, rope_off, m->theta, TLO_ROPE_INTERLEAVED, D, qr);
            tlo_rope(kk, n, NKV, D, rope_off, m->theta, TLO_ROPE_INTERLEAVED, D, kdst);
            memcpy(vdst, vv, sizeof(uint16_t) * (size_t)n * kvd);
            tlo_attention(qr, L->kc, L->vc, n, pos0 + n, NH, NKV, D, pos0, scale, 1, m->acc_mode, att);
            run_lin(m, &L->o, att, n, ao);
            tlo_add(x, ao, SH, x1);
            tlo_rms_norm(x1, L->ffn_norm_w, n, H, m->eps, xn);
            run_lin(m, &L->gate, xn, n, g);
            run_lin(m, &L->up, xn, n, u);
            tlo_swiglu(g, u, (size_t)n * I, g);
            run_lin(m, &L->down, g, n, ao);
            tlo_add(x1, ao, SH, x);
        } else {
            int W3 = H + 2 * kvd;
            tlo_layer_norm(x, L->norm_w, L->norm_b, n, H, m->eps, xn);
            run_lin(m, &L->qkv, xn, n, qkv);
            for (int s = 0; s < n; s++) {
                memcpy(q + (size_t)s * H, qkv + (size_t)s * W3, sizeof(uint16_t) * H);
                memcpy(kk + (size_t)s * kvd, qkv + (size_t)s * W3 + H, sizeof(uint16_t) * kvd);
                memcpy(vv + (size_t)s * kvd, qkv + (size_t)s * W3 + H + kvd, sizeof(uint16_t) * kvd);
            }
            tlo_rope(q, n, NH, D, pos0, m->theta, TLO_ROPE_NEOX, m->rot_dims, qr);
            tlo_rope(kk, n, NKV, D, pos0, m->theta, TLO_ROPE_NEOX, m->rot_dims, kdst);
            memcpy(vdst, vv, sizeof(uint16_t) * (size_t)n * kvd);
            tlo_attention(qr, L->kc, L->vc, n, pos0 + n, NH, NKV, D, pos0, scale, 1, m->acc_mode, att);
            run_lin(m, &L->o, att, n, ao);
            run_lin(m, &L->up, xn, n, g);
            tlo_gelu(g, (size_t)n * I, g);
            run_lin(m, &L->down, g, n, x1);
            tlo_add(x, ao, SH, x);
            tlo_add(x, x1, SH, x);
        }
    }
    if (hidden_out) memcpy(hidden_out, x, sizeof(uint16_t) * SH);
    if (logits_out) {
        const uint16_t* last = x + (size_t)(n - 1) * H;
        if (m->arch == 0) tlo_rms_norm(last, m->out_norm_w, 1, H, m->eps, xn);
        else tlo_layer_norm(last, m->out_norm_w, m->out_norm_b, 1, H, m->eps, xn);
        run_lin(m, &m->out, xn, 1, logits_out);
    }
    m->pos = pos0 + n;
done:
    free(x); free(xn); free(q); free(qr); free(kk); free(vv); free(att); free(ao);
    free(x1); free(g); free(u); free(qkv);
    return rc;
}

static float top_margin(const uint16_t* logits, int n, int best) {
    float b = H2F(logits[best]), second = -INFINITY;
    for (int i = 0; i < n; i++) if (i != best) { float v = H2F(logits[i]); if (v > second) second = v; }
    return b - second;
}

int tlo_model_set_program_semantics(tlo_model* m, int literal) {
    if (!m || m->arch != 0) return -1;
    m->literal = literal != 0;
    m->eps = m->literal ? 1e-6f : m->gguf_eps;
    return 0;
}

int tlo_model_generate(tlo_model* m, const int32_t* prompt, int n_prompt,
                       int n_decode, int32_t* tokens_out, float* margins_out,
                       uint16_t* last_logits) {
    if (!m || n_prompt <= 0 || n_prompt + n_decode > m->max_ctx) return -1;
    uint16_t* logits = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)m->vocab);
    tlo_model_reset(m);
    int rc = tlo_model_forward(m, prompt, n_prompt, 0, NULL, logits);
    for (int step = 0; rc == 0 && step <= n_decode; step++) {
        int tok = tlo_argmax_last(logits, m->vocab);
        tokens_out[step] = tok;
        if (margins_out) margins_out[step] = top_margin(logits, m->vocab, tok);
        if (step == n_decode) break;
        rc = tlo_model_forward(m, &tok, 1, m->pos, NULL, logits);
    }
    if (rc == 0 && last_logits) memcpy(last_logits, logits, sizeof(uint16_t) * (size_t)m->vocab);
    free(logits);
    return rc;
}
