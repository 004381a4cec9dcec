/*
 * tl_oracle.h -- CPU restatement of TensorLogic's quantized-LLM hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it, and only to check or to time the reference's CPU arithmetic.
 * The product (libtlhip.so, tensorlogic_amd/) never links, loads or calls it.
 *
 * Every function restates one reference function or Metal kernel; the
 * reference file:line it follows is given beside each declaration.  All
 * tensors are host arrays: f16 values are IEEE binary16 bit patterns in
 * uint16_t (little-endian), f32 is float, rows are contiguous (row-major).
 *
 * Two accumulation modes exist for contractions:
 *   TLO_ACC_F32 -- fp32 accumulation, f16 storage of every op output exactly
 *                  where the reference stores f16 (the parity oracle);
 *   TLO_ACC_F16 -- the reference CPU loops' own f16 accumulation
 *                  (src/ops/matmul.rs:201-228, unified.metal:2646-2684),
 *                  used only as the timed CPU baseline;
 *   TLO_ACC_F32_REV -- TLO_ACC_F32 with the linear and attention (scores
 *                  and context) sums taken in descending order: a second, equally valid
 *                  fp32 order, used only to measure how far a model's
 *                  outputs move between two fp32 summation orders.
 *
 * Pinning of each function is recorded in tests/ (test_oracle_*.py).
 */
#ifndef TL_ORACLE_H
#define TL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { TLO_ACC_F32 = 0, TLO_ACC_F16 = 1, TLO_ACC_F32_REV = 2 };
enum { TLO_ROPE_INTERLEAVED = 0, TLO_ROPE_NEOX = 1 };

/* Number of OpenMP threads used by the loops below (the calling thread's
 * setting; n <= 0 leaves it unchanged).  Returns the count now in force. */
int      tlo_set_threads(int n);

/* ---- binary16 <-> binary32 (the `half` 2.7.1 crate's from_f32/to_f32:
 *      RNE, subnormals kept, NaN kept quiet) --------------------------------*/
float    tlo_h2f(uint16_t h);
uint16_t tlo_f2h(float f);
void     tlo_h2f_array(const uint16_t* h, float* f, size_t n);
void     tlo_f2h_array(const float* f, uint16_t* h, size_t n);

/* ---- GGUF block dequantisation ------------------------------------------
 * Q4_0 block = f16 d + 16 bytes; element j (j<16) = low nibble of byte j,
 * element j+16 = high nibble; value = RNE_f16(((q & 15) - 8) * d).
 *   src/model/formats/gguf.rs:68-112, mmap_gguf.rs:383-414
 * Q8_0 block = f16 d + 32 int8; value = RNE_f16(f16(q) * d).
 *   src/model/formats/gguf.rs:22-53, mmap_gguf.rs:417-439                   */
void tlo_dequant_q4_0(const uint8_t* blocks, size_t nblocks, uint16_t* out);
void tlo_dequant_q8_0(const uint8_t* blocks, size_t nblocks, uint16_t* out);
/* Q6_K super-block = ql[128] + qh[64] + int8 sc[16] + f16 d (210 bytes,
 * 256 elements); value = f16(f32(d * sc) * (q6 - 32)), the f32 product exact.
 *   src/model/formats/gguf.rs:128-212, mmap_gguf.rs:457-545               */
void tlo_dequant_q6_k(const uint8_t* blocks, size_t nblocks, uint16_t* out);

/* ---- linear / matmul_transposed_b ---------------------------------------
 * y[M,N] = x[M,K] . W[N,K]^T (+ bias[N]) ; f16 in, f16 out.
 *   GPU: matmul_transposed_b_tiled_32x32_f16 unified.metal:4291-4348
 *        (fp32 accumulate in k order, half(sum) store)
 *   CPU: matmul.rs:293-297 -> matmul_cpu matmul.rs:201-228 (f16 accumulate)
 * Bias, when given, is a separate f16 add of the stored product
 *   (builtin_math.rs:76-131: linear(x, W, b) = add(matmul, b)).            */
/* linear() on TensorF32 operands (builtin_math.rs:121-175) =
 * matmul_transposed_b_tiled_32x32_f32 (unified.metal:4409-4461) + add(bias):
 * y[m][n] = (sum over k = 0 .. ceil32(K) - 1, from +0, of fmaf(x[m][k],
 * w[n][k], sum), zero terms past K) + bias[n].  The one fused multiply-add
 * per term is the contraction Metal's default fast math makes of the
 * kernel's `sum += A * B`; the reference's CPU branch (matmul.rs:201-228)
 * rounds the product and the sum separately.  bias may be NULL.            */
void tlo_linear_f32(const float* x, const float* w, const float* bias, int M, int N, int K, float* y);
void tlo_linear_f16(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                    int M, int N, int K, int acc_mode, uint16_t* y);
/* Same product with W given as packed GGUF blocks (dequantised row by row
 * exactly as tlo_dequant_*): wtype 2 = Q4_0, 8 = Q8_0, 14 = Q6_K (GGUF
 * type ids).                                                              */
void tlo_linear_q(const uint16_t* x, const uint8_t* wblocks, int wtype,
                  const uint16_t* bias, int M, int N, int K, int acc_mode,
                  uint16_t* y);

/* ---- normalisation ------------------------------------------------------
 * rms_norm_cpu normalization.rs:199-250 (== rms_norm_f16 unified.metal:
 * 1785-1831): y = f16((x * (1/sqrt(mean(x^2)+eps))) * w), f32 sums.         */
void tlo_rms_norm(const uint16_t* x, const uint16_t* w, int rows, int n,
                  float eps, uint16_t* y);
/* layer_norm_f16 unified.metal:1620-1697 / normalization.rs:457-535:
 * mean, biased variance in f32, y = f16((x-mean)*inv_std*w + b).            */
void tlo_layer_norm(const uint16_t* x, const uint16_t* w, const uint16_t* b,
                    int rows, int n, float eps, uint16_t* y);

/* ---- RoPE ----------------------------------------------------------------
 * x [S, H, D]; position of row s = offset + s.
 * INTERLEAVED: pairs (2i, 2i+1)  rope_f16 unified.metal:2355-2418,
 *              rope.rs:71-118,215-300, test_shader_mathematical_correctness
 *              .rs:66-101.
 * NEOX: pairs (i, i + rot/2) for i < rot/2 ("rotate_half"); dims >= rot
 *       pass through (Phi-2 partial rotary; no reference op, restated from
 *       the same frequency formula).
 * freq_i = 1 / powf(theta, 2i / rot) ; angle = f32(pos) * freq_i ;
 * cos/sin of the f32 angle (evaluated in double, rounded to f32) ;
 * out0 = f16(x0*c - x1*s), out1 = f16(x0*s + x1*c), no fused multiply-add. */
void tlo_rope(const uint16_t* x, int S, int H, int D, int offset, float theta,
              int layout, int rot_dims, uint16_t* y);
/* The cos/sin table the formula above produces: cs[2*(p*half + i) + 0/1]. */
void tlo_rope_table(int max_pos, int rot_dims, float theta, float* cs);

/* ---- softmax / elementwise ---------------------------------------------
 * softmax_f16 / softmax_simple_f16 unified.metal:2057-2200 (one thread per
 * row, activations.rs:204-209): max over finite values; e = exp(x - max)
 * (0 for non-finite x); out = f16(e); sum += e (f32, unrounded);
 * out = f16(f32(out) / sum); degenerate sum -> f16(1/n).                    */
void tlo_softmax(const uint16_t* x, int rows, int n, uint16_t* y);
/* sigmoid_cpu activations.rs:252-266: f16(1 / (1 + exp(-x))) in f32.       */
void tlo_sigmoid(const uint16_t* x, size_t n, uint16_t* y);
/* the TensorF32 arms (unified.metal:1129-1135, 1961-2036, 2202-2340,
   2420-2482, 2702-2768): f32 in and out */
void tlo_rms_norm_f32(const float* x, const float* w, int rows, int n, float eps, float* y);
void tlo_softmax_f32(const float* x, int rows, int n, float* y);
void tlo_rope_f32(const float* x, int S, int H, int D, int offset, float theta, int layout, int rot_dims, float* y);
void tlo_sigmoid_f32(const float* x, size_t n, float* y);
void tlo_einsum_scores_f32(const float* q, const float* k, int I, int J, int H, int Hkv, int D, float* out);
void tlo_einsum_context_f32(const float* p, const float* v, int I, int J, int H, int Hkv, int D, float* out);
/* layer_norm_f32 (unified.metal:1833-1958): per-row sums in element order,
   the squares fused; gelu_f32 (:1051-1062); TL silu / swiglu on f32
   (sigmoid_f32 then mul_f32). */
void tlo_layer_norm_f32(const float* x, const float* w, const float* b, int rows, int n, float eps, float* y);
void tlo_gelu_f32(const float* x, size_t n, float* y);
void tlo_silu_f32(const float* x, size_t n, float* y);
void tlo_swiglu_f32(const float* g, const float* u, size_t n, float* y);
/* TL silu(x) = x * sigmoid(x) (examples/chat_demo_optimized.tl:35-37):
 * s = sigmoid(x) stored f16, then f16(x * s).                              */
void tlo_silu(const uint16_t* x, size_t n, uint16_t* y);
/* f16 elementwise (elementwise.rs:122,309-328; `half` Add/Mul): f16(a op b) */
void tlo_add(const uint16_t* a, const uint16_t* b, size_t n, uint16_t* y);
void tlo_mul(const uint16_t* a, const uint16_t* b, size_t n, uint16_t* y);
void tlo_mul_scalar(const uint16_t* a, float s, size_t n, uint16_t* y);
/* swiglu(g, u) = mul(silu(g), u), the TL swiglu_ffn intermediate.          */
void tlo_swiglu(const uint16_t* g, const uint16_t* u, size_t n, uint16_t* y);
/* gelu_f16 unified.metal:837-848 (tanh form) restated in f32:
 * 0.5*x*(1+tanh(sqrt(2/pi)*(x+0.044715 x^3))).                             */
void tlo_gelu(const uint16_t* x, size_t n, uint16_t* y);

/* ---- attention -------------------------------------------------------------
 * The TL attention sequence (chat_demo_optimized.tl:52-97,
 * debug/chat_demo_with_kvcache.tl:43-89,250-277):
 *   scores = einsum("ihd,jhd->ihj", Q, K_expanded)   f32 acc, f16 store
 *            (einsum_ihd_jhd_ihj_f16 unified.metal:2524-2560)
 *   scaled = scores * scale                           f16 x f16 -> f16
 *   masked = apply_attention_mask(scaled, causal)     masked -> -10000
 *            (unified.metal:4474-4489, masking.rs:147-165)
 *   P      = softmax(masked)                          tlo_softmax
 *   out    = einsum("ihj,jhd->ihd", P, V_expanded)    acc per acc_mode
 *            (einsum_ihj_jhd_ihd_f16 unified.metal:2646-2684)
 * q [S, H, D]; k, v [J, Hkv, D]; query head h reads KV head h / (H/Hkv)
 * (broadcast_to [J,Hkv,1,D] -> [J,Hkv,H/Hkv,D]).  Query row s sits at
 * absolute position q_pos0 + s and sees keys j <= q_pos0 + s when causal. */
void tlo_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                   int S, int J, int H, int Hkv, int D, int q_pos0,
                   float scale, int causal, int acc_mode, uint16_t* out);
/* The same steps one builtin at a time, as a TL program calls them:
 * einsum("ihd,jhd->ihj", q [I,H,D], k [J,Hkv,D]) -> [I,H,J], f32 acc, f16
 * store (einsum.rs:653-686, unified.metal:2524-2560); einsum("ihj,jhd->ihd",
 * p [I,H,J], v [J,Hkv,D]) -> [I,H,D], accumulation per acc_mode
 * (unified.metal:2646-2684).  Head h of q / p reads KV head h / (H/Hkv), the
 * broadcast_to + contiguous expansion of the programs.                     */
void tlo_einsum_scores(const uint16_t* q, const uint16_t* k, int I, int J, int H, int Hkv, int D,
                       uint16_t* out);
void tlo_einsum_context(const uint16_t* p, const uint16_t* v, int I, int J, int H, int Hkv, int D,
                        int acc_mode, uint16_t* out);
/* apply_attention_mask(scores, mask) (masking.rs:36-51,147-165,
 * unified.metal:4474-4489): scores and mask of the same n elements; where
 * the mask value equals 0 the score becomes f16(-10000), else it is kept.  */
void tlo_apply_attention_mask(const uint16_t* scores, const uint16_t* mask, size_t n, uint16_t* out);

/* ---- masks, slicing, broadcasting, table RoPE ---------------------------
 * causal_mask builtin_nn.rs:423-460 / Tensor::causal_mask masking.rs:192-207:
 * [n, n] f16, 1 where j <= i, else 0.                                      */
void tlo_causal_mask(int n, uint16_t* out);
/* Tensor::slice_last slice.rs:25-60 (slice_last_axis0_f16 unified.metal):
 * the last index of axis 0, x [d0, d1, ...] -> [d1, ...] (a 1-D input gives
 * its last element).  Only axis 0 is supported, as in the reference.
 * elem = element bytes.  Returns 0, or -1 for an axis the reference rejects
 * (InvalidOperation).                                                      */
int tlo_slice_last(const void* x, const int64_t* shape, int ndim, int axis, int elem, void* y);
/* Tensor::argmax(dim, keepdim) reduce.rs:585-658 (the argmax() builtin,
 * builtin_tensor.rs:1438-1490), on values already widened to double (exact
 * for f16 and f32 inputs).  dim < 0: the whole tensor, scanned in order from
 * element 0 with a strict '>' against element 0's value (reduce.rs:589-598)
 * -- the first maximum wins and a NaN at element 0 keeps index 0.  dim >= 0:
 * each output element o scans its line from a running maximum of -inf with
 * a strict '>' (reduce.rs:644-668), so the first maximum wins and NaN and
 * -inf never do.  Output element o's line has the non-reduced coordinates
 * of o taken digit by digit with the FIRST non-reduced dim least significant
 * (reduce.rs:649-657), as the reference computes them; its output is
 * row-major in the kept dims, so for two or more kept dims larger than one
 * the lines land in the transposed order.  idx receives the indices (one per
 * output element; 1 for dim < 0).  Returns the output element count, or -1
 * for dim >= ndim (InvalidDimension) or an empty input with dim < 0.      */
int64_t tlo_tensor_argmax(const double* x, const int64_t* shape, int ndim, int dim, int64_t* idx);
/* Tensor::broadcast_to broadcast.rs:11-30 + broadcast_f16 unified.metal:
 * 3769-3815, TensorShape::can_broadcast_to shape.rs:37-49: dims aligned from
 * the right; an input dim of 1 repeats.  Returns 0, or -1 when the shapes
 * do not broadcast (ShapeMismatch).                                        */
int tlo_broadcast_to(const void* x, const int64_t* xshape, int xnd, const int64_t* tshape,
                     int tnd, int elem, void* y);
/* rope(x, cos, sin) = Tensor::rope_candle rope.rs:18-65 + rope_candle_f16
 * unified.metal:5122-5185: x [S, H, D] f16, cos/sin [L >= S, D] f16; pair
 * i of row s (elements 2i, 2i+1) is rotated by cos[s, i] / sin[s, i] --
 * column i, not 2i, exactly as the Metal kernel indexes the table (with
 * the duplicated tables of precompute_rope_*, pair i therefore turns by
 * the frequency of pair i/2).  f32 products, each rounded, f16 stores.
 * Returns 0, or -1 for the shapes rope_candle rejects (InvalidOperation)
 * and for odd D.                                                           */
int tlo_rope_cos_sin(const uint16_t* x, int S, int H, int D, const uint16_t* cos_t,
                     const uint16_t* sin_t, int L, uint16_t* y);
/* precompute_rope_cos / precompute_rope_sin builtin_tensor.rs:610-700:
 * theta_i = 1 / base^(2i/D) (f32 powf), angle = pos * theta_i (f32), each
 * value stored twice (columns 2i and 2i+1) in an f32 [L, D] table, then
 * converted to f16.  want_sin selects the table.                           */
void tlo_precompute_rope(int D, int L, float base, int want_sin, uint16_t* out);

/* ---- gather / sampling ----------------------------------------------------
 * embedding builtin_nn.rs:627-812 (+ unified.metal:658-676): row copy.
 * Returns 0, or -1 when an id is out of range (the builtin's bounds check).*/
int tlo_embedding(const uint16_t* table, int vocab, int hidden,
                  const int32_t* ids, int n, uint16_t* out);
/* temperature_sample(logits, T <= 1e-4) builtin_sampling.rs:170-176:
 * argmax with Iterator::max_by, i.e. the LAST of equal maxima wins.        */
int tlo_argmax_last(const uint16_t* logits, int n);
/* temperature_sample(logits, T > 1e-4) builtin_sampling.rs:178-215, for a
 * given draw r in [0, 1): s = x / T, softmax with exp(s - max) summed in
 * index order, p = e / sum, then the first index whose running sum of p
 * (index order, f32) exceeds r, else n - 1.                               */
int tlo_sample_temperature(const uint16_t* logits, int n, float temperature, float r);
/* The draw for (seed, counter): the splitmix64 output of seed +
 * (counter + 1) * 0x9E3779B97F4A7C15, top 24 bits * 2^-24.  (The reference
 * draws from an unseeded rand::thread_rng; this generator makes runs
 * repeatable and is what the device sampler uses.)                         */
float tlo_sample_uniform(uint64_t seed, uint64_t counter);

/* ---- GGUF reader (mmap_gguf.rs:187-379, spec-correct KV skipping) ------ */
typedef struct tlo_gguf tlo_gguf;
tlo_gguf* tlo_gguf_open(const char* path);
void      tlo_gguf_close(tlo_gguf* g);
int       tlo_gguf_n_tensors(const tlo_gguf* g);
/* Looks a tensor up by name.  dims are returned reversed (row-major,
 * gguf.rs:288-291): W[N,K] for a linear weight.  Returns the data pointer
 * (inside the mapped file) or NULL.                                         */
const void* tlo_gguf_tensor(const tlo_gguf* g, const char* name, int* gguf_type,
                            int* ndim, int64_t dims[4], size_t* nbytes);
const char* tlo_gguf_tensor_name(const tlo_gguf* g, int i);
/* Integer / float metadata lookup (0 = found). */
int tlo_gguf_kv_u32(const tlo_gguf* g, const char* key, uint32_t* v);
int tlo_gguf_kv_f32(const tlo_gguf* g, const char* key, float* v);

/* ---- decoder driver ------------------------------------------------------
 * arch 0 = llama (TinyLlama; debug/chat_demo_with_kvcache.tl op sequence,
 * RoPE applied at each token's absolute position, K stored post-RoPE in the
 * cache as model::llama::Cache, llama.rs:78-114);
 * arch 1 = phi2 (LayerNorm, fused QKV with bias, NeoX partial rotary,
 * GELU MLP in parallel with attention: h = (h + attn) + mlp).
 * Weights are read from a GGUF file and dequantised to f16 once at load, as
 * the reference does (gguf.rs:377-412).                                    */
typedef struct tlo_model tlo_model;
tlo_model* tlo_model_load(const char* gguf_path, int arch, int max_ctx, int acc_mode,
                          int n_threads);
void tlo_model_free(tlo_model* m);
/* Runs the prompt (prefill) and then n_decode greedy steps.  tokens_out gets
 * 1 + n_decode ids (the first comes from the prefill logits).  margins_out
 * (optional, 1 + n_decode floats) gets top1 - top2 logit per step.
 * last_logits (optional, vocab f16) gets the logits of the final step.
 * Returns 0 on success.                                                    */
int tlo_model_generate(tlo_model* m, const int32_t* prompt, int n_prompt,
                       int n_decode, int32_t* tokens_out, float* margins_out,
                       uint16_t* last_logits);
/* One forward pass over n tokens at positions pos0.. (appending to the
 * cache); writes the hidden state [n, hidden] after the last layer and the
 * last row's logits. Returns 0 on success.                                 */
int tlo_model_forward(tlo_model* m, const int32_t* ids, int n, int pos0,
                      uint16_t* hidden_out, uint16_t* logits_out);
void tlo_model_reset(tlo_model* m);
/* literal = 1: the op semantics of debug/chat_demo_with_kvcache.tl as
 * written -- rope(x) without an offset, so a single-token forward after the
 * prompt (the decode loop, :236,244) rotates its q and k at position 0
 * (builtin_tensor.rs:531-546) while prompt rows rotate at 0..S-1, and
 * rms_norm(x, w) at the builtin default eps 1e-6 (builtin_nn.rs:84-92).
 * literal = 0 (default): each row at its absolute position, eps from the
 * GGUF file.  llama only; returns -1 for phi2.                             */
int  tlo_model_set_program_semantics(tlo_model* m, int literal);
int  tlo_model_vocab(const tlo_model* m);
int  tlo_model_hidden(const tlo_model* m);

#ifdef __cplusplus
}
#endif
#endif
