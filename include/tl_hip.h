/*
 * tl_hip.h -- C ABI of libtlhip.so, the MI355X (gfx950) device backend for
 * TensorLogic's quantized-LLM hot path.
 *
 * This header replaces the Metal device contract under the reference's
 * src/device/ and the tensor operator surface the TL interpreter calls.
 * Each entry point names the reference function it stands in for.
 *
 * Conventions
 *  - Every function returns tlhip_status (0 = OK).  On error nothing was
 *    launched; tlhip_last_error() returns a thread-local message.  Error
 *    codes mirror the reference's TensorError variants (src/error.rs:9-49).
 *  - One context = one device + one HIP stream.  All launches are
 *    asynchronous on that stream; tlhip_tensor_download, tlhip_argmax and
 *    tlhip_sync wait.  Calls on one context are not thread-safe; separate
 *    contexts may be used from separate threads.
 *  - Tensors are opaque, reference-counted (tlhip_tensor_retain/free).  A
 *    free is stream-ordered: memory returns to the pool after the work
 *    already queued on the context's stream, with no host fence (replaces
 *    the GPU fence + buffer-pool recycle of src/tensor/tensor.rs:58-121).
 *  - Shapes are row-major (reference order).  A linear weight is W[N, K].
 *  - Quantized tensors (Q4_0, Q8_0) are uploaded as GGUF block bytes and
 *    stay packed and device-resident (no dequantise-on-load).
 *  - Host buffers in upload/download are plain host memory; sizes in bytes.
 */
#ifndef TL_HIP_H
#define TL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    TLHIP_OK = 0,
    TLHIP_ERR_SHAPE_MISMATCH = 1,     /* TensorError::ShapeMismatch */
    TLHIP_ERR_INVALID_DIMENSION = 2,  /* TensorError::InvalidDimension */
    TLHIP_ERR_INVALID_OPERATION = 3,  /* TensorError::InvalidOperation */
    TLHIP_ERR_ALLOCATION = 4,         /* TensorError::AllocationError */
    TLHIP_ERR_INDEX_OUT_OF_BOUNDS = 5,/* TensorError::IndexOutOfBounds */
    TLHIP_ERR_LOAD = 6,               /* TensorError::LoadError (GGUF) */
    TLHIP_ERR_DEVICE = 7,             /* TensorError::MetalError -> HIP error */
    TLHIP_ERR_DTYPE = 8,              /* unsupported dtype for the op */
    TLHIP_ERR_INVALID_ARGUMENT = 9    /* NULL handle, bad enum, ... */
} tlhip_status;

typedef enum {
    TLHIP_F16 = 0,
    TLHIP_F32 = 1,
    TLHIP_I32 = 2,
    TLHIP_Q4_0 = 3,   /* GGUF Q4_0: 32-element blocks along K, 18 B/block */
    TLHIP_Q8_0 = 4,   /* GGUF Q8_0: 32-element blocks along K, 34 B/block */
    TLHIP_Q6_K = 5    /* GGUF Q6_K: 256-element super-blocks, 210 B each
                         (dequantize_q6_k, gguf.rs:128-212)               */
} tlhip_dtype;

typedef enum {
    TLHIP_ROPE_INTERLEAVED = 0,  /* pairs (2i, 2i+1): rope_f16 unified.metal:2355-2418 */
    TLHIP_ROPE_NEOX = 1          /* pairs (i, i+rot/2), partial rotary allowed */
} tlhip_rope_layout;

typedef struct tlhip_ctx_s* tlhip_ctx;
typedef struct tlhip_tensor_s* tlhip_tensor;
typedef struct tlhip_gguf_s* tlhip_gguf;
typedef struct tlhip_model_s* tlhip_model;

/* ---- errors / context ---------------------------------------------------- */
/* Thread-local text of the last error (TensorError Display, src/error.rs). */
const char* tlhip_last_error(void);
/* MetalDevice::new() singleton (src/device/metal_device.rs:36-74): picks a
 * device, creates the stream.  device < 0 selects device 0.                */
tlhip_status tlhip_init(int device, tlhip_ctx* out);
tlhip_status tlhip_shutdown(tlhip_ctx ctx);
/* wait_until_completed() (metal_device.rs:195-200). */
tlhip_status tlhip_sync(tlhip_ctx ctx);
/* Name of the device (e.g. "AMD Instinct MI355X") and its gfx target. */
tlhip_status tlhip_device_name(tlhip_ctx ctx, char* buf, size_t len);
/* Debug: synchronise and check after every op (the build's counterpart of
 * the reference's TL_DEBUG* env switches).  Also enabled by the
 * environment variable TLHIP_SYNC_EVERY_OP=1.                              */
tlhip_status tlhip_set_sync_every_op(tlhip_ctx ctx, int on);

/* ---- tensors ------------------------------------------------------------- */
/* MetalBuffer::new_uninit_pooled (metal_buffer.rs:213): device allocation
 * from the stream-ordered pool.  For Q4_0/Q8_0, ndim must be 2 and shape
 * [N, K] with K % 32 == 0; for Q6_K, K % 256 == 0.                        */
tlhip_status tlhip_tensor_alloc(tlhip_ctx ctx, tlhip_dtype dtype, int ndim,
                                const int64_t* shape, tlhip_tensor* out);
/* MetalBuffer::from_slice (metal_buffer.rs:37) / Tensor::from_vec_gpu
 * (tensor_creation.rs:126).  bytes must equal tlhip_tensor_nbytes(t); for
 * Q types the host data is GGUF block bytes in file order.                 */
tlhip_status tlhip_tensor_upload(tlhip_ctx ctx, tlhip_tensor t, const void* host, size_t bytes);
/* MetalBuffer::to_vec (metal_buffer.rs:113) via sync_and_read
 * (tensor_io.rs:103-117): waits for queued work, then copies.  Q types are
 * returned as GGUF block bytes.                                            */
tlhip_status tlhip_tensor_download(tlhip_ctx ctx, tlhip_tensor t, void* host, size_t bytes);
tlhip_status tlhip_tensor_retain(tlhip_tensor t);
tlhip_status tlhip_tensor_free(tlhip_tensor t);
/* Shape / dtype query (TensorAccessors::dims). shape has room for 8 dims. */
tlhip_status tlhip_tensor_info(tlhip_tensor t, tlhip_dtype* dtype, int* ndim, int64_t* shape);
size_t tlhip_tensor_nbytes(tlhip_tensor t);
/* Metadata-only reshape (Tensor::reshape): returns a new handle sharing
 * the storage; element count must match.  Not allowed for Q types.        */
tlhip_status tlhip_tensor_reshape(tlhip_tensor t, int ndim, const int64_t* shape, tlhip_tensor* out);

/* ---- GGUF ------------------------------------------------------------------ */
/* MmapGGUFLoader::new / parse_header (mmap_gguf.rs:120-275), spec-correct. */
tlhip_status tlhip_gguf_open(const char* path, tlhip_gguf* out);
tlhip_status tlhip_gguf_close(tlhip_gguf g);
int tlhip_gguf_n_tensors(tlhip_gguf g);
const char* tlhip_gguf_tensor_name(tlhip_gguf g, int i);
/* get_tensor(model, name) (builtin_model.rs:204) without dequantisation:
 * F16/F32 tensors upload as F16 (F32 rounded RNE), Q4_0/Q8_0 stay packed.
 * Replaces GGUFLoader::load's per-tensor dequantize (gguf.rs:256-464).    */
tlhip_status tlhip_gguf_load_tensor(tlhip_ctx ctx, tlhip_gguf g, const char* name, tlhip_tensor* out);
tlhip_status tlhip_gguf_kv_u32(tlhip_gguf g, const char* key, uint32_t* v);
tlhip_status tlhip_gguf_kv_f32(tlhip_gguf g, const char* key, float* v);

/* ---- operators (Tensor methods / TL builtins) ---------------------------- */
/* dequantize_q4_0 / dequantize_q8_0 / dequantize_q6_k (gguf.rs:22-212,
 * mmap_gguf.rs:383-545) on the device: q [N,K] packed -> out [N,K] f16,
 * bit-exact.                                                              */
tlhip_status tlhip_dequantize(tlhip_ctx ctx, tlhip_tensor q, tlhip_tensor out_f16);
/* linear(x, W[, b]) (builtin_math.rs:76-131) = matmul_transposed_b
 * (matmul.rs:241-458) then add(bias): y[M,N] = x[M,K] W[N,K]^T, fp32
 * accumulation, f16 out.  W may be F16, Q4_0, Q8_0 or Q6_K; M <= 4 uses
 * the fused dequant-GEMV, larger M the MFMA dequant-GEMM (a Q6_K weight
 * keeps the dequantised f16 copy that GEMM reads, 2 bytes per weight, from
 * its first use with M > 4 until it is freed or re-uploaded).  bias may be
 * NULL.  The TensorF32 arm (builtin_math.rs:121-175): x, W, bias and y all
 * F32, each output the sum of the reference's f32 kernel
 * (matmul_transposed_b_tiled_32x32_f32, unified.metal:4409-4461: k in
 * order, one fused multiply-add per term, zero terms to a multiple of 32)
 * plus the bias; f16 mixed with f32 is a DtypeError.                      */
tlhip_status tlhip_linear(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor w, tlhip_tensor bias, tlhip_tensor y);
/* linear(x, W[, b]) exactly as tlhip_linear (same checks, kernels and bits),
 * but allocating nothing: no counterpart in the reference.  It is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The split-K
 * partials of the MFMA GEMM live in a 20 MiB device array that each GPU holds
 * from library load to process end (partials beyond it -> AllocationError;
 * the library's split policy needs at most 20 MiB: 320 tiles of 128 x 128
 * fp32 over all slices, e.g. [512 x 10240] @ [2560 x 10240]^T in 4 slices).
 * Its device address is resolved by tlhip_init, or on the first call if that
 * failed (a failure is reported by this call only).  A Q6_K weight with
 * M > 4 needs a dequantised f16 copy and is refused (InvalidOperation).  All
 * calls on one GPU share that array: calls overlapping in time on one GPU
 * (several contexts or threads) race and must be serialised by the caller. */
tlhip_status tlhip_linear_noalloc(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor w, tlhip_tensor bias, tlhip_tensor y);
/* matmul(a, b) (builtin_math.rs:36-60, matmul.rs:22-197): c[M,N] = a[M,K] b[K,N],
 * all f16 or all f32 (a mix: DtypeError); rank != 2 or an inner-dimension
 * mismatch: InvalidOperation, as Tensor::matmul returns. */
tlhip_status tlhip_matmul(tlhip_ctx ctx, tlhip_tensor a, tlhip_tensor b, tlhip_tensor c);
/* rms_norm(x, w[, eps]) (builtin_nn.rs:44-103, normalization.rs:42-250)
 * over the last dim.  x, w, y all f16, or all f32 (the TensorF32 arm,
 * rms_norm_simple_f32 / rms_norm_f32, unified.metal:1961-2036).            */
tlhip_status tlhip_rms_norm(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor w, float eps, tlhip_tensor y);
/* layer_norm (normalization.rs:271-535); w and b may be NULL.  All f16, or
 * all f32 (layer_norm_f32 / layer_norm_simple_f32, unified.metal:1833-1958:
 * per-row sums in element order).                                          */
tlhip_status tlhip_layer_norm(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor w, tlhip_tensor b, float eps, tlhip_tensor y);
/* rope(x[, offset]) (builtin_tensor.rs:514-556, rope.rs:71-300): x [..,S,H,D].
 * rot_dims 0 = D.  The reference's rope() is layout INTERLEAVED, theta 10000.
 * x and y both f16, or both f32 (rope_f32, unified.metal:2420-2482).       */
tlhip_status tlhip_rope(tlhip_ctx ctx, tlhip_tensor x, int offset, float theta,
                        tlhip_rope_layout layout, int rot_dims, tlhip_tensor y);
/* softmax(x) over the last dim (activations.rs:107-230); x and y both f16,
 * or both f32 (softmax_simple_f32 / softmax_f32, unified.metal:2202-2340). */
tlhip_status tlhip_softmax_lastdim(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor y);
/* sigmoid (activations.rs:239-266; f16, or f32 in and out: sigmoid_f32,
 * unified.metal:1129-1135); silu = x * sigmoid(x) as the TL function silu
 * (chat_demo_optimized.tl:35-37); silu_mul = silu(g) * u (swiglu_ffn's
 * intermediate); gelu (tanh form, unified.metal:837-848; f32: gelu_f32,
 * :1051-1062).  Each takes all-f16 or all-f32 operands.                   */
tlhip_status tlhip_sigmoid(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor y);
tlhip_status tlhip_silu(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor y);
tlhip_status tlhip_silu_mul(tlhip_ctx ctx, tlhip_tensor gate, tlhip_tensor up, tlhip_tensor y);
tlhip_status tlhip_gelu(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor y);
/* add / mul (elementwise.rs, add_f16/mul_f16 unified.metal:701-729; f32:
 * add_f32/mul_f32, :934-962); b may be a 1-D tensor matching a's last dim
 * (row broadcast, as bias).  All f16 or all f32.                          */
tlhip_status tlhip_add(tlhip_ctx ctx, tlhip_tensor a, tlhip_tensor b, tlhip_tensor y);
tlhip_status tlhip_mul(tlhip_ctx ctx, tlhip_tensor a, tlhip_tensor b, tlhip_tensor y);
/* tensor * scalar (mul_scalar(scalar: T), elementwise.rs:724-780): for an
 * f16 tensor the scalar is rounded to f16 first; for an f32 tensor it is
 * used as given (mul_scalar_f32, unified.metal:984-992).                  */
tlhip_status tlhip_mul_scalar(tlhip_ctx ctx, tlhip_tensor a, float s, tlhip_tensor y);
/* embedding(table, ids) (builtin_nn.rs:627-812): table [V,H] F16/Q4_0/Q8_0/Q6_K,
 * ids host int32[n] (bounds-checked on the host), out [n,H] f16; an F32
 * table gives f32 rows (embedding_lookup_f32, unified.metal:678-694).     */
tlhip_status tlhip_embedding(tlhip_ctx ctx, tlhip_tensor table, const int32_t* ids, int n, tlhip_tensor out);
/* apply_attention_mask(scores, mask) (masking.rs:36-51,147-165): where
 * mask == 0 the score becomes -10000.  mask broadcasts over leading dims.
 * All f16, or all f32 (apply_attention_mask_f32, unified.metal:4491-4503). */
tlhip_status tlhip_apply_attention_mask(tlhip_ctx ctx, tlhip_tensor scores, tlhip_tensor mask, tlhip_tensor y);
/* causal_mask(n) (builtin_nn.rs:423-460, masking.rs:192-207): out [n, n]
 * f16 = 1 where j <= i, else 0.                                          */
tlhip_status tlhip_causal_mask(tlhip_ctx ctx, tlhip_tensor out);
/* slice_last(x, axis) (builtin_tensor.rs:1949-1991, slice.rs:25-60): the
 * last index of axis 0, y = x's shape without axis 0 ([1] for a 1-D x,
 * where the reference returns a scalar).  axis != 0 -> InvalidOperation,
 * as in the reference.  F16 / F32 / I32.                                 */
tlhip_status tlhip_slice_last(tlhip_ctx ctx, tlhip_tensor x, int axis, tlhip_tensor y);
/* broadcast_to(x, shape) (broadcast.rs:11-120, shape.rs:37-49): y's shape is
 * the target; dims align from the right, an input dim of 1 repeats, else
 * ShapeMismatch.  F16 / F32 / I32.                                        */
tlhip_status tlhip_broadcast_to(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor y);
/* rope(x, cos, sin) (builtin_tensor.rs:569-597) = Tensor::rope_candle
 * (rope.rs:18-65, rope_candle_f16 unified.metal:5122-5185): x [S, H, D],
 * cos/sin [L >= S, D] f16; pair i of row s is rotated by cos[s, i] and
 * sin[s, i] -- column i, as the reference's kernel indexes the table.    */
tlhip_status tlhip_rope_cos_sin(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor cos_t, tlhip_tensor sin_t, tlhip_tensor y);
/* precompute_rope_cos / _sin(head_dim, max_seq_len, base)
 * (builtin_tensor.rs:610-700): out [max_seq_len, head_dim] f16, value of
 * pair i at columns 2i and 2i+1.  Synchronous.                           */
tlhip_status tlhip_precompute_rope(tlhip_ctx ctx, int head_dim, int max_seq_len, float base, int want_sin,
                                   tlhip_tensor out);
/* einsum("ihd,jhd->ihj") and einsum("ihj,jhd->ihd") (einsum.rs:653-886),
 * fp32 accumulation, f16 out; or all operands f32 (einsum_ihd_jhd_ihj_f32 /
 * einsum_ihj_jhd_ihd_f32, unified.metal:2702-2768: fused sums in index
 * order).  K/V may carry fewer heads than Q (GQA: head h reads
 * h / (H/Hkv)), replacing broadcast_to + contiguous.                      */
tlhip_status tlhip_einsum_scores(tlhip_ctx ctx, tlhip_tensor q, tlhip_tensor k, tlhip_tensor scores);
tlhip_status tlhip_einsum_context(tlhip_ctx ctx, tlhip_tensor p, tlhip_tensor v, tlhip_tensor out);
/* einsum(equation, operands...) (eval.rs:3264-3318 -> Tensor::einsum,
 * einsum.rs:39-82), parsed as the reference parses it (einsum.rs:84-128:
 * at most one "->"; without it the output is every index occurring once,
 * sorted).  "ihd,jhd->ihj" / "ihj,jhd->ihd" on rank-3 operands are
 * tlhip_einsum_scores / tlhip_einsum_context (the reference's Metal path,
 * f16 or f32).  Every other equation (the reference's Metal path panics on
 * them) computes general_einsum_cpu (einsum.rs:207-333) on f16 operands:
 * per output element, products in operand order and sums over the summed
 * indices nested outermost first, every step rounded to f16.  The
 * reference nests two or more summed indices in HashSet order, which Rust
 * randomises per process; here they nest in order of first appearance in
 * the inputs.  Up to 4 operands, 8 output and 8 summed indices, at most
 * 2^31 summed terms per output element and 2^36 in all (one thread walks
 * an element's terms); a scalar result is a [1] tensor.  Errors: operand count -> InvalidOperation, mixed
 * f16 / f32 -> DtypeError (the reference's TypeError), a repeated index of
 * two sizes -> ShapeMismatch, unknown output index or a spec whose length
 * is not the operand's rank -> InvalidOperation; f32 operands of a general
 * equation -> InvalidOperation.  tlhip_einsum_shape gives the output shape
 * (ndim and up to 8 dims) without launching anything.                     */
tlhip_status tlhip_einsum_shape(const char* equation, const tlhip_tensor* operands, int n_operands, int* ndim,
                                int64_t* shape);
tlhip_status tlhip_einsum(tlhip_ctx ctx, const char* equation, const tlhip_tensor* operands, int n_operands,
                          tlhip_tensor out);
/* Fused attention = einsum scores -> * scale (f16) -> causal mask (-10000)
 * -> softmax -> einsum context, with the reference's f16 storage points.
 * q [S,H,D]; k, v [J,Hkv,D] (a KV cache's first J rows); query row s sits
 * at position q_pos0 + s.  causal = 0 attends to all J keys.              */
tlhip_status tlhip_attention(tlhip_ctx ctx, tlhip_tensor q, tlhip_tensor k, tlhip_tensor v,
                             int q_pos0, float scale, int causal, tlhip_tensor out);
/* temperature_sample(logits, T<=1e-4) argmax (builtin_sampling.rs:170-176):
 * last maximum wins; logits [V] or [S,V] (last row).  Synchronous.        */
tlhip_status tlhip_argmax(tlhip_ctx ctx, tlhip_tensor logits, int32_t* out);
/* argmax(x[, dim[, keepdim]]) = Tensor::argmax(dim, keepdim) (reduce.rs:585-668;
 * builtin_tensor.rs:1438-1490): index of the FIRST largest value (a strict '>'
 * scan; NaN never wins, and neither does -inf along a dim), stored in x's own
 * dtype (f16 or f32) as the reference's T::from_f64(index).  dim < 0: the
 * whole tensor, y of shape [1] (keepdim: [1] * rank); else y has x's shape
 * without dim (keepdim: dim of size 1), reducing the only dim without keepdim
 * is a shape error as in the reference, and output element o is the line
 * whose kept coordinates are o's digits with the first kept dim least
 * significant (the reference's own index order).  The builtin's integer
 * result (no dim, no keepdim) is y's one element.                         */
tlhip_status tlhip_tensor_argmax(tlhip_ctx ctx, tlhip_tensor x, int dim, int keepdim, tlhip_tensor y);
/* temperature_sample(logits, T) (builtin_sampling.rs:66-231): T <= 1e-4 is
 * tlhip_argmax; otherwise softmax(x / T) and the inverse-CDF index of one
 * uniform draw, V <= 2^20.  The reference draws from an unseeded
 * thread_rng; here the draw is splitmix64(seed, counter), so a (seed,
 * counter) pair always picks the same token.  Synchronous.                 */
tlhip_status tlhip_temperature_sample(tlhip_ctx ctx, tlhip_tensor logits, float temperature, uint64_t seed,
                                      uint64_t counter, int32_t* out);

/* ---- KV cache (model::llama::Cache, llama.rs:50-114; KVCache builtins
 *      eval.rs:1247-1400), preallocated instead of concat-grown ----------- */
typedef struct tlhip_kvcache_s* tlhip_kvcache;
/* KVCache::new_f16(n_layers) with room for max_ctx rows of [Hkv, D];
 * max_ctx <= 65536, the most keys the attention entry points read
 * (InvalidDimension beyond).  The reference grows its cache without a cap
 * (llama.rs:87-88); past 8192 keys a single query row is attended in key
 * chunks and several rows on the matrix cores (head dims 64 / 80 / 128).  */
tlhip_status tlhip_kvcache_create(tlhip_ctx ctx, int n_layers, int max_ctx, int n_kv_heads,
                                  int head_dim, tlhip_kvcache* out);
/* KVCache::new_f32(n_layers) (eval.rs:942; set / append / get_k / get_v at
 * eval.rs:1302,1422,1506,1582): the same cache holding f32 rows; its set /
 * append take f32 K, V and get returns f32 views.  The attention entry
 * points below are f16 (a DtypeError on an f32 cache).                    */
tlhip_status tlhip_kvcache_create_f32(tlhip_ctx ctx, int n_layers, int max_ctx, int n_kv_heads,
                                      int head_dim, tlhip_kvcache* out);
tlhip_status tlhip_kvcache_free(tlhip_kvcache c);
/* cache.set(layer, K, V): replaces the layer's contents with K,V [S,Hkv,D]
 * (K and V of the same shape, else ShapeMismatch).                       */
tlhip_status tlhip_kvcache_set(tlhip_ctx ctx, tlhip_kvcache c, int layer, tlhip_tensor k, tlhip_tensor v);
/* cache.append(layer, K, V): appends S rows. */
tlhip_status tlhip_kvcache_append(tlhip_ctx ctx, tlhip_kvcache c, int layer, tlhip_tensor k, tlhip_tensor v);
/* cache.get_k / get_v: a view [len, Hkv, D] of the layer's rows (shares
 * storage; later appends do not change the view's length).               */
tlhip_status tlhip_kvcache_get(tlhip_kvcache c, int layer, int which_v, tlhip_tensor* out);
int tlhip_kvcache_len(tlhip_kvcache c, int layer);
/* Attention against a cache layer after cache.append -- the TL program's
 * get_k / get_v followed by einsum, scale, causal mask, softmax, einsum
 * (chat_demo_with_kvcache.tl, einsum.rs:653-886, masking.rs:147-165,
 * activations.rs:107-230): q [S, H, D] are the queries of the cache's last
 * S positions (len - S .. len - 1), causal; out [S, H, D].  _decode takes
 * the single new row (S = 1).  Same kernels and bars as tlhip_attention. */
tlhip_status tlhip_attention_prefill(tlhip_ctx ctx, tlhip_tensor q, tlhip_kvcache c, int layer, float scale,
                                     tlhip_tensor out);
tlhip_status tlhip_attention_decode(tlhip_ctx ctx, tlhip_tensor q, tlhip_kvcache c, int layer, float scale,
                                    tlhip_tensor out);

/* ---- decoder runner (the op sequence of debug/chat_demo_with_kvcache.tl,
 *      fused; arch 0 = llama/TinyLlama, 1 = phi2) ------------------------- */
tlhip_status tlhip_model_load(tlhip_ctx ctx, const char* gguf_path, int arch, int max_ctx,
                              tlhip_model* out);
tlhip_status tlhip_model_free(tlhip_model m);
tlhip_status tlhip_model_reset(tlhip_model m);
/* Prompt pass at positions [pos, pos+n): fills the cache and samples the
 * next token greedily (temperature_sample with T = 0).                   */
tlhip_status tlhip_model_prefill(tlhip_model m, const int32_t* ids, int n, int32_t* next_token);
/* One decode step for `token` at the current position; returns the next. */
tlhip_status tlhip_model_decode(tlhip_model m, int32_t token, int32_t* next_token);
/* prefill(prompt) then n_decode greedy steps; tokens_out gets 1 + n_decode
 * ids.  use_graph = 1 replays captured HIP graphs (one of 8 steps while 8
 * or more remain, then one of 1 step), with the token and position kept on
 * the device (no per-token host sync).                                    */
tlhip_status tlhip_model_generate(tlhip_model m, const int32_t* prompt, int n_prompt,
                                  int n_decode, int use_graph, int32_t* tokens_out);
/* Copies the last computed logits row (f16, vocab entries) to host.       */
tlhip_status tlhip_model_logits(tlhip_model m, uint16_t* host, size_t n);
/* Op semantics of the TL program the runner stands for (llama only).
 * literal = 0 (default): RoPE at each token's absolute position, as
 * rope(x, offset) allows (builtin_tensor.rs:514-556), and RMSNorm at the
 * GGUF file's eps (llama.attention.layer_norm_rms_epsilon).  literal = 1:
 * debug/chat_demo_with_kvcache.tl as written -- rope(x) with no offset in
 * its decode loop (:236,244) rotates every decode row as position 0, and
 * rms_norm(x, w) uses the builtin default eps 1e-6 (builtin_nn.rs:84-92);
 * prompt rows rotate at their positions either way.  Phi-2 ->
 * InvalidOperation.                                                       */
tlhip_status tlhip_model_set_program_semantics(tlhip_model m, int literal);
/* Architecture numbers: [n_layers, hidden, inter, n_heads, n_kv, head_dim, vocab, rot_dims]. */
tlhip_status tlhip_model_dims(tlhip_model m, int32_t* dims8);
/* The decode's token choice, temperature_sample(logits, T) as the chat
 * loop calls it (chat_demo_optimized.tl:204,239; builtin_sampling.rs:
 * 66-231): T <= 1e-4 greedy (the default), else a draw per step from
 * splitmix64(seed, step) on the device, inside the replayed graph.        */
tlhip_status tlhip_model_set_sampling(tlhip_model m, float temperature, uint64_t seed);

/* ---- measurement helpers (hipEvent timing on the context's stream) ------ */
/* Runs linear(x, w) `iters` times cycling over n_w weight tensors of equal
 * shape (to defeat the LLC) and returns the mean time per launch in us from
 * hipEvents on the context stream: per_launch = 0 brackets the whole
 * back-to-back sequence (throughput, gaps between launches included);
 * per_launch = 1 brackets every launch with its own event pair.           */
tlhip_status tlhip_bench_linear(tlhip_ctx ctx, tlhip_tensor x, const tlhip_tensor* w, int n_w,
                                tlhip_tensor y, int iters, int per_launch, float* avg_us);
/* Copies `bytes` (multiple of 16) from one of n_buf source buffers to one
 * destination `iters` times with a plain 16-byte-per-lane copy kernel, back
 * to back, and returns the mean us per copy (hipEvents): the streaming
 * bandwidth reference of the device and the known-size kernel that scales
 * the profiler's HBM byte counters.  Allocates and frees its own buffers. */
tlhip_status tlhip_bench_copy(tlhip_ctx ctx, size_t bytes, int n_buf, int iters, float* avg_us);
/* Times `n_decode` greedy steps after a prefill (use_graph = 1: captured
 * HIP graphs of 8 and 1 steps replayed, as tlhip_model_generate, captured
 * before the timed region; 0: the same kernels launched one by one);
 * returns the prefill and total decode ms (hipEvents on the context
 * stream) and the 1 + n_decode tokens.                                    */
tlhip_status tlhip_bench_decode(tlhip_model m, const int32_t* prompt, int n_prompt, int n_decode,
                                int use_graph, int32_t* tokens_out, float* prefill_ms, float* decode_ms);
/* Event pair on the context stream around any sequence of asynchronous
 * calls: timer_start records the first event; timer_stop records the
 * second, waits for it and returns the elapsed ms.                       */
tlhip_status tlhip_timer_start(tlhip_ctx ctx);
tlhip_status tlhip_timer_stop(tlhip_ctx ctx, float* ms);

#ifdef __cplusplus
}
#endif
#endif /* TL_HIP_H */
