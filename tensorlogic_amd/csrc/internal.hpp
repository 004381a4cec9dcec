// internal.hpp -- shared declarations of libtlhip (host side).
//
// Device memory model: every tensor is one allocation from the HIP
// stream-ordered pool (hipMallocAsync on the context stream).  Quantized
// weights are stored structure-of-arrays so that a wavefront streams packed
// blocks with 16-byte loads:
//   Q4_0 [N,K]: qs  = N rows x K/2 bytes (block b of a row at bytes 16b..16b+15,
//                     the GGUF nibble bytes untouched), then
//               d   = N x K/32 f16 scales, at a 256-byte aligned offset.
//   Q8_0 [N,K]: qs  = N rows x K int8, then d as above.
// The byte count is the GGUF one (18 or 34 bytes per 32 weights).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/tl_hip.h"

namespace tlhip {

void set_error(tlhip_status st, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
tlhip_status fail(tlhip_status st, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

#define TLHIP_CHECK_HIP(expr)                                                          \
    do {                                                                               \
        hipError_t e_ = (expr);                                                        \
        if (e_ != hipSuccess)                                                          \
            return ::tlhip::fail(TLHIP_ERR_DEVICE, "%s failed: %s", #expr,            \
                                 hipGetErrorString(e_));                               \
    } while (0)

tlhip_status abi_exception() noexcept;

// Handler of a function-try-block around an exported function's body:
// any host exception becomes a status (see abi_exception).
#define TLHIP_CATCH_STATUS \
    catch (...) {          \
        return ::tlhip::abi_exception(); \
    }
// The same for exported functions that return a value: the value on error.
#define TLHIP_CATCH_VALUE(v)             \
    catch (...) {                        \
        (void)::tlhip::abi_exception();  \
        return v;                        \
    }

#define TLHIP_TRY(expr)                                 \
    do {                                                \
        tlhip_status s_ = (expr);                       \
        if (s_ != TLHIP_OK) return s_;                  \
    } while (0)

struct RopeTable {
    float theta = 0.f;
    int rot_dims = 0;
    int max_pos = 0;
    float* dev = nullptr;   // [max_pos][rot/2][2] (cos, sin)
};

}  // namespace tlhip

struct tlhip_ctx_s {
    // references: the user's handle plus one per live tensor; the context is
    // destroyed when the last one goes (tensors may outlive tlhip_shutdown)
    int refs = 1;
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    bool sync_every_op = false;
    std::vector<tlhip::RopeTable> rope_tables;
    int32_t* d_scratch_i32 = nullptr;   // small scratch for argmax results
    uint32_t* d_tile_flags = nullptr;   // skinny GEMM split counters (zero between launches)
    float* d_ws = nullptr;              // linear's split-K partials, grown on demand
    size_t ws_bytes = 0;
    int32_t* h_pinned_i32 = nullptr;    // pinned host mirror
    // Blocks of freed tensors kept for this context's next allocations,
    // keyed by size class (block_class in runtime.cpp).  Reuse is stream-
    // ordered as hipFreeAsync's is: a block freed on the host is written
    // only by work queued after the free on this context's stream.
    std::mutex cache_mu;
    std::unordered_map<size_t, std::vector<void*>> block_cache;
    size_t cached_bytes = 0;
};

struct tlhip_tensor_s {
    int refcount = 1;
    tlhip_ctx ctx = nullptr;
    tlhip_dtype dtype = TLHIP_F16;
    int ndim = 0;
    int64_t shape[8] = {0};
    void* data = nullptr;       // payload (qs for Q types)
    uint16_t* scales = nullptr; // Q types: f16 scales [N][K/32]
    size_t alloc_bytes = 0;
    tlhip_tensor base = nullptr;  // owner when this is a view
    // Q6_K: the dequantised f16 weight the MFMA GEMM reads (linear with
    // M > 4), made on first use, dropped on upload, freed with the tensor
    tlhip_tensor f16_copy = nullptr;
};

namespace tlhip {

inline int64_t numel(const tlhip_tensor_s* t) {
    int64_t n = 1;
    for (int i = 0; i < t->ndim; i++) n *= t->shape[i];
    return n;
}
inline int64_t last_dim(const tlhip_tensor_s* t) { return t->ndim ? t->shape[t->ndim - 1] : 1; }
inline bool is_quant(tlhip_dtype d) { return d == TLHIP_Q4_0 || d == TLHIP_Q8_0 || d == TLHIP_Q6_K; }
__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
// Device layout of the packed types (rows of N, K along a row):
//   Q4_0 / Q8_0: data = qs rows (K/2 or K bytes each, GGUF payload bytes in
//     block order), then `scales` = f16 d [N][K/32];
//   Q6_K: data = four planes, each 256-aligned: q4 [N][K/2] (per 32-element
//     group: byte i = low 4 bits of elements i | i+16 << 4), q2 [N][K/4]
//     (per group: byte b of word w holds the high 2 bits of elements
//     16w + 4t + b at bits 2t..2t+1), sc [N][K/16] int8 (one per 16
//     elements, natural order); `scales` = f16 d [N][K/256].
inline size_t qs_row_bytes(tlhip_dtype d, int64_t K) { return d == TLHIP_Q8_0 ? (size_t)K : (size_t)K / 2; }
__host__ __device__ inline size_t q6k_q2_offset(int64_t N, int64_t K) { return align256((size_t)N * K / 2); }
__host__ __device__ inline size_t q6k_sc_offset(int64_t N, int64_t K) { return q6k_q2_offset(N, K) + align256((size_t)N * K / 4); }
inline size_t quant_data_bytes(tlhip_dtype d, int64_t N, int64_t K) {
    return d == TLHIP_Q6_K ? q6k_sc_offset(N, K) + align256((size_t)N * K / 16) : align256(qs_row_bytes(d, K) * (size_t)N);
}
inline int64_t quant_scale_count(tlhip_dtype d, int64_t N, int64_t K) { return N * (K / (d == TLHIP_Q6_K ? 256 : 32)); }
inline int64_t quant_group(tlhip_dtype d) { return d == TLHIP_Q6_K ? 256 : 32; }
size_t payload_bytes(tlhip_dtype d, const int64_t* shape, int ndim);
std::string shape_str(const tlhip_tensor_s* t);

tlhip_status check_ctx(tlhip_ctx ctx);
void ctx_release(tlhip_ctx ctx);
tlhip_status check_t(tlhip_tensor t, const char* what);
tlhip_status check_dtype(tlhip_tensor t, tlhip_dtype d, const char* op);
tlhip_status after_launch(tlhip_ctx ctx, const char* op);

// Internal allocation of a tensor (used by ops, model and kvcache code).
tlhip_status alloc_tensor(tlhip_ctx ctx, tlhip_dtype dtype, int ndim, const int64_t* shape,
                          tlhip_tensor* out);

float* ctx_workspace(tlhip_ctx ctx, size_t need);   // the context's grown device workspace (null: none)
// linear(x, W[, b]) behind tlhip_linear (fixed_ws = nullptr: split-K
// partials and the Q6_K f16 copy come from the stream-ordered pool) and
// tlhip_linear_noalloc (fixed_ws = a workspace of fixed_ws_bytes that the
// caller owns; nothing is allocated, Q6_K with M > 4 is refused).
tlhip_status linear_impl(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor w, tlhip_tensor bias, tlhip_tensor y,
                         float* fixed_ws, size_t fixed_ws_bytes);
// Once per device, with that device current (tlhip_init): resolves the
// device address of the no-allocation entry point's workspace.
tlhip_status noalloc_setup(int device);

// RoPE cos/sin table for (theta, rot_dims) covering positions [0, need_pos).
tlhip_status rope_table(tlhip_ctx ctx, float theta, int rot_dims, int need_pos, const float** dev);

bool gguf_lookup(tlhip_gguf g, const char* name, uint32_t* type, int* ndim, int64_t dims[4],
                 const uint8_t** data, size_t* nbytes);

// ---- kernel launchers (kernels_*.hip) --------------------------------------
struct GemvArgs {
    const uint16_t* x = nullptr;   // [M, K] f16
    const void* wq = nullptr;      // qs (Q types) or f16 W
    const uint16_t* wd = nullptr;  // scales (Q types)
    const uint16_t* bias = nullptr;   // [N] f16, optional (EPI_BIAS)
    const uint16_t* resid = nullptr;  // [M, N] f16 (EPI_RESID)
    uint16_t* y = nullptr;
    int M = 1, N = 0, K = 0;
    int ldy = 0;                   // row stride of y (elements), default N
    // fused normalisation prologue (GEMV, M = 1): x is the raw residual row
    int pro = 0;                   // PRO_NONE / PRO_RMS / PRO_LN
    const uint16_t* norm_w = nullptr;
    const uint16_t* norm_b = nullptr;
    float eps = 0.f;
    // EPI_QKV_ROPE: rows [0, nq) are q, [nq, nq+nk) k, [nq+nk, nq+2nk) v
    int nq = 0, nk = 0, head_dim = 0, rot = 0, layout = 0;
    int pos0 = 0;                  // position of activation row 0 (plus *d_pos)
    const float* rope_tab = nullptr;
    const int32_t* d_pos = nullptr;
    uint16_t* q_out = nullptr;     // [M, nq]
    uint16_t* kc = nullptr;        // K cache rows [pos][nk]
    uint16_t* vc = nullptr;        // V cache rows [pos][nk]
    // normalised GEMV only: x row = embd[*d_token] (decode), copied to x_out
    const uint16_t* embd = nullptr;
    const int32_t* d_token = nullptr;
    uint16_t* x_out = nullptr;
    // normalised GEMV with the QKV epilogue: workgroup 0 also writes the f16
    // normalised row here (Phi-2's MLP reads the same layer_norm output)
    uint16_t* xn_out = nullptr;
    // EPI_ARGMAX: one (value, index) key per workgroup, gemv_norm_slots(N) of them
    unsigned long long* amax_slots = nullptr;
    // normalised GEMV with layer_norm (QKV / greedy-key epilogues): the row
    // normalised is f16(x + x_add), and workgroup 0 writes it to x_out
    const uint16_t* x_add = nullptr;
    // GEMM split-K workspace (fp32 partials); none = no split
    float* ws = nullptr;
    size_t ws_bytes = 0;
    // arrival counters of the skinny GEMM's K split (SK_MAX_TILES_SPLIT of
    // them, zero between launches); none = no split across workgroups
    uint32_t* tile_flags = nullptr;
};
// weight-row tiles up to which the skinny GEMM splits K over workgroups (and
// so the counters a context holds for it)
constexpr int SK_MAX_TILES_SPLIT = 128;
// arrival counters of the key-chunked decode attention, one per head, after
// the skinny GEMM's in the context's counter array (zero between launches)
constexpr int ATTN_SPLIT_MAX_HEADS = 1024;
constexpr int CTX_FLAG_WORDS = SK_MAX_TILES_SPLIT + ATTN_SPLIT_MAX_HEADS;
enum GemvPro { PRO_NONE = 0, PRO_RMS = 1, PRO_LN = 2 };
// Epilogues fused into the GEMV/GEMM store (each step rounds to f16 where
// the reference's separate op would store f16):
//   STORE      y = f16(acc)
//   BIAS       y = f16(f16(acc) + b)                 linear(x, W, b)
//   RESID      y = f16(r + f16(acc))                 x + linear(a, W)
//   SWIGLU     rows (2i, 2i+1) = (gate_i, up_i):     silu(gate) * up
//   BIAS_RESID y = f16(r + f16(f16(acc) + b))        x + linear(a, W, b)
//   BIAS_GELU  y = gelu(f16(f16(acc) + b))           gelu(linear(x, W, b))
//   QKV_ROPE   rows (2i, 2i+1) of [q | k | v] (+ bias): RoPE'd q to q_out,
//              RoPE'd k and v into the KV cache at the row's position
//   ARGMAX     y = f16(acc) (+ bias), plus per-workgroup greedy keys
enum GemvEpi { EPI_STORE = 0, EPI_BIAS = 1, EPI_RESID = 2, EPI_SWIGLU_PAIR = 3, EPI_BIAS_RESID = 4,
               EPI_BIAS_GELU = 5, EPI_QKV_ROPE = 6, EPI_ARGMAX = 7 };

tlhip_status launch_gemv(hipStream_t s, tlhip_dtype wt, const GemvArgs& a, int epi);
int gemv_norm_slots(int N);   // workgroups (= argmax keys) of the normalised GEMV
tlhip_status launch_argmax_slots(hipStream_t s, const unsigned long long* slots, int n, int32_t* out,
                                 int32_t* token_log, int32_t* d_state);
tlhip_status launch_gemm(hipStream_t s, tlhip_dtype wt, const GemvArgs& a, int epi);
// y[M,N] = x[M,K] . w[N,K]^T (+ bias[N]) on f32 tensors (linear()'s TensorF32 arm)
tlhip_status launch_linear_f32(hipStream_t s, const float* x, const float* w, const float* bias, float* y, int M, int N,
                               int K);
bool gemm_skinny_ok(int M, int N, int K, int wt);   // the skinny M <= 64 GEMM takes the shape (and EPI_QKV_ROPE)
// Split-K partials (fp32) of any count gemm_splits picks stay within
// GEMM_SPLIT_PARTIALS_MAX bytes: M > 64 keeps tiles x slices <= GEMM_SPLIT_TILE_CAP
// tiles of 128 x 128 (20 MiB); the skinny GEMM (5 <= M <= 64) splits at most
// SK_MAX_TILES_SPLIT tiles (N <= 8192 at 64 rows) into 8 slices (16 MiB); the
// other M <= 64 shapes keep tiles x slices <= 512 tiles of 64 x 64 (8 MiB).
// kernels_gemm.hip ties these figures to its tile constants by static_assert.
constexpr int GEMM_SPLIT_TILE_CAP = 320;
constexpr size_t GEMM_SPLIT_PARTIALS_MAX = (size_t)GEMM_SPLIT_TILE_CAP * 128 * 128 * sizeof(float);
int gemm_splits(int M, int N, int K, int wt);   // split-K slices launch_gemm uses when given a workspace
                                                // (wt < 0: any weight type, the largest count)
uint16_t f32_to_f16(float f);            // host RNE rounding (F32 GGUF tensors)
// Rows 0..src_rows-1 of a GGUF block stream [src_rows, K] go to rows
// dst_row0 + r * dst_step of a packed tensor of dst_rows rows (to_gguf = 1:
// the reverse, packed tensor -> block stream).
tlhip_status launch_repack_rows(hipStream_t s, tlhip_dtype wt, const uint8_t* blocks, void* data,
                                uint16_t* d, int64_t src_rows, int64_t K, int64_t dst_rows, int64_t dst_row0,
                                int64_t dst_step, int to_gguf);
tlhip_status launch_dequant(hipStream_t s, tlhip_dtype wt, const void* qs, const uint16_t* d,
                            uint16_t* out, int64_t N, int64_t K);
tlhip_status launch_rms_norm(hipStream_t s, const uint16_t* x, const uint16_t* w, uint16_t* y,
                             int rows, int n, float eps);
tlhip_status launch_layer_norm(hipStream_t s, const uint16_t* x, const uint16_t* w,
                               const uint16_t* b, uint16_t* y, int rows, int n, float eps);
tlhip_status launch_rope(hipStream_t s, const uint16_t* x, uint16_t* y, int S, int H, int D,
                         int64_t batch, int offset, const int32_t* d_pos, int layout,
                         int rot_dims, const float* table, int x_row_stride, int y_row_stride);
tlhip_status launch_softmax(hipStream_t s, const uint16_t* x, uint16_t* y, int64_t rows, int n);
// the TensorF32 arms (f32 in and out)
tlhip_status launch_rms_norm_f32(hipStream_t s, const float* x, const float* w, float* y, int rows, int n, float eps);
tlhip_status launch_softmax_f32(hipStream_t s, const float* x, float* y, int64_t rows, int n);
tlhip_status launch_rope_f32(hipStream_t s, const float* x, float* y, int S, int H, int D, int64_t batch, int offset,
                             int layout, int rot_dims, const float* table);
tlhip_status launch_sigmoid_f32(hipStream_t s, const float* x, float* y, int64_t n);
tlhip_status launch_scores_f32(hipStream_t s, const float* q, const float* k, float* sc, int I, int J, int H, int Hkv,
                               int D);
tlhip_status launch_context_f32(hipStream_t s, const float* p, const float* v, float* out, int I, int J, int H, int Hkv,
                                int D);
tlhip_status launch_tensor_argmax(hipStream_t s, tlhip_dtype dt, const void* x, void* y, const int64_t* shape, int nd,
                                  int dim);   // dim < 0: whole tensor; y: one element per line
enum EwOp { EW_SIGMOID = 0, EW_SILU = 1, EW_GELU = 2, EW_ADD = 3, EW_MUL = 4, EW_MUL_SCALAR = 5,
            EW_SILU_MUL = 6 };
tlhip_status launch_elementwise(hipStream_t s, int op, const uint16_t* a, const uint16_t* b,
                                uint16_t* y, int64_t n, int64_t b_period, float scalar);
tlhip_status launch_elementwise_f32(hipStream_t s, int op, const float* a, const float* b, float* y, int64_t n,
                                    int64_t b_period, float scalar);
tlhip_status launch_layer_norm_f32(hipStream_t s, const float* x, const float* w, const float* b, float* y, int rows,
                                   int n, float eps);
tlhip_status launch_mask_f32(hipStream_t s, const float* sc, const float* mask, float* y, int64_t n,
                             int64_t mask_period);
tlhip_status launch_embedding_f32(hipStream_t s, const float* table, const int32_t* ids, float* out, int n,
                                  int hidden);
tlhip_status launch_causal_mask(hipStream_t s, uint16_t* out, int64_t n);
// general einsum (f16, general_einsum_cpu's arithmetic): for each output
// element, the operands' element offsets are the sums of coordinate x
// stride over the output indices and the summed indices (nested outermost
// first); sizes and strides in elements.
constexpr int EINSUM_MAX_OPS = 4, EINSUM_MAX_SUM = 8;
struct EinsumPlan {
    int n_ops = 0, n_out = 0, n_sum = 0;
    int64_t out_dim[8] = {};
    int64_t sum_dim[EINSUM_MAX_SUM] = {};
    int64_t out_stride[EINSUM_MAX_OPS][8] = {};
    int64_t sum_stride[EINSUM_MAX_OPS][EINSUM_MAX_SUM] = {};
    const uint16_t* op[EINSUM_MAX_OPS] = {};
};
tlhip_status launch_einsum_general(hipStream_t s, const EinsumPlan& p, uint16_t* out, int64_t n_out, int64_t n_sum);
// broadcast_to: target dims and, per target dim, the input stride (0 where
// the input has size 1 or no dim)
struct BcastDims {
    int nd = 0;
    int64_t shape[8] = {};
    int64_t xstride[8] = {};
};
tlhip_status launch_broadcast(hipStream_t s, const void* x, void* y, int elem, const BcastDims& b);
tlhip_status launch_rope_cs(hipStream_t s, const uint16_t* x, const uint16_t* ct, const uint16_t* st, uint16_t* y,
                            int S, int H, int D);
tlhip_status launch_mask(hipStream_t s, const uint16_t* sc, const uint16_t* mask, uint16_t* y,
                         int64_t n, int64_t mask_period);
tlhip_status launch_embedding(hipStream_t s, tlhip_dtype tt, const void* tq, const uint16_t* td,
                              const int32_t* ids, const int32_t* d_token, uint16_t* out, int n,
                              int hidden, int rows);
tlhip_status launch_argmax(hipStream_t s, const uint16_t* x, int n, int32_t* out,
                           int32_t* token_log, int32_t* d_state);
// temperature_sample with T > 1e-4 (draw from seed and counter
// [+ d_state[2]]); scratch of sample_scratch_bytes(n); d_state / token_log
// as launch_argmax.
size_t sample_scratch_bytes(int n);
tlhip_status launch_sample(hipStream_t s, const uint16_t* x, int n, float temperature, uint64_t seed,
                           uint64_t counter, void* scratch, int32_t* out, int32_t* token_log, int32_t* d_state);
tlhip_status launch_scores(hipStream_t s, const uint16_t* q, const uint16_t* k, uint16_t* sc,
                           int I, int J, int H, int Hkv, int D);
tlhip_status launch_context(hipStream_t s, const uint16_t* p, const uint16_t* v, uint16_t* out,
                            int I, int J, int H, int Hkv, int D);
struct AttnArgs {
    const uint16_t* q = nullptr;  // [S, H, D]
    const uint16_t* k = nullptr;  // [>=J, Hkv, D]
    const uint16_t* v = nullptr;
    uint16_t* out = nullptr;      // [S, H, D]
    int S = 1, H = 0, Hkv = 0, D = 0;
    int q_pos0 = 0;               // position of query row 0
    const int32_t* d_pos = nullptr;  // when set, q_pos0 is read from *d_pos (decode)
    int causal = 1;
    float scale_h = 0.125f;       // f16-rounded scale
    int q_stride = 0, out_stride = 0;  // row strides (elements); 0 = H*D
    int kv_rows = 0;              // rows allocated in k / v (bounds early loads); 0 = J
    uint32_t* head_flags = nullptr;  // key-chunked decode: the context's per-head counters
};
tlhip_status launch_stream_copy(hipStream_t s, const void* src, void* dst, size_t bytes);
tlhip_status launch_transpose(hipStream_t s, const uint16_t* src, uint16_t* dst, int rows, int cols);
tlhip_status launch_transpose_f32(hipStream_t s, const float* src, float* dst, int rows, int cols);
tlhip_status launch_attention(hipStream_t s, const AttnArgs& a);   // decode: J from *d_pos
tlhip_status launch_attention_j(hipStream_t s, const AttnArgs& a, int J);
// Prefill through the matrix cores when attention_mfma_ok(); vt is scratch
// of attention_mfma_scratch() bytes (V transposed per KV head).
bool attention_mfma_ok(const AttnArgs& a, int J);
size_t attention_mfma_scratch(int J, int Hkv, int D);
// Decode attention split over key chunks (head dims 80 / 128, caches of more
// than 512 rows, position read on the device); scratch of
// attention_split_scratch() bytes.
bool attention_split_ok(const AttnArgs& a);
size_t attention_split_scratch(int H, int kv_rows, int D);
tlhip_status launch_attention_split(hipStream_t s, const AttnArgs& a, float* scratch);
// Phi-2's decode step: that split attention and fc1 (GEMV + bias + GELU on
// the normalised row, weight type wt) in one launch; false (nothing
// launched) when the shapes are not the ones it is built for.
bool launch_attention_split_fc1(hipStream_t s, const AttnArgs& a, float* scratch, tlhip_dtype wt, const GemvArgs& f);
// Phi-2's decode step: dense + bias + residual and fc2 + bias (one row
// each) in one launch; false (nothing launched) for other shapes.
bool launch_m1_pair(hipStream_t s, tlhip_dtype wt, const GemvArgs& d, int epi_d, const GemvArgs& f, int epi_f);
// The same split for one query row over J keys known at launch (no device
// position; kv_rows is taken as J); scratch of attention_split_scratch(H, J, D).
bool attention_split_j_ok(const AttnArgs& a, int J);
tlhip_status launch_attention_split_j(hipStream_t s, const AttnArgs& a, int J, float* scratch);
tlhip_status launch_attention_mfma(hipStream_t s, const AttnArgs& a, int J, uint16_t* vt);
constexpr int kAttnRowKeys = 8192;    // keys the one-workgroup kernels hold in their LDS score row
constexpr int kAttnMaxKeys = 65536;   // keys any attention entry point reads (longer rows take the
                                      // key-chunked split for one query row, the matrix cores for more)
tlhip_status launch_copy_rows(hipStream_t s, const uint16_t* src, uint16_t* dst, int rows,
                              int row_elems, int src_stride, int dst_stride, const int32_t* d_pos,
                              int dst_row0);
tlhip_status launch_rope_kv(hipStream_t s, const uint16_t* qkv, int qkv_stride, int S, int H,
                            int Hkv, int D, int layout, int rot_dims, const float* table,
                            int pos0, const int32_t* d_pos, uint16_t* q_out, uint16_t* kcache,
                            uint16_t* vcache);

}  // namespace tlhip
