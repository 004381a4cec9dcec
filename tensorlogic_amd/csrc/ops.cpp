// ops.cpp -- C-ABI operator entry points: host-side shape/dtype checks
// (the reference checks shapes in Rust before encoding, e.g. matmul.rs:
// 249-280), then one or more stream-ordered launches.  Nothing is launched
// when a check fails.
#include <cmath>
#include <cstring>
#include <vector>

#include "internal.hpp"

using namespace tlhip;

namespace {

tlhip_status same_shape(tlhip_tensor a, tlhip_tensor b, const char* op) {
    if (a->ndim != b->ndim || memcmp(a->shape, b->shape, sizeof(int64_t) * a->ndim) != 0)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "%s: shape %s vs %s", op, shape_str(a).c_str(),
                    shape_str(b).c_str());
    return TLHIP_OK;
}

tlhip_status f16_args(const char* op, std::initializer_list<tlhip_tensor> ts) {
    for (tlhip_tensor t : ts) {
        TLHIP_TRY(check_t(t, op));
        TLHIP_TRY(check_dtype(t, TLHIP_F16, op));
    }
    return TLHIP_OK;
}

uint16_t* P(tlhip_tensor t) { return (uint16_t*)t->data; }
float* F(tlhip_tensor t) { return (float*)t->data; }

// Operands of an op with a TensorF16 and a TensorF32 arm: all F16 or all F32
// (a mix is the reference's TypeError); *f32 tells which.
tlhip_status float_args(const char* op, std::initializer_list<tlhip_tensor> ts, bool* f32) {
    const tlhip_tensor first = *ts.begin();
    TLHIP_TRY(check_t(first, op));
    *f32 = first->dtype == TLHIP_F32;
    for (tlhip_tensor t : ts) {
        TLHIP_TRY(check_t(t, op));
        TLHIP_TRY(check_dtype(t, *f32 ? TLHIP_F32 : TLHIP_F16, op));
    }
    return TLHIP_OK;
}

float round_f16(float f) {
    // scalar operands of f16 ops are f16 values (T::from_f32)
    _Float16 h = (_Float16)f;
    return (float)h;
}

}  // namespace

extern "C" {

tlhip_status tlhip_dequantize(tlhip_ctx ctx, tlhip_tensor q, tlhip_tensor out) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(check_t(q, "dequantize"));
    TLHIP_TRY(f16_args("dequantize", {out}));
    if (!is_quant(q->dtype)) return fail(TLHIP_ERR_DTYPE, "dequantize: input must be Q4_0, Q8_0 or Q6_K");
    if (out->ndim != 2 || out->shape[0] != q->shape[0] || out->shape[1] != q->shape[1])
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "dequantize: %s -> %s", shape_str(q).c_str(), shape_str(out).c_str());
    TLHIP_TRY(launch_dequant(ctx->stream, q->dtype, q->data, q->scales, P(out), q->shape[0], q->shape[1]));
    return after_launch(ctx, "dequantize");
} TLHIP_CATCH_STATUS

tlhip_status tlhip_linear(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor w, tlhip_tensor bias, tlhip_tensor y) try {
    return linear_impl(ctx, x, w, bias, y, nullptr, 0);
} TLHIP_CATCH_STATUS

}  // extern "C"

namespace tlhip {

// The context's device workspace (split-K partials, attention scratch),
// grown stream-ordered when a call needs more, so steady-state calls
// allocate nothing; null when it cannot grow.  Calls on the context's
// stream use it one after another.
float* ctx_workspace(tlhip_ctx ctx, size_t need) {
    if (need > ctx->ws_bytes) {
        void* grown = nullptr;
        if (hipMallocAsync(&grown, need, ctx->stream) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        if (ctx->d_ws) (void)hipFreeAsync(ctx->d_ws, ctx->stream);   // after the calls that used it
        ctx->d_ws = (float*)grown;
        ctx->ws_bytes = need;
    }
    return ctx->d_ws;
}

// linear() on TensorF32 operands (builtin_math.rs:121-175): x [M, K], w [N, K],
// bias [N] and y [M, N] all f32; a mix of f16 and f32 is the reference's
// TypeError (a dtype error here).
static tlhip_status linear_f32(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor w, tlhip_tensor bias, tlhip_tensor y) {
    TLHIP_TRY(check_t(w, "linear weight"));
    TLHIP_TRY(check_t(y, "linear output"));
    if (w->dtype != TLHIP_F32 || y->dtype != TLHIP_F32 || (bias && bias->dtype != TLHIP_F32))
        return fail(TLHIP_ERR_DTYPE, "linear(): f32 input needs f32 weight, bias and output");
    if (x->ndim != 2 || w->ndim != 2)
        return fail(TLHIP_ERR_INVALID_OPERATION, "matmul_transposed_b requires 2D tensors");
    const int64_t M = x->shape[0], K = x->shape[1], N = w->shape[0];
    if (w->shape[1] != K)
        return fail(TLHIP_ERR_INVALID_OPERATION, "matmul_transposed_b shape mismatch: [%lld, %lld] @ [%lld, %lld].T",
                    (long long)M, (long long)K, (long long)N, (long long)w->shape[1]);
    if (y->ndim != 2 || y->shape[0] != M || y->shape[1] != N)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "linear: output %s for [%lld, %lld]", shape_str(y).c_str(),
                    (long long)M, (long long)N);
    if (bias && (bias->ndim != 1 || bias->shape[0] != N))
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "linear: bias %s for %lld outputs", shape_str(bias).c_str(), (long long)N);
    if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return fail(TLHIP_ERR_INVALID_DIMENSION, "linear: too large");
    TLHIP_TRY(launch_linear_f32(ctx->stream, (const float*)x->data, (const float*)w->data,
                                bias ? (const float*)bias->data : nullptr, (float*)y->data, (int)M, (int)N, (int)K));
    return after_launch(ctx, "linear");
}

tlhip_status linear_impl(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor w, tlhip_tensor bias, tlhip_tensor y,
                         float* fixed_ws, size_t fixed_ws_bytes) {
    TLHIP_TRY(check_ctx(ctx));
    if (x && check_t(x, "linear") == TLHIP_OK && x->dtype == TLHIP_F32) return linear_f32(ctx, x, w, bias, y);
    TLHIP_TRY(f16_args("linear", {x, y}));
    TLHIP_TRY(check_t(w, "linear weight"));
    if (w->dtype != TLHIP_F16 && !is_quant(w->dtype))
        return fail(TLHIP_ERR_DTYPE, "linear: weight dtype %d unsupported", (int)w->dtype);
    if (x->ndim != 2 || w->ndim != 2)
        return fail(TLHIP_ERR_INVALID_OPERATION, "matmul_transposed_b requires 2D tensors");
    const int64_t M = x->shape[0], K = x->shape[1], N = w->shape[0];
    if (w->shape[1] != K)
        return fail(TLHIP_ERR_INVALID_OPERATION, "matmul_transposed_b shape mismatch: [%lld, %lld] @ [%lld, %lld].T",
                    (long long)M, (long long)K, (long long)N, (long long)w->shape[1]);
    if (y->ndim != 2 || y->shape[0] != M || y->shape[1] != N)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "linear: output %s, expected [%lld, %lld]", shape_str(y).c_str(),
                    (long long)M, (long long)N);
    if (bias) {
        TLHIP_TRY(f16_args("linear bias", {bias}));
        if (numel(bias) != N) return fail(TLHIP_ERR_SHAPE_MISMATCH, "linear: bias %s for N=%lld", shape_str(bias).c_str(), (long long)N);
    }
    if (M == 0 || N == 0) return TLHIP_OK;
    GemvArgs a;
    a.x = P(x);
    a.wq = w->data;
    a.wd = w->scales;
    a.bias = bias ? P(bias) : nullptr;
    a.y = P(y);
    a.tile_flags = ctx->d_tile_flags;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    const int epi = bias ? EPI_BIAS : EPI_STORE;
    tlhip_status st = TLHIP_ERR_INVALID_OPERATION;
    if (M <= 4) {
        st = launch_gemv(ctx->stream, w->dtype, a, epi);
        if (st != TLHIP_OK) (void)hipGetLastError();
    }
    if (st == TLHIP_OK) return after_launch(ctx, "linear");
    const bool no_alloc = fixed_ws != nullptr;
    // Q6_K weights reach the MFMA GEMM as their dequantised f16 copy (the
    // reference's own representation), made once per weight tensor on its
    // first use here and kept with it
    tlhip_dtype wt = w->dtype;
    if (wt == TLHIP_Q6_K && no_alloc)
        return fail(TLHIP_ERR_INVALID_OPERATION,
                    "linear_noalloc: a Q6_K weight with M = %lld > 4 needs a dequantised f16 copy, which "
                    "this entry point cannot allocate (use tlhip_linear)", (long long)M);
    if (wt == TLHIP_Q6_K) {
        if (!w->f16_copy) {
            tlhip_tensor wf = nullptr;
            int64_t shp[2] = {N, K};
            TLHIP_TRY(alloc_tensor(ctx, TLHIP_F16, 2, shp, &wf));
            st = launch_dequant(ctx->stream, TLHIP_Q6_K, w->data, w->scales, P(wf), N, K);
            // The copy is cached on the weight and any context may read it
            // next, with no ordering the caller knows of: it is complete
            // before it is published (once per weight and upload).
            if (st == TLHIP_OK && hipStreamSynchronize(ctx->stream) != hipSuccess) {
                (void)hipGetLastError();
                st = fail(TLHIP_ERR_DEVICE, "linear: Q6_K dequantised copy failed");
            }
            if (st != TLHIP_OK) {
                tlhip_tensor_free(wf);
                return st;
            }
            w->f16_copy = wf;
        }
        a.wq = w->f16_copy->data;
        a.wd = nullptr;
        wt = TLHIP_F16;
    }
    // MFMA GEMM; a split-K workspace when the output has too few tiles to
    // fill the device: the context's, grown (stream-ordered) when a call
    // needs more, so steady-state calls allocate nothing
    const int sp = gemm_splits((int)M, (int)N, (int)K, (int)wt);
    const size_t need = (size_t)sp * M * N * sizeof(float);
    if (sp > 1 && no_alloc) {
        // the caller's fixed workspace: the same split as the pool path, so
        // the same kernels and the same bits
        if (need > fixed_ws_bytes)
            return fail(TLHIP_ERR_ALLOCATION,
                        "linear_noalloc: split-K partials of %zu bytes for [%lld x %lld] exceed the fixed "
                        "workspace of %zu bytes", need, (long long)M, (long long)N, fixed_ws_bytes);
        a.ws = fixed_ws;
        a.ws_bytes = need;
    } else if (sp > 1) {
        if (float* ws = ctx_workspace(ctx, need)) {   // (none: the GEMM runs unsplit)
            a.ws = ws;
            a.ws_bytes = need;
        }
    }
    TLHIP_TRY(launch_gemm(ctx->stream, wt, a, epi));
    return after_launch(ctx, "linear");
}

}  // namespace tlhip

extern "C" {

tlhip_status tlhip_matmul(tlhip_ctx ctx, tlhip_tensor a, tlhip_tensor b, tlhip_tensor c) try {
    TLHIP_TRY(check_ctx(ctx));
    // Tensor::matmul (matmul.rs:22-60) on TensorF16 or TensorF32 operands,
    // both the same (builtin_math.rs:49-58; a mix is the reference's TypeError)
    TLHIP_TRY(check_t(a, "matmul"));
    const bool f32 = a->dtype == TLHIP_F32;
    if (f32) {
        for (tlhip_tensor t : {b, c}) {
            TLHIP_TRY(check_t(t, "matmul"));
            if (t->dtype != TLHIP_F32) return fail(TLHIP_ERR_DTYPE, "matmul(): f32 input needs f32 operands");
        }
    } else {
        TLHIP_TRY(f16_args("matmul", {a, b, c}));
    }
    if (a->ndim != 2 || b->ndim != 2) return fail(TLHIP_ERR_INVALID_OPERATION, "matmul requires 2D tensors");
    const int64_t M = a->shape[0], K = a->shape[1], N = b->shape[1];
    if (b->shape[0] != K)
        return fail(TLHIP_ERR_INVALID_OPERATION, "matmul shape mismatch: [%lld, %lld] @ [%lld, %lld]", (long long)M,
                    (long long)K, (long long)b->shape[0], (long long)N);
    if (c->ndim != 2 || c->shape[0] != M || c->shape[1] != N)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "matmul: output %s", shape_str(c).c_str());
    if (M == 0 || N == 0) return TLHIP_OK;
    if (K > INT32_MAX || N > INT32_MAX) return fail(TLHIP_ERR_INVALID_DIMENSION, "matmul: too large");
    // matmul(a, b) = matmul_transposed_b(a, b^T): one transpose kernel, then
    // the same fp32-accumulating product as linear().
    tlhip_tensor bt;
    int64_t shp[2] = {N, K};
    TLHIP_TRY(alloc_tensor(ctx, f32 ? TLHIP_F32 : TLHIP_F16, 2, shp, &bt));
    tlhip_status st = f32 ? launch_transpose_f32(ctx->stream, (const float*)b->data, (float*)bt->data, (int)K, (int)N)
                          : launch_transpose(ctx->stream, P(b), P(bt), (int)K, (int)N);
    if (st == TLHIP_OK) st = tlhip_linear(ctx, a, bt, nullptr, c);
    tlhip_tensor_free(bt);
    return st;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_rms_norm(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor w, float eps, tlhip_tensor y) try {
    TLHIP_TRY(check_ctx(ctx));
    bool f32;
    TLHIP_TRY(float_args("rms_norm", {x, w, y}, &f32));
    TLHIP_TRY(same_shape(x, y, "rms_norm"));
    const int64_t n = last_dim(x);
    if (w->ndim != 1 || w->shape[0] != n)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "rms_norm: weight %s for normalized_shape [%lld]", shape_str(w).c_str(),
                    (long long)n);
    if (n == 0) return TLHIP_OK;
    if (f32) TLHIP_TRY(launch_rms_norm_f32(ctx->stream, F(x), F(w), F(y), (int)(numel(x) / n), (int)n, eps));
    else TLHIP_TRY(launch_rms_norm(ctx->stream, P(x), P(w), P(y), (int)(numel(x) / n), (int)n, eps));
    return after_launch(ctx, "rms_norm");
} TLHIP_CATCH_STATUS

tlhip_status tlhip_layer_norm(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor w, tlhip_tensor b, float eps,
                              tlhip_tensor y) try {
    TLHIP_TRY(check_ctx(ctx));
    bool f32;
    TLHIP_TRY(float_args("layer_norm", {x, y}, &f32));
    TLHIP_TRY(same_shape(x, y, "layer_norm"));
    const int64_t n = last_dim(x);
    for (tlhip_tensor t : {w, b}) {
        if (!t) continue;
        TLHIP_TRY(check_t(t, "layer_norm"));
        TLHIP_TRY(check_dtype(t, f32 ? TLHIP_F32 : TLHIP_F16, "layer_norm"));
        if (t->ndim != 1 || t->shape[0] != n)
            return fail(TLHIP_ERR_SHAPE_MISMATCH, "layer_norm: param %s for [%lld]", shape_str(t).c_str(), (long long)n);
    }
    if (n == 0) return TLHIP_OK;
    if (f32)
        TLHIP_TRY(launch_layer_norm_f32(ctx->stream, F(x), w ? F(w) : nullptr, b ? F(b) : nullptr, F(y),
                                        (int)(numel(x) / n), (int)n, eps));
    else
        TLHIP_TRY(launch_layer_norm(ctx->stream, P(x), w ? P(w) : nullptr, b ? P(b) : nullptr, P(y),
                                    (int)(numel(x) / n), (int)n, eps));
    return after_launch(ctx, "layer_norm");
} TLHIP_CATCH_STATUS

tlhip_status tlhip_rope(tlhip_ctx ctx, tlhip_tensor x, int offset, float theta, tlhip_rope_layout layout,
                        int rot_dims, tlhip_tensor y) try {
    TLHIP_TRY(check_ctx(ctx));
    bool f32;
    TLHIP_TRY(float_args("rope", {x, y}, &f32));
    TLHIP_TRY(same_shape(x, y, "rope"));
    if (x->ndim < 3) return fail(TLHIP_ERR_INVALID_OPERATION, "RoPE requires at least 3D tensor (got %dD)", x->ndim);
    const int64_t D = x->shape[x->ndim - 1], H = x->shape[x->ndim - 2], S = x->shape[x->ndim - 3];
    if (rot_dims <= 0) rot_dims = (int)D;
    if (D % 2 != 0 || rot_dims % 2 != 0 || rot_dims > D)
        return fail(TLHIP_ERR_INVALID_OPERATION, "RoPE requires even head_dim (got %lld, rot %d)", (long long)D, rot_dims);
    if (offset < 0) return fail(TLHIP_ERR_INVALID_ARGUMENT, "negative RoPE offset");
    if (layout != TLHIP_ROPE_INTERLEAVED && layout != TLHIP_ROPE_NEOX)
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "bad RoPE layout %d", (int)layout);
    if (numel(x) == 0) return TLHIP_OK;
    const float* table;
    TLHIP_TRY(rope_table(ctx, theta, rot_dims, offset + (int)S, &table));
    if (f32)
        TLHIP_TRY(launch_rope_f32(ctx->stream, F(x), F(y), (int)S, (int)H, (int)D, numel(x) / (S * H * D), offset,
                                  (int)layout, rot_dims, table));
    else
        TLHIP_TRY(launch_rope(ctx->stream, P(x), P(y), (int)S, (int)H, (int)D, numel(x) / (S * H * D), offset,
                              nullptr, (int)layout, rot_dims, table, 0, 0));
    return after_launch(ctx, "rope");
} TLHIP_CATCH_STATUS

tlhip_status tlhip_softmax_lastdim(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor y) try {
    TLHIP_TRY(check_ctx(ctx));
    bool f32;
    TLHIP_TRY(float_args("softmax", {x, y}, &f32));
    TLHIP_TRY(same_shape(x, y, "softmax"));
    if (x->ndim == 0) return fail(TLHIP_ERR_INVALID_OPERATION, "softmax requires non-empty tensor");
    const int64_t n = last_dim(x);
    if (n == 0 || numel(x) == 0) return TLHIP_OK;
    if (f32) TLHIP_TRY(launch_softmax_f32(ctx->stream, F(x), F(y), numel(x) / n, (int)n));
    else TLHIP_TRY(launch_softmax(ctx->stream, P(x), P(y), numel(x) / n, (int)n));
    return after_launch(ctx, "softmax");
} TLHIP_CATCH_STATUS

static tlhip_status unary(tlhip_ctx ctx, int op, tlhip_tensor x, tlhip_tensor y, const char* nm) {
    TLHIP_TRY(check_ctx(ctx));
    bool f32;
    TLHIP_TRY(float_args(nm, {x, y}, &f32));
    TLHIP_TRY(same_shape(x, y, nm));
    if (f32) TLHIP_TRY(launch_elementwise_f32(ctx->stream, op, F(x), nullptr, F(y), numel(x), 0, 0.f));
    else TLHIP_TRY(launch_elementwise(ctx->stream, op, P(x), nullptr, P(y), numel(x), 0, 0.f));
    return after_launch(ctx, nm);
}

tlhip_status tlhip_sigmoid(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor y) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(check_t(x, "sigmoid"));
    if (x->dtype != TLHIP_F32) return unary(ctx, EW_SIGMOID, x, y, "sigmoid");
    bool f32;
    TLHIP_TRY(float_args("sigmoid", {x, y}, &f32));
    TLHIP_TRY(same_shape(x, y, "sigmoid"));
    TLHIP_TRY(launch_sigmoid_f32(ctx->stream, F(x), F(y), numel(x)));
    return after_launch(ctx, "sigmoid");
} TLHIP_CATCH_STATUS
tlhip_status tlhip_silu(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor y) try { return unary(ctx, EW_SILU, x, y, "silu"); } TLHIP_CATCH_STATUS
tlhip_status tlhip_gelu(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor y) try { return unary(ctx, EW_GELU, x, y, "gelu"); } TLHIP_CATCH_STATUS

tlhip_status tlhip_silu_mul(tlhip_ctx ctx, tlhip_tensor g, tlhip_tensor u, tlhip_tensor y) try {
    TLHIP_TRY(check_ctx(ctx));
    bool f32;
    TLHIP_TRY(float_args("silu_mul", {g, u, y}, &f32));
    TLHIP_TRY(same_shape(g, u, "silu_mul"));
    TLHIP_TRY(same_shape(g, y, "silu_mul"));
    if (f32) TLHIP_TRY(launch_elementwise_f32(ctx->stream, EW_SILU_MUL, F(g), F(u), F(y), numel(g), 0, 0.f));
    else TLHIP_TRY(launch_elementwise(ctx->stream, EW_SILU_MUL, P(g), P(u), P(y), numel(g), 0, 0.f));
    return after_launch(ctx, "silu_mul");
} TLHIP_CATCH_STATUS

static tlhip_status binary(tlhip_ctx ctx, int op, tlhip_tensor a, tlhip_tensor b, tlhip_tensor y, const char* nm) {
    TLHIP_TRY(check_ctx(ctx));
    bool f32;
    TLHIP_TRY(float_args(nm, {a, b, y}, &f32));
    TLHIP_TRY(same_shape(a, y, nm));
    int64_t period = 0;
    if (numel(b) != numel(a)) {
        // row broadcast: b matches a's last dim (bias-style add)
        if (b->ndim == 1 && b->shape[0] == last_dim(a)) period = b->shape[0];
        else return fail(TLHIP_ERR_SHAPE_MISMATCH, "%s: %s vs %s", nm, shape_str(a).c_str(), shape_str(b).c_str());
    } else {
        TLHIP_TRY(same_shape(a, b, nm));
    }
    if (f32) TLHIP_TRY(launch_elementwise_f32(ctx->stream, op, F(a), F(b), F(y), numel(a), period, 0.f));
    else TLHIP_TRY(launch_elementwise(ctx->stream, op, P(a), P(b), P(y), numel(a), period, 0.f));
    return after_launch(ctx, nm);
}

tlhip_status tlhip_add(tlhip_ctx ctx, tlhip_tensor a, tlhip_tensor b, tlhip_tensor y) try { return binary(ctx, EW_ADD, a, b, y, "add"); } TLHIP_CATCH_STATUS
tlhip_status tlhip_mul(tlhip_ctx ctx, tlhip_tensor a, tlhip_tensor b, tlhip_tensor y) try { return binary(ctx, EW_MUL, a, b, y, "mul"); } TLHIP_CATCH_STATUS

tlhip_status tlhip_mul_scalar(tlhip_ctx ctx, tlhip_tensor a, float s, tlhip_tensor y) try {
    TLHIP_TRY(check_ctx(ctx));
    bool f32;
    TLHIP_TRY(float_args("mul_scalar", {a, y}, &f32));
    TLHIP_TRY(same_shape(a, y, "mul_scalar"));
    // the scalar is a value of the tensor's type (mul_scalar(scalar: T))
    if (f32) TLHIP_TRY(launch_elementwise_f32(ctx->stream, EW_MUL_SCALAR, F(a), nullptr, F(y), numel(a), 0, s));
    else TLHIP_TRY(launch_elementwise(ctx->stream, EW_MUL_SCALAR, P(a), nullptr, P(y), numel(a), 0, round_f16(s)));
    return after_launch(ctx, "mul_scalar");
} TLHIP_CATCH_STATUS

tlhip_status tlhip_embedding(tlhip_ctx ctx, tlhip_tensor table, const int32_t* ids, int n, tlhip_tensor out) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(check_t(table, "embedding table"));
    // an f32 table gives f32 rows (embedding_lookup_f32); every other table f16
    const bool f32 = table->dtype == TLHIP_F32;
    if (!f32 && table->dtype != TLHIP_F16 && !is_quant(table->dtype))
        return fail(TLHIP_ERR_DTYPE, "embedding: table must be F16, F32, Q4_0, Q8_0 or Q6_K (dtype %d)",
                    (int)table->dtype);
    TLHIP_TRY(check_t(out, "embedding"));
    TLHIP_TRY(check_dtype(out, f32 ? TLHIP_F32 : TLHIP_F16, "embedding"));
    if (table->ndim != 2) return fail(TLHIP_ERR_INVALID_DIMENSION, "embedding table must be 2-D");
    const int64_t V = table->shape[0], Hd = table->shape[1];
    if (n < 0 || (n > 0 && !ids)) return fail(TLHIP_ERR_INVALID_ARGUMENT, "embedding: bad ids");
    if (out->ndim != 2 || out->shape[0] != n || out->shape[1] != Hd)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "embedding: output %s, expected [%d, %lld]", shape_str(out).c_str(), n,
                    (long long)Hd);
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= V)
            return fail(TLHIP_ERR_INDEX_OUT_OF_BOUNDS, "token id %d out of range [0, %lld)", ids[i], (long long)V);
    if (n == 0) return TLHIP_OK;
    int32_t* d_ids = nullptr;
    TLHIP_CHECK_HIP(hipMallocAsync(&d_ids, sizeof(int32_t) * n, ctx->stream));
    TLHIP_CHECK_HIP(hipMemcpyAsync(d_ids, ids, sizeof(int32_t) * n, hipMemcpyHostToDevice, ctx->stream));
    tlhip_status st = f32 ? launch_embedding_f32(ctx->stream, F(table), d_ids, F(out), n, (int)Hd)
                          : launch_embedding(ctx->stream, table->dtype, table->data, table->scales, d_ids, nullptr,
                                             P(out), n, (int)Hd, (int)V);
    (void)hipFreeAsync(d_ids, ctx->stream);
    // the host ids buffer must stay valid until the copy ran
    TLHIP_CHECK_HIP(hipStreamSynchronize(ctx->stream));
    TLHIP_TRY(st);
    return after_launch(ctx, "embedding");
} TLHIP_CATCH_STATUS

tlhip_status tlhip_apply_attention_mask(tlhip_ctx ctx, tlhip_tensor sc, tlhip_tensor mask, tlhip_tensor y) try {
    TLHIP_TRY(check_ctx(ctx));
    bool f32;
    TLHIP_TRY(float_args("apply_attention_mask", {sc, mask, y}, &f32));
    TLHIP_TRY(same_shape(sc, y, "apply_attention_mask"));
    int64_t period;
    if (numel(mask) == numel(sc)) period = numel(sc);
    else if (sc->ndim == 3 && mask->ndim == 2 && mask->shape[0] == sc->shape[0] && mask->shape[1] == sc->shape[2] &&
             sc->shape[2] < 32768 && sc->shape[1] < 65536)
        period = -(sc->shape[2] * 65536 + sc->shape[1]);
    else
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "apply_attention_mask: scores %s, mask %s", shape_str(sc).c_str(),
                    shape_str(mask).c_str());
    if (f32) TLHIP_TRY(launch_mask_f32(ctx->stream, F(sc), F(mask), F(y), numel(sc), period));
    else TLHIP_TRY(launch_mask(ctx->stream, P(sc), P(mask), P(y), numel(sc), period));
    return after_launch(ctx, "apply_attention_mask");
} TLHIP_CATCH_STATUS

// causal_mask(n) (builtin_nn.rs:423-460): out must be [n, n] f16.
tlhip_status tlhip_causal_mask(tlhip_ctx ctx, tlhip_tensor out) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(f16_args("causal_mask", {out}));
    if (out->ndim != 2 || out->shape[0] != out->shape[1])
        return fail(TLHIP_ERR_INVALID_DIMENSION, "causal_mask: output must be [n, n], got %s", shape_str(out).c_str());
    TLHIP_TRY(launch_causal_mask(ctx->stream, P(out), out->shape[0]));
    return after_launch(ctx, "causal_mask");
} TLHIP_CATCH_STATUS

static int elem_bytes(tlhip_dtype d) { return d == TLHIP_F16 ? 2 : (d == TLHIP_F32 || d == TLHIP_I32) ? 4 : 0; }

// slice_last(x, axis) (builtin_tensor.rs:1949-1991, slice.rs:25-60): the
// last index of axis 0; y is x's shape without axis 0 ([1] for a 1-D x,
// where the reference returns a scalar).
tlhip_status tlhip_slice_last(tlhip_ctx ctx, tlhip_tensor x, int axis, tlhip_tensor y) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(check_t(x, "slice_last"));
    TLHIP_TRY(check_t(y, "slice_last"));
    const int eb = elem_bytes(x->dtype);
    if (!eb || y->dtype != x->dtype) return fail(TLHIP_ERR_DTYPE, "slice_last: dtypes %d -> %d", (int)x->dtype, (int)y->dtype);
    if (axis < 0 || axis >= x->ndim)
        return fail(TLHIP_ERR_INVALID_OPERATION, "slice_last() axis %d out of bounds for %dD tensor", axis, x->ndim);
    if (axis != 0)
        return fail(TLHIP_ERR_INVALID_OPERATION, "slice_last() currently only supports axis=0, got axis=%d", axis);
    const bool ok = x->ndim == 1 ? (y->ndim == 1 && y->shape[0] == 1)
                                 : (y->ndim == x->ndim - 1 &&
                                    memcmp(y->shape, x->shape + 1, sizeof(int64_t) * (x->ndim - 1)) == 0);
    if (!ok) return fail(TLHIP_ERR_SHAPE_MISMATCH, "slice_last: %s -> %s", shape_str(x).c_str(), shape_str(y).c_str());
    if (x->shape[0] <= 0) return fail(TLHIP_ERR_INVALID_DIMENSION, "slice_last: empty axis 0");
    const size_t inner = (size_t)numel(y) * eb;
    if (inner)
        TLHIP_CHECK_HIP(hipMemcpyAsync(y->data, (const uint8_t*)x->data + (size_t)(x->shape[0] - 1) * inner, inner,
                                       hipMemcpyDeviceToDevice, ctx->stream));
    return after_launch(ctx, "slice_last");
} TLHIP_CATCH_STATUS

// broadcast_to(x, shape) (broadcast.rs:11-120, shape.rs:37-49): y's shape is
// the target; dims align from the right and an input dim of 1 repeats.  An
// equal shape is a copy (the reference returns the tensor itself).
tlhip_status tlhip_broadcast_to(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor y) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(check_t(x, "broadcast_to"));
    TLHIP_TRY(check_t(y, "broadcast_to"));
    const int eb = elem_bytes(x->dtype);
    if (!eb || y->dtype != x->dtype) return fail(TLHIP_ERR_DTYPE, "broadcast_to: dtypes %d -> %d", (int)x->dtype, (int)y->dtype);
    bool ok = x->ndim <= y->ndim;
    for (int k = 1; ok && k <= x->ndim; k++) {
        const int64_t a = x->shape[x->ndim - k], b = y->shape[y->ndim - k];
        ok = a == b || a == 1;
    }
    if (!ok) return fail(TLHIP_ERR_SHAPE_MISMATCH, "broadcast_to: expected %s, actual %s", shape_str(y).c_str(),
                         shape_str(x).c_str());
    BcastDims b;
    b.nd = y->ndim;
    const int rd = y->ndim - x->ndim;
    int64_t st = 1;
    for (int i = y->ndim - 1; i >= 0; i--) {
        b.shape[i] = y->shape[i];
        if (i >= rd) {
            const int64_t xd = x->shape[i - rd];
            b.xstride[i] = xd == 1 ? 0 : st;
            st *= xd;
        }
    }
    TLHIP_TRY(launch_broadcast(ctx->stream, x->data, y->data, eb, b));
    return after_launch(ctx, "broadcast_to");
} TLHIP_CATCH_STATUS

// rope(x, cos, sin) = Tensor::rope_candle (builtin_tensor.rs:569-597,
// rope.rs:18-65): x [S, H, D], cos/sin [L >= S, D] f16.
tlhip_status tlhip_rope_cos_sin(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor cos_t, tlhip_tensor sin_t, tlhip_tensor y) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(f16_args("rope(x, cos, sin)", {x, cos_t, sin_t, y}));
    if (x->ndim != 3)
        return fail(TLHIP_ERR_INVALID_OPERATION, "rope_candle requires 3D tensor [seq_len, n_heads, head_dim], got %dD",
                    x->ndim);
    if (cos_t->ndim != 2 || sin_t->ndim != 2)
        return fail(TLHIP_ERR_INVALID_OPERATION, "cos/sin must be 2D [max_seq_len, head_dim], got cos: %dD, sin: %dD",
                    cos_t->ndim, sin_t->ndim);
    const int64_t S = x->shape[0], H = x->shape[1], D = x->shape[2];
    if (cos_t->shape[1] != D || sin_t->shape[1] != D)
        return fail(TLHIP_ERR_INVALID_OPERATION, "cos/sin last dim must be head_dim = %lld", (long long)D);
    if (cos_t->shape[0] < S || sin_t->shape[0] < S)
        return fail(TLHIP_ERR_INVALID_OPERATION, "cos/sin first dim must be >= seq_len = %lld", (long long)S);
    if (D % 2) return fail(TLHIP_ERR_INVALID_DIMENSION, "rope(x, cos, sin): head_dim %lld is odd", (long long)D);
    TLHIP_TRY(same_shape(x, y, "rope(x, cos, sin)"));
    if (S * H * D > INT32_MAX) return fail(TLHIP_ERR_INVALID_DIMENSION, "rope(x, cos, sin): tensor too large");
    TLHIP_TRY(launch_rope_cs(ctx->stream, P(x), P(cos_t), P(sin_t), P(y), (int)S, (int)H, (int)D));
    return after_launch(ctx, "rope(x, cos, sin)");
} TLHIP_CATCH_STATUS

// precompute_rope_cos / precompute_rope_sin (builtin_tensor.rs:610-700):
// computed on the host in f32 as the reference does, each value stored in
// columns 2i and 2i+1, converted to f16 and uploaded; out [max_seq_len,
// head_dim] f16.  Synchronous (the host table is freed on return).
tlhip_status tlhip_precompute_rope(tlhip_ctx ctx, int head_dim, int max_seq_len, float base, int want_sin,
                                   tlhip_tensor out) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(f16_args("precompute_rope", {out}));
    if (head_dim <= 0 || head_dim % 2)
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "head_dim must be even, got %d", head_dim);
    if (max_seq_len < 0 || out->ndim != 2 || out->shape[0] != max_seq_len || out->shape[1] != head_dim)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "precompute_rope: output %s for [%d, %d]", shape_str(out).c_str(),
                    max_seq_len, head_dim);
    std::vector<_Float16> tab((size_t)max_seq_len * head_dim);
    for (int pos = 0; pos < max_seq_len; pos++)
        for (int i = 0; i < head_dim / 2; i++) {
            const float theta = 1.0f / powf(base, (float)(2 * i) / (float)head_dim);
            const float ang = (float)pos * theta;
            const _Float16 v = (_Float16)(want_sin ? sinf(ang) : cosf(ang));
            tab[(size_t)pos * head_dim + 2 * i] = v;
            tab[(size_t)pos * head_dim + 2 * i + 1] = v;
        }
    return tlhip_tensor_upload(ctx, out, tab.data(), tab.size() * sizeof(_Float16));
} TLHIP_CATCH_STATUS

static tlhip_status qkv_dims(tlhip_tensor q, tlhip_tensor k, const char* nm, int* H, int* Hkv, int* D) {
    if (q->ndim != 3 || k->ndim != 3) return fail(TLHIP_ERR_INVALID_DIMENSION, "%s: expects 3-D tensors", nm);
    *H = (int)q->shape[1];
    *Hkv = (int)k->shape[1];
    *D = (int)k->shape[2];
    if (*Hkv <= 0 || *H % *Hkv) return fail(TLHIP_ERR_SHAPE_MISMATCH, "%s: %d heads vs %d KV heads", nm, *H, *Hkv);
    return TLHIP_OK;
}

tlhip_status tlhip_einsum_scores(tlhip_ctx ctx, tlhip_tensor q, tlhip_tensor k, tlhip_tensor sc) try {
    TLHIP_TRY(check_ctx(ctx));
    bool f32;
    TLHIP_TRY(float_args("einsum ihd,jhd->ihj", {q, k, sc}, &f32));
    int H, Hkv, D;
    TLHIP_TRY(qkv_dims(q, k, "einsum ihd,jhd->ihj", &H, &Hkv, &D));
    const int I = (int)q->shape[0], J = (int)k->shape[0];
    if (q->shape[2] != D) return fail(TLHIP_ERR_SHAPE_MISMATCH, "einsum: head_dim mismatch");
    if (sc->ndim != 3 || sc->shape[0] != I || sc->shape[1] != H || sc->shape[2] != J)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "einsum: output %s", shape_str(sc).c_str());
    if (f32) TLHIP_TRY(launch_scores_f32(ctx->stream, F(q), F(k), F(sc), I, J, H, Hkv, D));
    else TLHIP_TRY(launch_scores(ctx->stream, P(q), P(k), P(sc), I, J, H, Hkv, D));
    return after_launch(ctx, "einsum_scores");
} TLHIP_CATCH_STATUS

tlhip_status tlhip_einsum_context(tlhip_ctx ctx, tlhip_tensor p, tlhip_tensor v, tlhip_tensor out) try {
    TLHIP_TRY(check_ctx(ctx));
    bool f32;
    TLHIP_TRY(float_args("einsum ihj,jhd->ihd", {p, v, out}, &f32));
    if (p->ndim != 3 || v->ndim != 3 || out->ndim != 3)
        return fail(TLHIP_ERR_INVALID_DIMENSION, "einsum ihj,jhd->ihd expects 3-D tensors");
    const int I = (int)p->shape[0], H = (int)p->shape[1], J = (int)p->shape[2];
    const int Hkv = (int)v->shape[1], D = (int)v->shape[2];
    if (v->shape[0] != J || Hkv <= 0 || H % Hkv)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "einsum: P %s, V %s", shape_str(p).c_str(), shape_str(v).c_str());
    if (out->shape[0] != I || out->shape[1] != H || out->shape[2] != D)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "einsum: output %s", shape_str(out).c_str());
    if (f32) TLHIP_TRY(launch_context_f32(ctx->stream, F(p), F(v), F(out), I, J, H, Hkv, D));
    else TLHIP_TRY(launch_context(ctx->stream, P(p), P(v), P(out), I, J, H, Hkv, D));
    return after_launch(ctx, "einsum_context");
} TLHIP_CATCH_STATUS

tlhip_status tlhip_attention(tlhip_ctx ctx, tlhip_tensor q, tlhip_tensor k, tlhip_tensor v, int q_pos0, float scale,
                             int causal, tlhip_tensor out) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(f16_args("attention", {q, k, v, out}));
    int H, Hkv, D;
    TLHIP_TRY(qkv_dims(q, k, "attention", &H, &Hkv, &D));
    TLHIP_TRY(same_shape(k, v, "attention k/v"));
    TLHIP_TRY(same_shape(q, out, "attention q/out"));
    if (q->shape[2] != D) return fail(TLHIP_ERR_SHAPE_MISMATCH, "attention: head_dim mismatch");
    if (q_pos0 < 0) return fail(TLHIP_ERR_INVALID_ARGUMENT, "attention: negative q_pos0");
    const int S = (int)q->shape[0], J = (int)k->shape[0];
    if (J > kAttnMaxKeys) return fail(TLHIP_ERR_INVALID_DIMENSION, "attention: %d keys > %d", J, kAttnMaxKeys);
    if (causal && q_pos0 + S > J)
        return fail(TLHIP_ERR_INVALID_DIMENSION, "attention: query positions up to %d but only %d keys", q_pos0 + S, J);
    AttnArgs a;
    a.q = P(q);
    a.k = P(k);
    a.v = P(v);
    a.out = P(out);
    a.S = S;
    a.H = H;
    a.Hkv = Hkv;
    a.D = D;
    a.q_pos0 = q_pos0;
    a.causal = causal;
    a.scale_h = round_f16(scale);
    a.head_flags = ctx->d_tile_flags + SK_MAX_TILES_SPLIT;
    if (attention_mfma_ok(a, J)) {
        float* vt = ctx_workspace(ctx, attention_mfma_scratch(J, Hkv, D));
        if (!vt) return fail(TLHIP_ERR_ALLOCATION, "attention: no workspace for V^T (%zu bytes)", attention_mfma_scratch(J, Hkv, D));
        TLHIP_TRY(launch_attention_mfma(ctx->stream, a, J, (uint16_t*)vt));
    } else if (attention_split_j_ok(a, J) && (J > kAttnRowKeys || J > (D == 64 ? 1024 : 512))) {
        // one row over many keys: key-chunked (more workgroups than the one
        // per head of the one-row kernels; measured faster on MI355X past
        // ~1,024 keys at head dim 64 and ~512 at 80 / 128), and the only path
        // past their score row
        float* sc = ctx_workspace(ctx, attention_split_scratch(H, J, D));
        if (sc) TLHIP_TRY(launch_attention_split_j(ctx->stream, a, J, sc));
        else if (J > kAttnRowKeys) return fail(TLHIP_ERR_ALLOCATION, "attention: no workspace for the key chunks");
        else TLHIP_TRY(launch_attention_j(ctx->stream, a, J));
    } else if (J > kAttnRowKeys) {
        return fail(TLHIP_ERR_INVALID_DIMENSION,
                    "attention: %d keys needs head_dim 64/80/128 and 16-byte aligned rows (more than %d keys)", J,
                    kAttnRowKeys);
    } else {
        TLHIP_TRY(launch_attention_j(ctx->stream, a, J));
    }
    return after_launch(ctx, "attention");
} TLHIP_CATCH_STATUS

tlhip_status tlhip_tensor_argmax(tlhip_ctx ctx, tlhip_tensor x, int dim, int keepdim, tlhip_tensor y) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(check_t(x, "argmax"));
    TLHIP_TRY(check_t(y, "argmax"));
    if (x->dtype != TLHIP_F16 && x->dtype != TLHIP_F32)
        return fail(TLHIP_ERR_DTYPE, "argmax: input must be f16 or f32 (dtype %d)", (int)x->dtype);
    if (y->dtype != x->dtype) return fail(TLHIP_ERR_DTYPE, "argmax: result dtype %d != input dtype %d", (int)y->dtype, (int)x->dtype);
    if (dim >= x->ndim) return fail(TLHIP_ERR_INVALID_DIMENSION, "Invalid dimension: %d", dim);
    if (x->ndim > 8) return fail(TLHIP_ERR_INVALID_DIMENSION, "argmax: rank %d > 8", x->ndim);
    // result shape (reduce.rs:600-606, 625-636): the whole tensor -> [1]
    // ([1] * rank with keepdim); a dim -> the other dims (that dim as 1 with
    // keepdim).  Reducing the only dim without keepdim leaves no dims, which
    // the reference's Tensor::from_vec rejects (a dimensionless shape has
    // numel 0, tensor_creation.rs:111-118).
    std::vector<int64_t> want;
    if (dim < 0) {
        if (numel(x) == 0) return fail(TLHIP_ERR_INVALID_OPERATION, "argmax of an empty tensor");
        want.assign(keepdim ? x->ndim : 1, 1);
    } else {
        for (int i = 0; i < x->ndim; i++)
            if (i != dim) want.push_back(x->shape[i]);
            else if (keepdim) want.push_back(1);
        if (want.empty()) return fail(TLHIP_ERR_SHAPE_MISMATCH, "argmax: no dims left (expected [0], got [1])");
    }
    if ((int)want.size() != y->ndim || memcmp(want.data(), y->shape, sizeof(int64_t) * want.size()) != 0)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "argmax: result shape %s for %s along dim %d", shape_str(y).c_str(),
                    shape_str(x).c_str(), dim);
    TLHIP_TRY(launch_tensor_argmax(ctx->stream, x->dtype, x->data, y->data, x->shape, x->ndim, dim < 0 ? -1 : dim));
    return after_launch(ctx, "argmax");
} TLHIP_CATCH_STATUS

tlhip_status tlhip_argmax(tlhip_ctx ctx, tlhip_tensor logits, int32_t* out) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(f16_args("argmax", {logits}));
    if (!out) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null output");
    if (logits->ndim != 1 && logits->ndim != 2)
        return fail(TLHIP_ERR_INVALID_DIMENSION, "temperature_sample() expects 1D or 2D logits tensor");
    const int64_t V = last_dim(logits);
    const int64_t rows = numel(logits) / (V ? V : 1);
    if (V == 0 || rows == 0) return fail(TLHIP_ERR_INVALID_DIMENSION, "argmax of an empty tensor");
    const uint16_t* last = P(logits) + (size_t)(rows - 1) * V;
    TLHIP_TRY(launch_argmax(ctx->stream, last, (int)V, ctx->d_scratch_i32, nullptr, nullptr));
    TLHIP_CHECK_HIP(hipMemcpyAsync(ctx->h_pinned_i32, ctx->d_scratch_i32, 4, hipMemcpyDeviceToHost, ctx->stream));
    TLHIP_CHECK_HIP(hipStreamSynchronize(ctx->stream));
    *out = ctx->h_pinned_i32[0];
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_temperature_sample(tlhip_ctx ctx, tlhip_tensor logits, float temperature, uint64_t seed,
                                      uint64_t counter, int32_t* out) try {
    if (!(temperature > 1e-4f)) return tlhip_argmax(ctx, logits, out);
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(f16_args("temperature_sample", {logits}));
    if (!out) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null output");
    if (logits->ndim != 1 && logits->ndim != 2)
        return fail(TLHIP_ERR_INVALID_DIMENSION, "temperature_sample() expects 1D or 2D logits tensor");
    const int64_t V = last_dim(logits);
    const int64_t rows = numel(logits) / (V ? V : 1);
    if (V == 0 || rows == 0) return fail(TLHIP_ERR_INVALID_DIMENSION, "temperature_sample of an empty tensor");
    const uint16_t* last = P(logits) + (size_t)(rows - 1) * V;
    void* scratch = nullptr;
    TLHIP_CHECK_HIP(hipMallocAsync(&scratch, sample_scratch_bytes((int)V), ctx->stream));
    const tlhip_status st = launch_sample(ctx->stream, last, (int)V, temperature, seed, counter, scratch,
                                          ctx->d_scratch_i32, nullptr, nullptr);
    (void)hipFreeAsync(scratch, ctx->stream);
    TLHIP_TRY(st);
    TLHIP_CHECK_HIP(hipMemcpyAsync(ctx->h_pinned_i32, ctx->d_scratch_i32, 4, hipMemcpyDeviceToHost, ctx->stream));
    TLHIP_CHECK_HIP(hipStreamSynchronize(ctx->stream));
    *out = ctx->h_pinned_i32[0];
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

}  // extern "C"
