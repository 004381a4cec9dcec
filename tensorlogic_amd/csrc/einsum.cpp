// einsum.cpp -- einsum(equation, operands...) (eval.rs:3264-3318,
// einsum.rs:39-82): the equation is parsed on the host as the reference
// parses it (einsum.rs:84-128), the two attention equations go to their
// kernels (the reference's Metal path, einsum.rs:647-684), and every other
// equation runs general_einsum_cpu's arithmetic (einsum.rs:207-333) on the
// device, one thread per output element (einsum_general_kernel).
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "internal.hpp"

using namespace tlhip;

namespace {

std::string trim(const std::string& s) {
    size_t a = 0, b = s.size();
    while (a < b && (s[a] == ' ' || s[a] == '\t')) a++;
    while (b > a && (s[b - 1] == ' ' || s[b - 1] == '\t')) b--;
    return s.substr(a, b - a);
}

bool is_letter(char c) { return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z'); }

// What one equation over these operands computes.
struct Einsum {
    int kind = 0;   // 0 general, 1 "ihd,jhd->ihj", 2 "ihj,jhd->ihd"
    bool f32 = false;
    int out_nd = 0;
    int64_t out_shape[8] = {};
    EinsumPlan plan;
    int64_t n_out = 0, n_sum = 0;
};

// parse_einsum_equation / infer_output_spec (einsum.rs:84-128): at most one
// "->"; inputs split at ','; without "->" the output is every index that
// occurs exactly once, in sorted order.
tlhip_status parse(const char* equation, std::vector<std::string>* ins, std::string* out) {
    if (!equation) return fail(TLHIP_ERR_INVALID_ARGUMENT, "einsum: null equation");
    const std::string s(equation);
    const size_t arrow = s.find("->");
    if (arrow != std::string::npos && s.find("->", arrow + 2) != std::string::npos)
        return fail(TLHIP_ERR_INVALID_OPERATION, "Invalid einsum equation: too many arrows");
    const std::string lhs = arrow == std::string::npos ? s : s.substr(0, arrow);
    size_t start = 0;
    for (;;) {
        const size_t comma = lhs.find(',', start);
        ins->push_back(trim(lhs.substr(start, comma == std::string::npos ? std::string::npos : comma - start)));
        if (comma == std::string::npos) break;
        start = comma + 1;
    }
    if (arrow != std::string::npos) {
        *out = trim(s.substr(arrow + 2));
    } else {
        int count[128] = {};
        for (char c : lhs)
            if (is_letter(c)) count[(int)c]++;
        out->clear();
        for (int c = 0; c < 128; c++)
            if (count[c] == 1) out->push_back((char)c);
    }
    return TLHIP_OK;
}

tlhip_status plan_einsum(const char* equation, const tlhip_tensor* ops, int n, Einsum* e) {
    std::vector<std::string> ins;
    std::string out;
    TLHIP_TRY(parse(equation, &ins, &out));
    if (n < 1 || !ops) return fail(TLHIP_ERR_INVALID_OPERATION, "einsum requires at least one tensor");
    if ((int)ins.size() != n)
        return fail(TLHIP_ERR_INVALID_OPERATION, "Expected %d operands, got %d", (int)ins.size(), n);
    for (int k = 0; k < n; k++) TLHIP_TRY(check_t(ops[k], "einsum"));
    e->f32 = ops[0]->dtype == TLHIP_F32;
    for (int k = 0; k < n; k++)
        if (ops[k]->dtype != (e->f32 ? TLHIP_F32 : TLHIP_F16))
            return fail(TLHIP_ERR_DTYPE, "einsum requires all tensors to be the same type (all f16 or all f32)");
    // the Metal path's two equations (matched on the equation text, rank 3)
    const std::string eq(equation);
    if (n == 2 && ops[0]->ndim == 3 && ops[1]->ndim == 3 && (eq == "ihd,jhd->ihj" || eq == "ihj,jhd->ihd")) {
        e->kind = eq == "ihd,jhd->ihj" ? 1 : 2;
        e->out_nd = 3;
        e->out_shape[0] = ops[0]->shape[0];
        e->out_shape[1] = ops[0]->shape[1];
        e->out_shape[2] = e->kind == 1 ? ops[1]->shape[0] : ops[1]->shape[2];
        return TLHIP_OK;
    }
    if (e->f32)
        return fail(TLHIP_ERR_INVALID_OPERATION,
                    "einsum '%s' on f32 tensors: only ihd,jhd->ihj and ihj,jhd->ihd have f32 kernels", equation);
    if (n > EINSUM_MAX_OPS) return fail(TLHIP_ERR_INVALID_OPERATION, "einsum: at most %d operands", EINSUM_MAX_OPS);
    // index sizes (a repeated index must agree: ShapeMismatch, einsum.rs:231-246)
    int64_t dim_of[128];
    for (int c = 0; c < 128; c++) dim_of[c] = -1;
    std::string order;   // indices in order of first appearance
    for (int k = 0; k < n; k++) {
        const std::string& sp = ins[k];
        if ((int)sp.size() != ops[k]->ndim)
            return fail(TLHIP_ERR_INVALID_OPERATION, "einsum: operand %d has %d dims, spec '%s' names %d", k,
                        ops[k]->ndim, sp.c_str(), (int)sp.size());
        for (size_t i = 0; i < sp.size(); i++) {
            const char c = sp[i];
            if (!is_letter(c)) return fail(TLHIP_ERR_INVALID_OPERATION, "einsum: '%c' is not an index letter", c);
            const int64_t d = ops[k]->shape[i];
            if (dim_of[(int)c] < 0) {
                dim_of[(int)c] = d;
                order.push_back(c);
            } else if (dim_of[(int)c] != d) {
                return fail(TLHIP_ERR_SHAPE_MISMATCH, "einsum: index '%c' is %lld in one operand, %lld in another", c,
                            (long long)dim_of[(int)c], (long long)d);
            }
        }
    }
    if (out.size() > 8) return fail(TLHIP_ERR_INVALID_OPERATION, "einsum: output of %d dims", (int)out.size());
    for (size_t i = 0; i < out.size(); i++) {
        const char c = out[i];
        if (!is_letter(c) || dim_of[(int)c] < 0)
            return fail(TLHIP_ERR_INVALID_OPERATION, "Unknown index in output: %c", c);
        if (out.find(c) != i) return fail(TLHIP_ERR_INVALID_OPERATION, "einsum: output index '%c' repeats", c);
    }
    // summed indices: those not in the output, nested in order of first
    // appearance (outermost first)
    std::string sum;
    for (char c : order)
        if (out.find(c) == std::string::npos) sum.push_back(c);
    if ((int)sum.size() > EINSUM_MAX_SUM)
        return fail(TLHIP_ERR_INVALID_OPERATION, "einsum: %d summed indices (at most %d)", (int)sum.size(),
                    EINSUM_MAX_SUM);
    EinsumPlan& p = e->plan;
    p = EinsumPlan{};
    p.n_ops = n;
    p.n_out = (int)out.size();
    p.n_sum = (int)sum.size();
    e->n_out = 1;
    e->n_sum = 1;
    for (int d = 0; d < p.n_out; d++) {
        p.out_dim[d] = dim_of[(int)out[d]];
        e->out_shape[d] = p.out_dim[d];
        if (__builtin_mul_overflow(e->n_out, p.out_dim[d], &e->n_out))
            return fail(TLHIP_ERR_INVALID_OPERATION, "einsum: output too large");
    }
    // the reference's scalar output is a [1] tensor here (no rank-0 tensors)
    e->out_nd = p.n_out ? p.n_out : 1;
    if (!p.n_out) e->out_shape[0] = 1;
    for (int d = 0; d < p.n_sum; d++) {
        p.sum_dim[d] = dim_of[(int)sum[d]];
        if (__builtin_mul_overflow(e->n_sum, p.sum_dim[d], &e->n_sum))
            return fail(TLHIP_ERR_INVALID_OPERATION, "einsum: summation space too large");
    }
    // one thread walks an output element's whole summation space: bound it
    // (2^31 terms per element, 2^36 in all) so that one launch cannot hold
    // the device for minutes
    int64_t work = 0;
    if (e->n_sum > ((int64_t)1 << 31) || __builtin_mul_overflow(e->n_out, e->n_sum, &work) ||
        work > ((int64_t)1 << 36))
        return fail(TLHIP_ERR_INVALID_OPERATION,
                    "einsum: %lld output elements x %lld summed terms is beyond the general kernel's bound",
                    (long long)e->n_out, (long long)e->n_sum);
    // element strides of every operand along each output / summed index (a
    // repeated index in one operand, e.g. "ii", adds its strides: the diagonal)
    for (int k = 0; k < n; k++) {
        const std::string& sp = ins[k];
        int64_t stride = 1;
        for (int i = (int)sp.size() - 1; i >= 0; i--) {
            const size_t po = out.find(sp[i]);
            if (po != std::string::npos) p.out_stride[k][po] += stride;
            else p.sum_stride[k][sum.find(sp[i])] += stride;
            stride *= ops[k]->shape[i];
        }
        p.op[k] = (const uint16_t*)ops[k]->data;
    }
    return TLHIP_OK;
}

}  // namespace

extern "C" {

tlhip_status tlhip_einsum_shape(const char* equation, const tlhip_tensor* operands, int n_operands, int* ndim,
                                int64_t* shape) try {
    if (!ndim || !shape) return fail(TLHIP_ERR_INVALID_ARGUMENT, "einsum_shape: null output");
    Einsum e;
    TLHIP_TRY(plan_einsum(equation, operands, n_operands, &e));
    *ndim = e.out_nd;
    for (int d = 0; d < e.out_nd; d++) shape[d] = e.out_shape[d];
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_einsum(tlhip_ctx ctx, const char* equation, const tlhip_tensor* operands, int n_operands,
                          tlhip_tensor out) try {
    TLHIP_TRY(check_ctx(ctx));
    Einsum e;
    TLHIP_TRY(plan_einsum(equation, operands, n_operands, &e));
    if (e.kind == 1) return tlhip_einsum_scores(ctx, operands[0], operands[1], out);
    if (e.kind == 2) return tlhip_einsum_context(ctx, operands[0], operands[1], out);
    TLHIP_TRY(check_t(out, "einsum output"));
    TLHIP_TRY(check_dtype(out, TLHIP_F16, "einsum"));
    if (out->ndim != e.out_nd || memcmp(out->shape, e.out_shape, sizeof(int64_t) * e.out_nd) != 0)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "einsum: output %s", shape_str(out).c_str());
    for (int k = 0; k < n_operands; k++)
        if (operands[k]->data == out->data)
            return fail(TLHIP_ERR_INVALID_ARGUMENT, "einsum: the output may not alias operand %d", k);
    if (e.n_out == 0) return TLHIP_OK;
    TLHIP_TRY(launch_einsum_general(ctx->stream, e.plan, (uint16_t*)out->data, e.n_out, e.n_sum));
    return after_launch(ctx, "einsum");
} TLHIP_CATCH_STATUS

}  // extern "C"
