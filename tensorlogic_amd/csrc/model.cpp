// model.cpp -- KV cache and the decoder runner.
//
// The runner executes the operator sequence of the reference's LLM programs
// (debug/chat_demo_with_kvcache.tl prefill/decode loops, chat_demo_optimized
// .tl:35-138) with the same f16 storage points, fused into fewer launches:
//   llama (TinyLlama) per layer, decode step:
//     rms_norm -> GEMV[q|k|v] -> rope(q,k) + cache write -> attention
//     -> GEMV[o] + residual -> rms_norm -> GEMV[gate/up rows interleaved]
//        + silu(gate)*up -> GEMV[down] + residual
//   phi2 per layer: layer_norm -> GEMV[qkv]+bias -> rope(NeoX, partial) +
//     cache write -> attention -> GEMV[o]+bias+residual ;
//     GEMV[up]+bias+gelu -> GEMV[down]+bias+residual
//   then final norm -> GEMV[lm_head] -> greedy argmax on the device.
// RoPE is applied at each token's absolute position and RMSNorm takes the
// GGUF file's eps by default: the reference's demo calls rope() without an
// offset in its decode loop, which rotates every new token as position 0,
// and rms_norm(x, w) at the builtin default 1e-6; the runner passes the
// position as rope(x, offset) allows (builtin_tensor.rs:514-556) and the
// model's own eps.  tlhip_model_set_program_semantics selects the program's
// literal choices instead.
//
// Decode state lives on the device: {token, pos, step}.  The embedding reads
// the token, RoPE / cache writes / attention read pos, the argmax writes the
// next token, advances pos and logs the token.  A decode step therefore has
// no host inputs and is captured once as a HIP graph and replayed.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "internal.hpp"

using namespace tlhip;

struct tlhip_kvcache_s {
    tlhip_ctx ctx = nullptr;
    tlhip_dtype dtype = TLHIP_F16;   // KVCache::new_f16 / new_f32
    int n_layers = 0, max_ctx = 0, n_kv = 0, head_dim = 0;
    std::vector<tlhip_tensor> k, v;
    std::vector<int> len;
};

namespace {

struct Lin {
    tlhip_tensor w = nullptr;
    tlhip_tensor b = nullptr;
};

struct Layer {
    tlhip_tensor norm_w = nullptr, norm_b = nullptr, ffn_norm_w = nullptr;
    Lin qkv, o, gu, up, down;
};

}  // namespace

struct tlhip_model_s {
    tlhip_ctx ctx = nullptr;
    int arch = 0;
    int n_layers = 0, hidden = 0, inter = 0, n_heads = 0, n_kv = 0, head_dim = 0, vocab = 0, rot = 0;
    int max_ctx = 0, max_rows = 0;
    float eps = 1e-5f, theta = 10000.0f;
    float gguf_eps = 1e-5f;                 // eps read from the file
    int literal = 0;                        // tlhip_model_set_program_semantics
    float* rope_id = nullptr;               // identity rotation table (every position = position 0)
    tlhip_tensor embd = nullptr, out_norm_w = nullptr, out_norm_b = nullptr;
    Lin out;
    std::vector<Layer> layers;
    tlhip_kvcache kv = nullptr;
    // activations, sized for max_rows tokens per pass
    tlhip_tensor x = nullptr, xn = nullptr, qkv = nullptr, qrot = nullptr, att = nullptr, hmid = nullptr,
                 logits = nullptr;
    unsigned long long* d_amax = nullptr;   // per-workgroup greedy keys of the lm_head GEMV
    uint16_t* d_vt = nullptr;                // V transposed per KV head for matrix-core prefill attention
    float* d_asplit = nullptr;               // decode attention split over key chunks (long caches)
    void* d_sample = nullptr;                // per-slice statistics of the temperature sampler
    float* ws = nullptr;          // split-K partials of the prefill GEMMs
    size_t ws_bytes = 0;
    int32_t* d_state = nullptr;   // {token, pos, step}
    int32_t* d_tokens = nullptr;  // token log
    int32_t* d_ids = nullptr;     // prompt ids
    int32_t* h_state = nullptr;   // pinned
    const float* rope_tab = nullptr;
    int pos = 0;
    float temperature = 0.0f;               // decode token choice: <= 1e-4 greedy, else sampled
    uint64_t seed = 0;
    // decode graphs of kGraphSteps[i] steps each (made on first use)
    hipGraphExec_t gexec[2] = {nullptr, nullptr};
    hipGraph_t graph[2] = {nullptr, nullptr};
    // phi2, one row: x + dense (x1) and fc2 + bias (mlp) of a layer whose
    // dense and fc2 shared a launch; the next layer_norm prologue adds them
    tlhip_tensor x1 = nullptr, mlp = nullptr;
};

namespace {

uint16_t* P(tlhip_tensor t) { return (uint16_t*)t->data; }

void free_lin(Lin& l) {
    tlhip_tensor_free(l.w);
    tlhip_tensor_free(l.b);
    l.w = l.b = nullptr;
}

tlhip_dtype dtype_of(uint32_t gt) {
    switch (gt) {
        case 0: case 1: return TLHIP_F16;
        case 2: return TLHIP_Q4_0;
        case 8: return TLHIP_Q8_0;
        case 14: return TLHIP_Q6_K;
        default: return (tlhip_dtype)-1;
    }
}

// Loads a 1-D f16 vector of length n.
tlhip_status load_vec(tlhip_ctx ctx, tlhip_gguf g, const std::string& name, int64_t n, tlhip_tensor* out) {
    TLHIP_TRY(tlhip_gguf_load_tensor(ctx, g, name.c_str(), out));
    const int64_t got = numel(*out);
    if (got != n || (*out)->dtype != TLHIP_F16) {
        tlhip_tensor_free(*out);
        *out = nullptr;
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "%s: %lld elements, expected %lld f16", name.c_str(),
                    (long long)got, (long long)n);
    }
    return TLHIP_OK;
}

// Places the rows of GGUF weight `name` [n, k] into `dst` rows
// dst_row0, dst_row0 + step, ... (step 1: concatenation, 2: interleave).
tlhip_status place_rows(tlhip_ctx ctx, tlhip_gguf g, const std::string& name, int64_t n, int64_t k,
                        tlhip_tensor dst, int64_t dst_row0, int64_t step) {
    uint32_t gt;
    int nd;
    int64_t dims[4];
    const uint8_t* data;
    size_t nbytes;
    if (!gguf_lookup(g, name.c_str(), &gt, &nd, dims, &data, &nbytes))
        return fail(TLHIP_ERR_LOAD, "tensor %s not found in GGUF", name.c_str());
    if (nd != 2 || dims[0] != n || dims[1] != k)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "%s: [%lld, %lld], expected [%lld, %lld]", name.c_str(),
                    (long long)dims[0], (long long)dims[1], (long long)n, (long long)k);
    if (dtype_of(gt) != dst->dtype)
        return fail(TLHIP_ERR_DTYPE, "%s: GGUF type %u differs from the fused tensor's dtype", name.c_str(), gt);
    // F32 weights are rounded to f16 (RNE) on the host, as the reference's
    // loader stores them (gguf.rs: f32 -> f16 at load)
    std::vector<uint16_t> h16;
    if (gt == 0) {
        const size_t ne = (size_t)n * k;
        h16.resize(ne);
        const float* f = (const float*)data;
        for (size_t i = 0; i < ne; i++) h16[i] = f32_to_f16(f[i]);
        data = (const uint8_t*)h16.data();
        nbytes = ne * 2;
    }
    void* stage = nullptr;
    TLHIP_CHECK_HIP(hipMallocAsync(&stage, nbytes, ctx->stream));
    TLHIP_CHECK_HIP(hipMemcpyAsync(stage, data, nbytes, hipMemcpyHostToDevice, ctx->stream));
    tlhip_status st = TLHIP_OK;
    if (is_quant(dst->dtype)) {
        st = launch_repack_rows(ctx->stream, dst->dtype, (const uint8_t*)stage, dst->data, dst->scales, n, k,
                                dst->shape[0], dst_row0, step, 0);
    } else {
        const size_t rb = (size_t)k * 2;
        hipError_t e = hipMemcpy2DAsync((uint8_t*)dst->data + (size_t)dst_row0 * rb, rb * step, stage, rb, rb,
                                        (size_t)n, hipMemcpyDeviceToDevice, ctx->stream);
        if (e != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "hipMemcpy2DAsync: %s", hipGetErrorString(e));
    }
    (void)hipFreeAsync(stage, ctx->stream);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (st == TLHIP_OK && e != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "load %s: %s", name.c_str(), hipGetErrorString(e));
    return st;
}

// Row order of a stacked [q | k | v] projection for the fused QKV + RoPE
// epilogue: within each q and k head, rotary pair i (dims i and i + rot/2 of
// the half-rotation layout) moves to rows 2i, 2i + 1; pass-through dims and
// v keep their place.  perm[new_row] = source row.
std::vector<int64_t> neox_pair_order(int64_t nq, int64_t nk, int64_t nv, int D, int rot) {
    std::vector<int64_t> perm(nq + nk + nv);
    for (int64_t r = 0; r < nq + nk + nv; r++) {
        int64_t src = r;
        if (r < nq + nk) {
            const int64_t head0 = (r / D) * D;
            const int e = (int)(r % D);
            if (e < rot) src = head0 + (e / 2) + (e % 2) * (rot / 2);
        }
        perm[r] = src;
    }
    return perm;
}

// Uploads GGUF weight `name` [n, k] with its rows reordered by perm
// (Q4_0 / Q8_0 / f16), through a host copy of the reordered block rows.
tlhip_status load_rows_permuted(tlhip_ctx ctx, tlhip_gguf g, const std::string& name, int64_t n, int64_t k,
                                const std::vector<int64_t>& perm, tlhip_tensor* out) {
    uint32_t gt;
    int nd;
    int64_t dims[4];
    const uint8_t* data;
    size_t nbytes;
    if (!gguf_lookup(g, name.c_str(), &gt, &nd, dims, &data, &nbytes))
        return fail(TLHIP_ERR_LOAD, "tensor %s not found in GGUF", name.c_str());
    if (nd != 2 || dims[0] != n || dims[1] != k || (int64_t)perm.size() != n)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "%s: [%lld, %lld], expected [%lld, %lld]", name.c_str(),
                    (long long)dims[0], (long long)dims[1], (long long)n, (long long)k);
    const tlhip_dtype dt = dtype_of(gt);
    if (dt != TLHIP_Q4_0 && dt != TLHIP_Q8_0 && dt != TLHIP_F16)
        return fail(TLHIP_ERR_DTYPE, "%s: GGUF type %u not supported by the runner", name.c_str(), gt);
    std::vector<uint16_t> h16;
    if (gt == 0) {   // F32 -> f16 (RNE) on the host
        const size_t ne = (size_t)n * k;
        h16.resize(ne);
        const float* f = (const float*)data;
        for (size_t i = 0; i < ne; i++) h16[i] = f32_to_f16(f[i]);
        data = (const uint8_t*)h16.data();
        nbytes = ne * 2;
    }
    const size_t rb = nbytes / (size_t)n;
    std::vector<uint8_t> host(nbytes);
    for (int64_t r = 0; r < n; r++) memcpy(host.data() + (size_t)r * rb, data + (size_t)perm[r] * rb, rb);
    int64_t shp[2] = {n, k};
    TLHIP_TRY(alloc_tensor(ctx, dt, 2, shp, out));
    tlhip_status st = tlhip_tensor_upload(ctx, *out, host.data(), nbytes);
    if (st == TLHIP_OK && hipStreamSynchronize(ctx->stream) != hipSuccess)
        st = fail(TLHIP_ERR_DEVICE, "load %s", name.c_str());
    if (st != TLHIP_OK) {
        tlhip_tensor_free(*out);
        *out = nullptr;
    }
    return st;
}

// A 1-D f16 vector with its entries reordered by perm.
tlhip_status load_vec_permuted(tlhip_ctx ctx, tlhip_gguf g, const std::string& name,
                               const std::vector<int64_t>& perm, tlhip_tensor* out) {
    uint32_t gt;
    int nd;
    int64_t dims[4];
    const uint8_t* data;
    size_t nbytes;
    if (!gguf_lookup(g, name.c_str(), &gt, &nd, dims, &data, &nbytes))
        return fail(TLHIP_ERR_LOAD, "tensor %s not found in GGUF", name.c_str());
    if (!((gt == 1 && nbytes == perm.size() * 2) || (gt == 0 && nbytes == perm.size() * 4)))
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "%s: expected %zu f16 / f32 entries", name.c_str(), perm.size());
    std::vector<uint16_t> host(perm.size());
    for (size_t i = 0; i < perm.size(); i++) {
        if (gt == 1) {
            memcpy(&host[i], data + 2 * perm[i], 2);
        } else {
            float f;
            memcpy(&f, data + 4 * perm[i], 4);
            host[i] = f32_to_f16(f);
        }
    }
    int64_t shp[1] = {(int64_t)perm.size()};
    TLHIP_TRY(alloc_tensor(ctx, TLHIP_F16, 1, shp, out));
    tlhip_status st = tlhip_tensor_upload(ctx, *out, host.data(), host.size() * 2);
    if (st == TLHIP_OK && hipStreamSynchronize(ctx->stream) != hipSuccess)
        st = fail(TLHIP_ERR_DEVICE, "load %s", name.c_str());
    if (st != TLHIP_OK) {
        tlhip_tensor_free(*out);
        *out = nullptr;
    }
    return st;
}

tlhip_status weight_dtype(tlhip_gguf g, const std::string& name, tlhip_dtype* dt) {
    uint32_t gt;
    int nd;
    int64_t dims[4];
    const uint8_t* data;
    size_t nbytes;
    if (!gguf_lookup(g, name.c_str(), &gt, &nd, dims, &data, &nbytes))
        return fail(TLHIP_ERR_LOAD, "tensor %s not found in GGUF", name.c_str());
    *dt = dtype_of(gt);
    if ((int)*dt < 0) return fail(TLHIP_ERR_DTYPE, "%s: GGUF type %u not supported on the device", name.c_str(), gt);
    return TLHIP_OK;
}

// A fused weight made of `parts` (name, rows) stacked along N.
tlhip_status fused_weight(tlhip_ctx ctx, tlhip_gguf g, const std::vector<std::pair<std::string, int64_t>>& parts,
                          int64_t k, bool interleave, tlhip_tensor* out) {
    tlhip_dtype dt;
    TLHIP_TRY(weight_dtype(g, parts[0].first, &dt));
    // Q6_K (real Q4_0 checkpoints store output.weight so) runs through the
    // decode GEMV only; the runner computes logits for one row at a time
    if (dt == TLHIP_Q6_K && !(parts.size() == 1 && parts[0].first == "output.weight"))
        return fail(TLHIP_ERR_DTYPE, "%s: Q6_K is supported for output.weight and token_embd.weight",
                    parts[0].first.c_str());
    int64_t n = 0;
    for (auto& p : parts) n += p.second;
    int64_t shp[2] = {n, k};
    TLHIP_TRY(alloc_tensor(ctx, dt, 2, shp, out));
    int64_t row0 = 0;
    for (size_t i = 0; i < parts.size(); i++) {
        tlhip_status st = interleave ? place_rows(ctx, g, parts[i].first, parts[i].second, k, *out, (int64_t)i,
                                                  (int64_t)parts.size())
                                     : place_rows(ctx, g, parts[i].first, parts[i].second, k, *out, row0, 1);
        if (st != TLHIP_OK) {
            tlhip_tensor_free(*out);
            *out = nullptr;
            return st;
        }
        row0 += parts[i].second;
    }
    return TLHIP_OK;
}

tlhip_status linear_into(hipStream_t s, const Lin& l, const uint16_t* x, int M, uint16_t* y, int epi,
                         const uint16_t* resid, int ldy = 0, float* ws = nullptr, size_t ws_bytes = 0,
                         uint32_t* tile_flags = nullptr) {
    GemvArgs a;
    a.ws = ws;
    a.ws_bytes = ws_bytes;
    a.tile_flags = tile_flags;
    a.x = x;
    a.wq = l.w->data;
    a.wd = l.w->scales;
    a.bias = l.b ? P(l.b) : nullptr;
    a.resid = resid;
    a.y = y;
    a.M = M;
    a.N = (int)l.w->shape[0];
    a.K = (int)l.w->shape[1];
    a.ldy = ldy;
    if (M <= 4) {
        tlhip_status st = launch_gemv(s, l.w->dtype, a, epi);
        if (st == TLHIP_OK) return st;
    }
    return launch_gemm(s, l.w->dtype, a, epi);
}

// One activation row through norm -> linear in a single GEMV launch: the
// normalisation (rms_norm or layer_norm with the reference's formula and
// f16 store) is formed in registers by every wave.
GemvArgs fused_norm_args(tlhip_model m, const Lin& l, const uint16_t* x, tlhip_tensor nw, tlhip_tensor nb) {
    GemvArgs a;
    a.x = x;
    a.wq = l.w->data;
    a.wd = l.w->scales;
    a.bias = l.b ? P(l.b) : nullptr;
    a.M = 1;
    a.N = (int)l.w->shape[0];
    a.K = (int)l.w->shape[1];
    a.pro = m->arch == 0 ? PRO_RMS : PRO_LN;
    a.norm_w = P(nw);
    a.norm_b = nb ? P(nb) : nullptr;
    a.eps = m->eps;
    return a;
}

// Enqueues the layers and the head for S tokens at positions pos0.. (plus
// *d_pos when given), ending with the argmax that updates d_state.
// A single-row pass (every decode step) runs five launches per llama layer:
//   [rms_norm + qkv + rope + cache write] [attention] [o + residual]
//   [rms_norm + gate/up + silu*mul] [down + residual]
// and norm + lm_head as one launch; longer passes run the unfused sequence
// with the MFMA GEMM.
tlhip_status enqueue_forward(tlhip_model m, int S, int pos0, const int32_t* ids_dev, bool decode) {
    hipStream_t s = m->ctx->stream;
    const int H = m->hidden, D = m->head_dim, NH = m->n_heads, NKV = m->n_kv, kvd = NKV * D;
    const int32_t* d_pos = decode ? m->d_state + 1 : nullptr;
    const bool row1 = S == 1;
    // decode with an f16 table: the embedding row is read by layer 0's fused
    // norm + QKV GEMV directly (and copied to the residual stream there)
    const bool embd_fused = decode && m->embd->dtype == TLHIP_F16;
    if (!embd_fused)
        TLHIP_TRY(launch_embedding(s, m->embd->dtype, m->embd->data, m->embd->scales, ids_dev,
                                   decode ? m->d_state : nullptr, P(m->x), S, H, m->vocab));
    auto embed_into = [&](GemvArgs& a, int li) {
        if (embd_fused && li == 0) {
            a.embd = P(m->embd);
            a.d_token = m->d_state;
            a.x_out = P(m->x);
        }
    };
    const int qkv_w = H + 2 * kvd;
    // phi2, one row: after a layer whose dense and fc2 shared one launch the
    // residual is x1 + mlp, added by the next layer_norm prologue (which
    // writes the sum back to x for that layer's dense)
    bool pending_add = false;
    for (int li = 0; li < m->n_layers; li++) {
        Layer& L = m->layers[li];
        uint16_t* kc = P(m->kv->k[li]);
        uint16_t* vc = P(m->kv->v[li]);
        if (row1) {
            // norm + qkv (+ bias) + RoPE + cache write in one launch; phi2's
            // q / k rows were loaded in rotary-pair order
            GemvArgs a = fused_norm_args(m, L.qkv, P(m->x), L.norm_w, L.norm_b);
            embed_into(a, li);
            if (pending_add) {
                a.x = P(m->x1);
                a.x_add = P(m->mlp);
                a.x_out = P(m->x);
            }
            a.nq = H;
            a.nk = kvd;
            a.head_dim = D;
            a.rot = m->rot;
            a.layout = m->arch == 0 ? 0 : 1;
            a.pos0 = decode ? 0 : pos0;
            a.d_pos = d_pos;
            // the program as written rotates a decode row as position 0:
            // cos 1, sin 0 at every cache row
            a.rope_tab = decode && m->literal ? m->rope_id : m->rope_tab;
            a.q_out = P(m->qrot);
            a.kc = kc;
            a.vc = vc;
            // phi2: the MLP's layer_norm is this one (same row, same weights):
            // the normalised row is kept for the fc1 GEMV
            if (m->arch == 1) a.xn_out = P(m->xn);
            TLHIP_TRY(launch_gemv(s, L.qkv.w->dtype, a, EPI_QKV_ROPE));
        } else {
            if (m->arch == 0) TLHIP_TRY(launch_rms_norm(s, P(m->x), P(L.norm_w), P(m->xn), S, H, m->eps));
            else TLHIP_TRY(launch_layer_norm(s, P(m->x), P(L.norm_w), P(L.norm_b), P(m->xn), S, H, m->eps));
            if (!decode && gemm_skinny_ok(S, qkv_w, H, L.qkv.w->dtype)) {
                // qkv (+ bias) + RoPE + cache write in the GEMM's epilogue
                GemvArgs a;
                a.x = P(m->xn);
                a.wq = L.qkv.w->data;
                a.wd = L.qkv.w->scales;
                a.bias = L.qkv.b ? P(L.qkv.b) : nullptr;
                a.y = P(m->qkv);
                a.M = S;
                a.N = qkv_w;
                a.K = H;
                a.ws = m->ws;
                a.ws_bytes = m->ws_bytes;
                a.tile_flags = m->ctx->d_tile_flags;
                a.nq = H;
                a.nk = kvd;
                a.head_dim = D;
                a.rot = m->rot;
                a.layout = m->arch == 0 ? 0 : 1;
                a.pos0 = pos0;
                a.rope_tab = m->rope_tab;
                a.q_out = P(m->qrot);
                a.kc = kc;
                a.vc = vc;
                TLHIP_TRY(launch_gemm(s, L.qkv.w->dtype, a, EPI_QKV_ROPE));
            } else {
                TLHIP_TRY(linear_into(s, L.qkv, P(m->xn), S, P(m->qkv), L.qkv.b ? EPI_BIAS : EPI_STORE, nullptr, 0, m->ws, m->ws_bytes, m->ctx->d_tile_flags));
                TLHIP_TRY(launch_rope_kv(s, P(m->qkv), qkv_w, S, NH, NKV, D, m->arch == 0 ? 0 : 2, m->rot,
                                         m->rope_tab, decode ? 0 : pos0, d_pos, P(m->qrot), kc, vc));
            }
        }
        AttnArgs at;
        at.q = P(m->qrot);
        at.k = kc;
        at.v = vc;
        at.out = P(m->att);
        at.S = S;
        at.H = NH;
        at.Hkv = NKV;
        at.D = D;
        at.causal = 1;
        at.kv_rows = m->max_ctx;
        at.scale_h = (float)(_Float16)(1.0f / sqrtf((float)D));
        at.head_flags = m->ctx->d_tile_flags + SK_MAX_TILES_SPLIT;
        // phi2, decode: fc1 reads only the normalised row the QKV launch
        // wrote, so it shares the attention's launch when the shapes allow
        bool fc1_done = false;
        if (decode) {
            at.d_pos = d_pos;
            if (m->arch == 1 && row1 && m->d_asplit) {
                GemvArgs f;
                f.x = P(m->xn);
                f.wq = L.up.w->data;
                f.wd = L.up.w->scales;
                f.bias = L.up.b ? P(L.up.b) : nullptr;
                f.y = P(m->hmid);
                f.M = 1;
                f.N = (int)L.up.w->shape[0];
                f.K = (int)L.up.w->shape[1];
                fc1_done = launch_attention_split_fc1(s, at, m->d_asplit, L.up.w->dtype, f);
            }
            if (!fc1_done) {
                if (m->d_asplit && attention_split_ok(at)) TLHIP_TRY(launch_attention_split(s, at, m->d_asplit));
                else TLHIP_TRY(launch_attention(s, at));
            }
        } else {
            at.q_pos0 = pos0;
            if (attention_mfma_ok(at, pos0 + S)) TLHIP_TRY(launch_attention_mfma(s, at, pos0 + S, m->d_vt));
            else if (pos0 + S > kAttnRowKeys && m->d_asplit && attention_split_j_ok(at, pos0 + S))
                TLHIP_TRY(launch_attention_split_j(s, at, pos0 + S, m->d_asplit));   // one row past the score row
            else TLHIP_TRY(launch_attention_j(s, at, pos0 + S));
        }
        if (m->arch == 0) {
            TLHIP_TRY(linear_into(s, L.o, P(m->att), S, P(m->x), EPI_RESID, P(m->x), 0, m->ws, m->ws_bytes, m->ctx->d_tile_flags));
            if (row1) {
                GemvArgs a = fused_norm_args(m, L.gu, P(m->x), L.ffn_norm_w, nullptr);
                a.y = P(m->hmid);
                TLHIP_TRY(launch_gemv(s, L.gu.w->dtype, a, EPI_SWIGLU_PAIR));
            } else {
                TLHIP_TRY(launch_rms_norm(s, P(m->x), P(L.ffn_norm_w), P(m->xn), S, H, m->eps));
                TLHIP_TRY(linear_into(s, L.gu, P(m->xn), S, P(m->hmid), EPI_SWIGLU_PAIR, nullptr, 0, m->ws, m->ws_bytes, m->ctx->d_tile_flags));
            }
            TLHIP_TRY(linear_into(s, L.down, P(m->hmid), S, P(m->x), EPI_RESID, P(m->x), 0, m->ws, m->ws_bytes, m->ctx->d_tile_flags));
        } else {
            // phi2: the MLP reads the same layer_norm output as attention --
            // with one row, the one the QKV launch wrote (measured on MI355X:
            // fc1 [10240 x 2560] Q8_0 as its own normalised GEMV 8.67 us)
            if (!fc1_done)
                TLHIP_TRY(linear_into(s, L.up, P(m->xn), S, P(m->hmid), EPI_BIAS_GELU, nullptr, 0, m->ws, m->ws_bytes, m->ctx->d_tile_flags));
            // one row: dense (x1 = x + dense + bias) and fc2 (mlp = fc2 + bias)
            // in one launch; the reference's x + dense + mlp is then completed,
            // with the same f16 roundings, by the next layer_norm prologue
            bool paired = false;
            if (row1 && m->x1 && m->mlp && L.o.b && L.down.b && L.o.w->dtype == L.down.w->dtype) {
                GemvArgs d, f;
                d.x = P(m->att);
                d.wq = L.o.w->data;
                d.wd = L.o.w->scales;
                d.bias = P(L.o.b);
                d.resid = P(m->x);
                d.y = P(m->x1);
                d.N = (int)L.o.w->shape[0];
                d.K = (int)L.o.w->shape[1];
                f.x = P(m->hmid);
                f.wq = L.down.w->data;
                f.wd = L.down.w->scales;
                f.bias = P(L.down.b);
                f.y = P(m->mlp);
                f.N = (int)L.down.w->shape[0];
                f.K = (int)L.down.w->shape[1];
                paired = launch_m1_pair(s, L.o.w->dtype, d, EPI_BIAS_RESID, f, EPI_BIAS);
            }
            if (!paired) {
                TLHIP_TRY(linear_into(s, L.o, P(m->att), S, P(m->x), EPI_BIAS_RESID, P(m->x), 0, m->ws, m->ws_bytes, m->ctx->d_tile_flags));
                TLHIP_TRY(linear_into(s, L.down, P(m->hmid), S, P(m->x), EPI_BIAS_RESID, P(m->x), 0, m->ws, m->ws_bytes, m->ctx->d_tile_flags));
            }
            pending_add = paired;
        }
    }
    const uint16_t* last = P(m->x) + (size_t)(S - 1) * H;
    {
        // final norm + lm_head (+ bias) + per-workgroup greedy keys, then the
        // one-workgroup reduction that picks the token and advances d_state
        GemvArgs a = fused_norm_args(m, m->out, last, m->out_norm_w, m->out_norm_b);
        if (pending_add) {   // (one row)
            a.x = P(m->x1);
            a.x_add = P(m->mlp);
        }
        a.y = P(m->logits);
        a.amax_slots = m->d_amax;
        TLHIP_TRY(launch_gemv(s, m->out.w->dtype, a, EPI_ARGMAX));
    }
    if (m->temperature > 1e-4f)
        TLHIP_TRY(launch_sample(s, P(m->logits), m->vocab, m->temperature, m->seed, 0, m->d_sample, nullptr, m->d_tokens,
                                m->d_state));
    else
        TLHIP_TRY(launch_argmax_slots(s, m->d_amax, gemv_norm_slots(m->vocab), nullptr, m->d_tokens, m->d_state));
    return TLHIP_OK;
}

tlhip_status set_state(tlhip_model m, int token, int pos, int step) {
    // h_state is only rewritten after the stream has drained (every caller
    // synchronises before returning), so the async copy reads stable memory.
    m->h_state[0] = token;
    m->h_state[1] = pos;
    m->h_state[2] = step;
    TLHIP_CHECK_HIP(hipMemcpyAsync(m->d_state, m->h_state, 3 * sizeof(int32_t), hipMemcpyHostToDevice, m->ctx->stream));
    return TLHIP_OK;
}

tlhip_status read_state(tlhip_model m, int32_t* token) {
    TLHIP_CHECK_HIP(hipMemcpyAsync(m->h_state, m->d_state, 3 * sizeof(int32_t), hipMemcpyDeviceToHost, m->ctx->stream));
    TLHIP_CHECK_HIP(hipStreamSynchronize(m->ctx->stream));
    if (token) *token = m->h_state[0];
    return TLHIP_OK;
}

// Prefill in chunks of at most max_rows tokens; leaves d_state =
// {next token, pos0 + n, step + 1} and logs the token at `step`.
tlhip_status prefill(tlhip_model m, const int32_t* ids, int n, int step) {
    if (n <= 0) return fail(TLHIP_ERR_INVALID_ARGUMENT, "prefill of %d tokens", n);
    if (m->pos + n > m->max_ctx)
        return fail(TLHIP_ERR_INDEX_OUT_OF_BOUNDS, "context overflow: %d + %d > %d", m->pos, n, m->max_ctx);
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= m->vocab)
            return fail(TLHIP_ERR_INDEX_OUT_OF_BOUNDS, "token id %d out of range [0, %d)", ids[i], m->vocab);
    for (int c0 = 0; c0 < n; c0 += m->max_rows) {
        const int S = std::min(m->max_rows, n - c0);
        TLHIP_CHECK_HIP(hipMemcpyAsync(m->d_ids, ids + c0, sizeof(int32_t) * S, hipMemcpyHostToDevice, m->ctx->stream));
        TLHIP_TRY(set_state(m, 0, m->pos + S - 1, step));
        TLHIP_TRY(enqueue_forward(m, S, m->pos, m->d_ids, false));
        TLHIP_CHECK_HIP(hipStreamSynchronize(m->ctx->stream));   // ids / h_state reuse
        m->pos += S;
    }
    TLHIP_CHECK_HIP(hipGetLastError());
    return TLHIP_OK;
}

// Steps per captured decode graph.  Each step reads its token and position
// from d_state and advances them, so k steps captured back to back replay as
// k decode steps; a launch of the 8-step graph pays the per-launch cost of a
// graph once for 8 tokens (measured on MI355X, config-4 decode: 2144 -> 2167
// tok/s, same tokens).
constexpr int kGraphSteps[2] = {1, 8};

tlhip_status ensure_graph(tlhip_model m, int k) {
    if (m->gexec[k]) return TLHIP_OK;
    hipStream_t s = m->ctx->stream;
    TLHIP_CHECK_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    tlhip_status st = TLHIP_OK;
    for (int i = 0; i < kGraphSteps[k] && st == TLHIP_OK; i++) st = enqueue_forward(m, 1, 0, nullptr, true);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (st != TLHIP_OK) {
        if (g) (void)hipGraphDestroy(g);
        return st;
    }
    if (e != hipSuccess) return fail(TLHIP_ERR_DEVICE, "graph capture failed: %s", hipGetErrorString(e));
    e = hipGraphInstantiate(&m->gexec[k], g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return fail(TLHIP_ERR_DEVICE, "graph instantiate failed: %s", hipGetErrorString(e));
    }
    m->graph[k] = g;
    return TLHIP_OK;
}

// Drops the captured graphs (their launches bake in the sampling and
// semantics settings).
void drop_graphs(tlhip_model m) {
    for (int k = 0; k < 2; k++) {
        if (m->gexec[k]) (void)hipGraphExecDestroy(m->gexec[k]);
        if (m->graph[k]) (void)hipGraphDestroy(m->graph[k]);
        m->gexec[k] = nullptr;
        m->graph[k] = nullptr;
    }
}

tlhip_status decode_steps(tlhip_model m, int n, bool use_graph) {
    if (m->pos + n > m->max_ctx)
        return fail(TLHIP_ERR_INDEX_OUT_OF_BOUNDS, "context overflow: %d + %d > %d", m->pos, n, m->max_ctx);
    if (use_graph) {
        int i = 0;
        if (n >= kGraphSteps[1]) {
            TLHIP_TRY(ensure_graph(m, 1));
            for (; i + kGraphSteps[1] <= n; i += kGraphSteps[1]) TLHIP_CHECK_HIP(hipGraphLaunch(m->gexec[1], m->ctx->stream));
        }
        if (i < n) TLHIP_TRY(ensure_graph(m, 0));
        for (; i < n; i++) TLHIP_CHECK_HIP(hipGraphLaunch(m->gexec[0], m->ctx->stream));
    } else {
        for (int i = 0; i < n; i++) TLHIP_TRY(enqueue_forward(m, 1, 0, nullptr, true));
    }
    m->pos += n;
    return TLHIP_OK;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------------------
// KV cache
// ---------------------------------------------------------------------------
static tlhip_status kvcache_create(tlhip_ctx ctx, int n_layers, int max_ctx, int n_kv_heads, int head_dim,
                                   tlhip_dtype dtype, tlhip_kvcache* out) {
    TLHIP_TRY(check_ctx(ctx));
    if (!out) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null output");
    *out = nullptr;
    if (n_layers <= 0 || max_ctx <= 0 || n_kv_heads <= 0 || head_dim <= 0)
        return fail(TLHIP_ERR_INVALID_DIMENSION, "kvcache: bad sizes");
    // the attention entry points read at most kAttnMaxKeys keys: a longer
    // cache could be appended past what it can attend
    if (max_ctx > kAttnMaxKeys)
        return fail(TLHIP_ERR_INVALID_DIMENSION, "kvcache: max_ctx %d > %d keys, the most attention reads", max_ctx,
                    kAttnMaxKeys);
    auto* c = new tlhip_kvcache_s();
    c->ctx = ctx;
    c->dtype = dtype;
    c->n_layers = n_layers;
    c->max_ctx = max_ctx;
    c->n_kv = n_kv_heads;
    c->head_dim = head_dim;
    c->len.assign(n_layers, 0);
    int64_t shp[3] = {max_ctx, n_kv_heads, head_dim};
    for (int i = 0; i < n_layers; i++) {
        tlhip_tensor k = nullptr, v = nullptr;
        tlhip_status st = alloc_tensor(ctx, dtype, 3, shp, &k);
        if (st == TLHIP_OK) st = alloc_tensor(ctx, dtype, 3, shp, &v);
        if (st != TLHIP_OK) {
            tlhip_tensor_free(k);
            tlhip_kvcache_free(c);
            return st;
        }
        c->k.push_back(k);
        c->v.push_back(v);
    }
    *out = c;
    return TLHIP_OK;
}

tlhip_status tlhip_kvcache_create(tlhip_ctx ctx, int n_layers, int max_ctx, int n_kv_heads, int head_dim,
                                  tlhip_kvcache* out) try {
    return kvcache_create(ctx, n_layers, max_ctx, n_kv_heads, head_dim, TLHIP_F16, out);
} TLHIP_CATCH_STATUS

tlhip_status tlhip_kvcache_create_f32(tlhip_ctx ctx, int n_layers, int max_ctx, int n_kv_heads, int head_dim,
                                      tlhip_kvcache* out) try {
    return kvcache_create(ctx, n_layers, max_ctx, n_kv_heads, head_dim, TLHIP_F32, out);
} TLHIP_CATCH_STATUS

tlhip_status tlhip_kvcache_free(tlhip_kvcache c) try {
    if (!c) return TLHIP_OK;
    for (auto t : c->k) tlhip_tensor_free(t);
    for (auto t : c->v) tlhip_tensor_free(t);
    delete c;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

static tlhip_status kv_write(tlhip_ctx ctx, tlhip_kvcache c, int layer, tlhip_tensor k, tlhip_tensor v, bool append) {
    TLHIP_TRY(check_ctx(ctx));
    if (!c || layer < 0 || layer >= c->n_layers) return fail(TLHIP_ERR_INDEX_OUT_OF_BOUNDS, "kvcache layer %d", layer);
    TLHIP_TRY(check_t(k, "kvcache K"));
    TLHIP_TRY(check_t(v, "kvcache V"));
    TLHIP_TRY(check_dtype(k, c->dtype, "kvcache"));
    TLHIP_TRY(check_dtype(v, c->dtype, "kvcache"));
    const int64_t row = (int64_t)c->n_kv * c->head_dim;
    // K and V must have the same shape: same element count alone would let a
    // V of another layout (e.g. [S, D, Hkv]) be stored as if it were [S, Hkv, D]
    const bool same = k->ndim == v->ndim && memcmp(k->shape, v->shape, sizeof(int64_t) * k->ndim) == 0;
    if (k->ndim < 1 || numel(k) % row != 0 || !same || last_dim(k) != c->head_dim)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "kvcache: K %s / V %s for rows of [%d, %d]", shape_str(k).c_str(),
                    shape_str(v).c_str(), c->n_kv, c->head_dim);
    const int S = (int)(numel(k) / row);
    const int start = append ? c->len[layer] : 0;
    if (start + S > c->max_ctx)
        return fail(TLHIP_ERR_INDEX_OUT_OF_BOUNDS, "kvcache: %d + %d rows > %d", start, S, c->max_ctx);
    // (rows copied as 16-bit units: an f32 row is twice as many)
    const int ru = (int)row * (c->dtype == TLHIP_F32 ? 2 : 1);
    TLHIP_TRY(launch_copy_rows(ctx->stream, P(k), P(c->k[layer]), S, ru, ru, ru, nullptr, start));
    TLHIP_TRY(launch_copy_rows(ctx->stream, P(v), P(c->v[layer]), S, ru, ru, ru, nullptr, start));
    c->len[layer] = start + S;
    return after_launch(ctx, append ? "kvcache_append" : "kvcache_set");
}

tlhip_status tlhip_kvcache_set(tlhip_ctx ctx, tlhip_kvcache c, int layer, tlhip_tensor k, tlhip_tensor v) try {
    return kv_write(ctx, c, layer, k, v, false);
} TLHIP_CATCH_STATUS

tlhip_status tlhip_kvcache_append(tlhip_ctx ctx, tlhip_kvcache c, int layer, tlhip_tensor k, tlhip_tensor v) try {
    return kv_write(ctx, c, layer, k, v, true);
} TLHIP_CATCH_STATUS

tlhip_status tlhip_kvcache_get(tlhip_kvcache c, int layer, int which_v, tlhip_tensor* out) try {
    if (!c || !out || layer < 0 || layer >= c->n_layers)
        return fail(TLHIP_ERR_INDEX_OUT_OF_BOUNDS, "kvcache layer %d", layer);
    if (c->len[layer] == 0) return fail(TLHIP_ERR_INVALID_OPERATION, "kvcache layer %d is empty", layer);
    tlhip_tensor src = which_v ? c->v[layer] : c->k[layer];
    int64_t shp[3] = {c->len[layer], c->n_kv, c->head_dim};
    // a view of the first len rows: same storage, shorter leading dim
    auto* view = new tlhip_tensor_s();
    *view = *src;
    view->refcount = 1;
    view->f16_copy = nullptr;
    view->shape[0] = shp[0];
    view->base = src;
    src->refcount++;
    *out = view;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

int tlhip_kvcache_len(tlhip_kvcache c, int layer) try {
    if (!c || layer < 0 || layer >= c->n_layers) return -1;
    return c->len[layer];
} TLHIP_CATCH_VALUE(-1)

// Attention of S query rows against a KV cache layer after cache.append (the
// TL program's get_k / get_v + einsum / mask / softmax / einsum sequence):
// the queries are the cache's last S positions, len - S .. len - 1, causal.
tlhip_status tlhip_attention_prefill(tlhip_ctx ctx, tlhip_tensor q, tlhip_kvcache c, int layer, float scale,
                                     tlhip_tensor out) try {
    if (!c || layer < 0 || layer >= c->n_layers) return fail(TLHIP_ERR_INDEX_OUT_OF_BOUNDS, "kvcache layer %d", layer);
    TLHIP_TRY(check_t(q, "attention_prefill"));
    if (q->ndim != 3) return fail(TLHIP_ERR_INVALID_DIMENSION, "attention_prefill: q must be [S, H, D]");
    const int len = c->len[layer];
    const int64_t S = q->shape[0];
    if (S < 1 || S > len)
        return fail(TLHIP_ERR_INVALID_DIMENSION, "attention: %lld query rows for a cache of %d rows", (long long)S, len);
    tlhip_tensor k = nullptr, v = nullptr;
    TLHIP_TRY(tlhip_kvcache_get(c, layer, 0, &k));
    tlhip_status st = tlhip_kvcache_get(c, layer, 1, &v);
    if (st == TLHIP_OK) st = tlhip_attention(ctx, q, k, v, len - (int)S, scale, 1, out);
    (void)tlhip_tensor_free(k);
    if (v) (void)tlhip_tensor_free(v);
    return st;
} TLHIP_CATCH_STATUS

// One decode row: q [1, H, D] at the cache's last position.
tlhip_status tlhip_attention_decode(tlhip_ctx ctx, tlhip_tensor q, tlhip_kvcache c, int layer, float scale,
                                    tlhip_tensor out) try {
    TLHIP_TRY(check_t(q, "attention_decode"));
    if (q->ndim != 3 || q->shape[0] != 1)
        return fail(TLHIP_ERR_INVALID_DIMENSION, "attention_decode: q must be [1, H, D], got %s", shape_str(q).c_str());
    return tlhip_attention_prefill(ctx, q, c, layer, scale, out);
} TLHIP_CATCH_STATUS

// ---------------------------------------------------------------------------
// model
// ---------------------------------------------------------------------------
tlhip_status tlhip_model_free(tlhip_model m) try {
    if (!m) return TLHIP_OK;
    if (m->ctx) (void)hipStreamSynchronize(m->ctx->stream);
    drop_graphs(m);
    for (auto& L : m->layers) {
        tlhip_tensor_free(L.norm_w);
        tlhip_tensor_free(L.norm_b);
        tlhip_tensor_free(L.ffn_norm_w);
        free_lin(L.qkv);
        free_lin(L.o);
        free_lin(L.gu);
        free_lin(L.up);
        free_lin(L.down);
    }
    tlhip_tensor_free(m->embd);
    tlhip_tensor_free(m->out_norm_w);
    tlhip_tensor_free(m->out_norm_b);
    free_lin(m->out);
    tlhip_kvcache_free(m->kv);
    for (tlhip_tensor t : {m->x, m->xn, m->qkv, m->qrot, m->att, m->hmid, m->logits, m->x1, m->mlp}) tlhip_tensor_free(t);
    if (m->d_amax) (void)hipFree(m->d_amax);
    if (m->d_vt) (void)hipFree(m->d_vt);
    if (m->d_asplit) (void)hipFree(m->d_asplit);
    if (m->d_sample) (void)hipFree(m->d_sample);
    if (m->ws) (void)hipFree(m->ws);
    if (m->d_state) (void)hipFree(m->d_state);
    if (m->rope_id) (void)hipFree(m->rope_id);
    if (m->d_tokens) (void)hipFree(m->d_tokens);
    if (m->d_ids) (void)hipFree(m->d_ids);
    if (m->h_state) (void)hipHostFree(m->h_state);
    delete m;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_model_load(tlhip_ctx ctx, const char* path, int arch, int max_ctx, tlhip_model* out) try {
    TLHIP_TRY(check_ctx(ctx));
    if (!path || !out) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    if (arch != 0 && arch != 1) return fail(TLHIP_ERR_INVALID_ARGUMENT, "arch %d (0 = llama, 1 = phi2)", arch);
    if (max_ctx <= 0 || max_ctx > kAttnMaxKeys)
        return fail(TLHIP_ERR_INVALID_DIMENSION, "max_ctx %d not in 1..%d", max_ctx, kAttnMaxKeys);
    tlhip_gguf g;
    TLHIP_TRY(tlhip_gguf_open(path, &g));
    auto* m = new tlhip_model_s();
    m->ctx = ctx;
    m->arch = arch;
    m->max_ctx = max_ctx;
    const std::string a = arch == 0 ? "llama." : "phi2.";
    tlhip_status st = TLHIP_OK;
    auto kv_u = [&](const char* k, int* dst) {
        uint32_t u;
        if (st == TLHIP_OK) st = tlhip_gguf_kv_u32(g, (a + k).c_str(), &u);
        if (st == TLHIP_OK) *dst = (int)u;
    };
    kv_u("block_count", &m->n_layers);
    kv_u("embedding_length", &m->hidden);
    kv_u("feed_forward_length", &m->inter);
    kv_u("attention.head_count", &m->n_heads);
    kv_u("attention.head_count_kv", &m->n_kv);
    do {
        if (st != TLHIP_OK) break;
        if (m->n_heads <= 0 || m->hidden % m->n_heads || m->n_kv <= 0 || m->n_heads % m->n_kv) {
            st = fail(TLHIP_ERR_LOAD, "inconsistent head counts");
            break;
        }
        m->head_dim = m->hidden / m->n_heads;
        if (max_ctx > kAttnRowKeys && m->head_dim != 64 && m->head_dim != 80 && m->head_dim != 128) {
            // past the one-workgroup kernels' score row, attention takes the
            // key-chunked and matrix-core paths, which cover these head dims
            st = fail(TLHIP_ERR_INVALID_DIMENSION, "max_ctx %d > %d needs head_dim 64, 80 or 128 (got %d)", max_ctx,
                      kAttnRowKeys, m->head_dim);
            break;
        }
        float f;
        if (tlhip_gguf_kv_f32(g, (a + (arch == 0 ? "attention.layer_norm_rms_epsilon" : "attention.layer_norm_epsilon")).c_str(), &f) == TLHIP_OK)
            m->eps = f;
        m->gguf_eps = m->eps;
        if (tlhip_gguf_kv_f32(g, (a + "rope.freq_base").c_str(), &f) == TLHIP_OK) m->theta = f;
        uint32_t u;
        m->rot = tlhip_gguf_kv_u32(g, (a + "rope.dimension_count").c_str(), &u) == TLHIP_OK ? (int)u : m->head_dim;
        if (m->rot <= 0 || m->rot > m->head_dim || m->rot % 2) {
            st = fail(TLHIP_ERR_LOAD, "bad rope.dimension_count %d", m->rot);
            break;
        }
        const int64_t H = m->hidden, kvd = (int64_t)m->n_kv * m->head_dim, I = m->inter;
        if ((st = tlhip_gguf_load_tensor(ctx, g, "token_embd.weight", &m->embd)) != TLHIP_OK) break;
        if (m->embd->ndim != 2 || m->embd->shape[1] != H) {
            st = fail(TLHIP_ERR_SHAPE_MISMATCH, "token_embd.weight %s", shape_str(m->embd).c_str());
            break;
        }
        m->vocab = (int)m->embd->shape[0];
        if ((st = load_vec(ctx, g, "output_norm.weight", H, &m->out_norm_w)) != TLHIP_OK) break;
        if (arch == 1 && (st = load_vec(ctx, g, "output_norm.bias", H, &m->out_norm_b)) != TLHIP_OK) break;
        if ((st = fused_weight(ctx, g, {{"output.weight", m->vocab}}, H, false, &m->out.w)) != TLHIP_OK) break;
        if (arch == 1 && (st = load_vec(ctx, g, "output.bias", m->vocab, &m->out.b)) != TLHIP_OK) break;
        m->layers.resize(m->n_layers);
        for (int i = 0; i < m->n_layers && st == TLHIP_OK; i++) {
            Layer& L = m->layers[i];
            const std::string p = "blk." + std::to_string(i) + ".";
            if ((st = load_vec(ctx, g, p + "attn_norm.weight", H, &L.norm_w)) != TLHIP_OK) break;
            if (arch == 0) {
                if ((st = load_vec(ctx, g, p + "ffn_norm.weight", H, &L.ffn_norm_w)) != TLHIP_OK) break;
                if ((st = fused_weight(ctx, g, {{p + "attn_q.weight", H}, {p + "attn_k.weight", kvd}, {p + "attn_v.weight", kvd}},
                                       H, false, &L.qkv.w)) != TLHIP_OK) break;
                if ((st = fused_weight(ctx, g, {{p + "attn_output.weight", H}}, H, false, &L.o.w)) != TLHIP_OK) break;
                if ((st = fused_weight(ctx, g, {{p + "ffn_gate.weight", I}, {p + "ffn_up.weight", I}}, H, true, &L.gu.w)) != TLHIP_OK) break;
                if ((st = fused_weight(ctx, g, {{p + "ffn_down.weight", H}}, I, false, &L.down.w)) != TLHIP_OK) break;
            } else {
                if ((st = load_vec(ctx, g, p + "attn_norm.bias", H, &L.norm_b)) != TLHIP_OK) break;
                // q / k rows in rotary-pair order (see neox_pair_order)
                const auto perm = neox_pair_order(H, kvd, kvd, m->head_dim, m->rot);
                if ((st = load_rows_permuted(ctx, g, p + "attn_qkv.weight", H + 2 * kvd, H, perm, &L.qkv.w)) != TLHIP_OK) break;
                if ((st = load_vec_permuted(ctx, g, p + "attn_qkv.bias", perm, &L.qkv.b)) != TLHIP_OK) break;
                if ((st = fused_weight(ctx, g, {{p + "attn_output.weight", H}}, H, false, &L.o.w)) != TLHIP_OK) break;
                if ((st = load_vec(ctx, g, p + "attn_output.bias", H, &L.o.b)) != TLHIP_OK) break;
                if ((st = fused_weight(ctx, g, {{p + "ffn_up.weight", I}}, H, false, &L.up.w)) != TLHIP_OK) break;
                if ((st = load_vec(ctx, g, p + "ffn_up.bias", I, &L.up.b)) != TLHIP_OK) break;
                if ((st = fused_weight(ctx, g, {{p + "ffn_down.weight", H}}, I, false, &L.down.w)) != TLHIP_OK) break;
                if ((st = load_vec(ctx, g, p + "ffn_down.bias", H, &L.down.b)) != TLHIP_OK) break;
            }
        }
        if (st != TLHIP_OK) break;
        if ((st = tlhip_kvcache_create(ctx, m->n_layers, max_ctx, m->n_kv, m->head_dim, &m->kv)) != TLHIP_OK) break;
        m->max_rows = std::min(max_ctx, 512);
        const int64_t R = m->max_rows;
        const int64_t wide = std::max<int64_t>(H + 2 * kvd, arch == 0 ? I : I);
        int64_t s_x[2] = {R, H}, s_qkv[2] = {R, H + 2 * kvd}, s_h[2] = {R, std::max<int64_t>(wide, I)},
                s_l[1] = {m->vocab};
        if ((st = alloc_tensor(ctx, TLHIP_F16, 2, s_x, &m->x)) != TLHIP_OK) break;
        if ((st = alloc_tensor(ctx, TLHIP_F16, 2, s_x, &m->xn)) != TLHIP_OK) break;
        if ((st = alloc_tensor(ctx, TLHIP_F16, 2, s_qkv, &m->qkv)) != TLHIP_OK) break;
        if ((st = alloc_tensor(ctx, TLHIP_F16, 2, s_x, &m->qrot)) != TLHIP_OK) break;
        if ((st = alloc_tensor(ctx, TLHIP_F16, 2, s_x, &m->att)) != TLHIP_OK) break;
        if ((st = alloc_tensor(ctx, TLHIP_F16, 2, s_h, &m->hmid)) != TLHIP_OK) break;
        if ((st = alloc_tensor(ctx, TLHIP_F16, 1, s_l, &m->logits)) != TLHIP_OK) break;
        if (arch == 1) {
            const int64_t s_r[2] = {1, H};
            if ((st = alloc_tensor(ctx, TLHIP_F16, 2, s_r, &m->x1)) != TLHIP_OK) break;
            if ((st = alloc_tensor(ctx, TLHIP_F16, 2, s_r, &m->mlp)) != TLHIP_OK) break;
        }
        hipError_t e = hipMalloc(&m->d_state, 4 * sizeof(int32_t));
        if (e == hipSuccess) e = hipMalloc(&m->d_amax, sizeof(unsigned long long) * gemv_norm_slots(m->vocab));
        if (e == hipSuccess) e = hipMalloc(&m->d_vt, attention_mfma_scratch(m->max_ctx, m->n_kv, m->head_dim));
        {
            AttnArgs probe;
            probe.d_pos = (const int32_t*)m->d_state;
            probe.S = 1;
            probe.H = m->n_heads;
            probe.Hkv = m->n_kv;
            probe.D = m->head_dim;
            probe.kv_rows = m->max_ctx;
            if (e == hipSuccess && attention_split_ok(probe))
                e = hipMalloc(&m->d_asplit, attention_split_scratch(m->n_heads, m->max_ctx, m->head_dim));
        }
        if (e == hipSuccess) e = hipMalloc(&m->d_sample, sample_scratch_bytes(m->vocab));
        // split-K workspace: the largest partial set any prefill GEMM of this model uses
        if (e == hipSuccess) {
            const int64_t shapes[4][2] = {{H + 2 * kvd, H}, {H, H}, {arch == 0 ? 2 * I : I, H}, {H, I}};
            size_t need = 0;
            for (int rows = 5; rows <= (int)R; rows++)
                for (auto& sh : shapes) {
                    const int sp = gemm_splits(rows, (int)sh[0], (int)sh[1], -1);
                    if (sp > 1) need = std::max(need, (size_t)sp * rows * sh[0] * sizeof(float));
                }
            if (need) {
                e = hipMalloc(&m->ws, need);
                m->ws_bytes = need;
            }
        }
        if (e == hipSuccess) e = hipMalloc(&m->d_tokens, sizeof(int32_t) * (max_ctx + 1));
        if (e == hipSuccess) e = hipMalloc(&m->d_ids, sizeof(int32_t) * R);
        if (e == hipSuccess) e = hipHostMalloc(&m->h_state, 4 * sizeof(int32_t), hipHostMallocDefault);
        if (e != hipSuccess) {
            st = fail(TLHIP_ERR_ALLOCATION, "model buffers: %s", hipGetErrorString(e));
            break;
        }
        st = rope_table(ctx, m->theta, m->rot, max_ctx, &m->rope_tab);
    } while (0);
    tlhip_gguf_close(g);
    if (st == TLHIP_OK) {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "model load: %s", hipGetErrorString(e));
    }
    if (st != TLHIP_OK) {
        std::string msg = tlhip_last_error();
        tlhip_model_free(m);
        set_error(st, "%s", msg.c_str() + (msg.find(": ") != std::string::npos ? msg.find(": ") + 2 : 0));
        return st;
    }
    *out = m;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_model_reset(tlhip_model m) try {
    if (!m) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null model");
    m->pos = 0;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_model_set_sampling(tlhip_model m, float temperature, uint64_t seed) try {
    if (!m) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null model");
    if (!(temperature >= 0.0f) || !std::isfinite(temperature))
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "temperature %g", temperature);
    if (temperature == m->temperature && seed == m->seed) return TLHIP_OK;
    // the decode graph holds the token-choice kernel: capture it again
    TLHIP_CHECK_HIP(hipStreamSynchronize(m->ctx->stream));
    drop_graphs(m);
    m->temperature = temperature;
    m->seed = seed;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_model_set_program_semantics(tlhip_model m, int literal) try {
    if (!m) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null model");
    if (m->arch != 0)
        return fail(TLHIP_ERR_INVALID_OPERATION, "program semantics are defined for the llama program only");
    literal = literal != 0;
    if (literal == m->literal) return TLHIP_OK;
    // eps and the rotation table are arguments of the captured decode kernels
    TLHIP_CHECK_HIP(hipStreamSynchronize(m->ctx->stream));
    drop_graphs(m);
    if (literal && !m->rope_id) {
        // [max_ctx][rot/2] (cos, sin) = (1, 0): the table of position 0 at every row
        std::vector<float> h((size_t)m->max_ctx * (m->rot / 2) * 2);
        for (size_t i = 0; i < h.size(); i += 2) {
            h[i] = 1.0f;
            h[i + 1] = 0.0f;
        }
        TLHIP_CHECK_HIP(hipMalloc(&m->rope_id, h.size() * sizeof(float)));
        TLHIP_CHECK_HIP(hipMemcpy(m->rope_id, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
    }
    m->literal = literal;
    m->eps = literal ? 1e-6f : m->gguf_eps;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_model_dims(tlhip_model m, int32_t* d) try {
    if (!m || !d) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null argument");
    int32_t v[8] = {m->n_layers, m->hidden, m->inter, m->n_heads, m->n_kv, m->head_dim, m->vocab, m->rot};
    memcpy(d, v, sizeof v);
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_model_prefill(tlhip_model m, const int32_t* ids, int n, int32_t* next) try {
    if (!m || !ids) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null argument");
    TLHIP_TRY(prefill(m, ids, n, 0));
    return read_state(m, next);
} TLHIP_CATCH_STATUS

tlhip_status tlhip_model_decode(tlhip_model m, int32_t token, int32_t* next) try {
    if (!m) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null model");
    if (token < 0 || token >= m->vocab)
        return fail(TLHIP_ERR_INDEX_OUT_OF_BOUNDS, "token id %d out of range [0, %d)", token, m->vocab);
    TLHIP_TRY(set_state(m, token, m->pos, 0));
    TLHIP_TRY(decode_steps(m, 1, false));
    return read_state(m, next);
} TLHIP_CATCH_STATUS

tlhip_status tlhip_model_generate(tlhip_model m, const int32_t* prompt, int n_prompt, int n_decode, int use_graph,
                                  int32_t* tokens_out) try {
    if (!m || !prompt || !tokens_out) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null argument");
    if (n_decode < 0) return fail(TLHIP_ERR_INVALID_ARGUMENT, "n_decode < 0");
    m->pos = 0;
    if (n_prompt + n_decode > m->max_ctx)
        return fail(TLHIP_ERR_INDEX_OUT_OF_BOUNDS, "context overflow: %d + %d > %d", n_prompt, n_decode, m->max_ctx);
    TLHIP_TRY(prefill(m, prompt, n_prompt, 0));
    TLHIP_TRY(decode_steps(m, n_decode, use_graph != 0));
    TLHIP_CHECK_HIP(hipMemcpyAsync(tokens_out, m->d_tokens, sizeof(int32_t) * (n_decode + 1), hipMemcpyDeviceToHost,
                                   m->ctx->stream));
    TLHIP_CHECK_HIP(hipStreamSynchronize(m->ctx->stream));
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_model_logits(tlhip_model m, uint16_t* host, size_t n) try {
    if (!m || !host) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null argument");
    if (n != (size_t)m->vocab) return fail(TLHIP_ERR_SHAPE_MISMATCH, "logits has %d entries", m->vocab);
    TLHIP_CHECK_HIP(hipMemcpyAsync(host, m->logits->data, n * 2, hipMemcpyDeviceToHost, m->ctx->stream));
    TLHIP_CHECK_HIP(hipStreamSynchronize(m->ctx->stream));
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

// ---------------------------------------------------------------------------
// measurement helpers
// ---------------------------------------------------------------------------
tlhip_status tlhip_bench_linear(tlhip_ctx ctx, tlhip_tensor x, const tlhip_tensor* w, int n_w, tlhip_tensor y,
                                int iters, int per_launch, float* avg_us) try {
    TLHIP_TRY(check_ctx(ctx));
    if (!w || n_w <= 0 || iters <= 0 || !avg_us) return fail(TLHIP_ERR_INVALID_ARGUMENT, "bad bench arguments");
    for (int i = 0; i < n_w; i++) TLHIP_TRY(tlhip_linear(ctx, x, w[i], nullptr, y));   // checks + warm-up
    TLHIP_CHECK_HIP(hipStreamSynchronize(ctx->stream));
    Lin l;
    const bool gemm = x->shape[0] > 4;   // GEMMs go through tlhip_linear (split-K workspace)
    if (!per_launch) {
        TLHIP_CHECK_HIP(hipEventRecord(ctx->ev0, ctx->stream));
        for (int i = 0; i < iters; i++) {
            l.w = w[i % n_w];
            if (gemm) TLHIP_TRY(tlhip_linear(ctx, x, l.w, nullptr, y));
            else TLHIP_TRY(linear_into(ctx->stream, l, P(x), (int)x->shape[0], P(y), EPI_STORE, nullptr));
        }
        TLHIP_CHECK_HIP(hipEventRecord(ctx->ev1, ctx->stream));
        TLHIP_CHECK_HIP(hipEventSynchronize(ctx->ev1));
        float ms = 0.f;
        TLHIP_CHECK_HIP(hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1));
        *avg_us = ms * 1000.0f / (float)iters;
        return TLHIP_OK;
    }
    // one event pair around every launch: the mean of the bracketed times
    std::vector<hipEvent_t> ev(2 * (size_t)iters, nullptr);
    tlhip_status st = TLHIP_OK;
    for (auto& e : ev)
        if (hipEventCreate(&e) != hipSuccess) {
            st = fail(TLHIP_ERR_DEVICE, "hipEventCreate failed");
            break;
        }
    double total = 0.0;
    for (int i = 0; i < iters && st == TLHIP_OK; i++) {
        l.w = w[i % n_w];
        if (hipEventRecord(ev[2 * i], ctx->stream) != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "hipEventRecord");
        if (st == TLHIP_OK)
            st = gemm ? tlhip_linear(ctx, x, l.w, nullptr, y)
                      : linear_into(ctx->stream, l, P(x), (int)x->shape[0], P(y), EPI_STORE, nullptr);
        if (st == TLHIP_OK && hipEventRecord(ev[2 * i + 1], ctx->stream) != hipSuccess)
            st = fail(TLHIP_ERR_DEVICE, "hipEventRecord");
    }
    if (st == TLHIP_OK && hipStreamSynchronize(ctx->stream) != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "sync");
    for (int i = 0; i < iters && st == TLHIP_OK; i++) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]) != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "elapsed");
        total += ms;
    }
    for (auto e : ev)
        if (e) (void)hipEventDestroy(e);
    if (st == TLHIP_OK) *avg_us = (float)(total * 1000.0 / iters);
    return st;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_bench_copy(tlhip_ctx ctx, size_t bytes, int n_buf, int iters, float* avg_us) try {
    TLHIP_TRY(check_ctx(ctx));
    if (bytes < 16 || bytes % 16 || n_buf <= 0 || iters <= 0 || !avg_us)
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "bench_copy: bytes must be a positive multiple of 16");
    std::vector<void*> src(n_buf, nullptr);
    void* dst = nullptr;
    tlhip_status st = TLHIP_OK;
    for (auto& b : src)
        if (hipMalloc(&b, bytes) != hipSuccess) st = fail(TLHIP_ERR_ALLOCATION, "bench_copy: %zu bytes", bytes);
    if (st == TLHIP_OK && hipMalloc(&dst, bytes) != hipSuccess) st = fail(TLHIP_ERR_ALLOCATION, "bench_copy");
    for (auto b : src)
        if (st == TLHIP_OK && hipMemsetAsync(b, 1, bytes, ctx->stream) != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "memset");
    for (int i = 0; i < n_buf && st == TLHIP_OK; i++) st = launch_stream_copy(ctx->stream, src[i], dst, bytes);
    if (st == TLHIP_OK && hipStreamSynchronize(ctx->stream) != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "sync");
    float ms = 0.f;
    if (st == TLHIP_OK && hipEventRecord(ctx->ev0, ctx->stream) != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "event");
    for (int i = 0; i < iters && st == TLHIP_OK; i++) st = launch_stream_copy(ctx->stream, src[i % n_buf], dst, bytes);
    if (st == TLHIP_OK && hipEventRecord(ctx->ev1, ctx->stream) != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "event");
    if (st == TLHIP_OK && hipEventSynchronize(ctx->ev1) != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "sync");
    if (st == TLHIP_OK && hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1) != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "elapsed");
    (void)hipStreamSynchronize(ctx->stream);
    for (auto b : src)
        if (b) (void)hipFree(b);
    if (dst) (void)hipFree(dst);
    if (st == TLHIP_OK) *avg_us = ms * 1000.0f / (float)iters;
    return st;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_timer_start(tlhip_ctx ctx) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_CHECK_HIP(hipEventRecord(ctx->ev0, ctx->stream));
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_timer_stop(tlhip_ctx ctx, float* ms) try {
    TLHIP_TRY(check_ctx(ctx));
    if (!ms) return fail(TLHIP_ERR_INVALID_ARGUMENT, "timer_stop: null output");
    TLHIP_CHECK_HIP(hipEventRecord(ctx->ev1, ctx->stream));
    TLHIP_CHECK_HIP(hipEventSynchronize(ctx->ev1));
    TLHIP_CHECK_HIP(hipEventElapsedTime(ms, ctx->ev0, ctx->ev1));
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_bench_decode(tlhip_model m, const int32_t* prompt, int n_prompt, int n_decode, int use_graph,
                                int32_t* tokens_out, float* prefill_ms, float* decode_ms) try {
    if (!m || !prompt || !tokens_out || !prefill_ms || !decode_ms)
        return fail(TLHIP_ERR_INVALID_ARGUMENT, "null argument");
    if (n_prompt + n_decode > m->max_ctx)
        return fail(TLHIP_ERR_INDEX_OUT_OF_BOUNDS, "context overflow: %d + %d > %d", n_prompt, n_decode, m->max_ctx);
    tlhip_ctx ctx = m->ctx;
    if (use_graph) {   // (captured before the timed region)
        TLHIP_TRY(ensure_graph(m, 0));
        if (n_decode >= kGraphSteps[1]) TLHIP_TRY(ensure_graph(m, 1));
    }
    m->pos = 0;
    TLHIP_CHECK_HIP(hipStreamSynchronize(ctx->stream));
    TLHIP_CHECK_HIP(hipEventRecord(ctx->ev0, ctx->stream));
    TLHIP_TRY(prefill(m, prompt, n_prompt, 0));
    TLHIP_CHECK_HIP(hipEventRecord(ctx->ev1, ctx->stream));
    TLHIP_CHECK_HIP(hipEventSynchronize(ctx->ev1));
    TLHIP_CHECK_HIP(hipEventElapsedTime(prefill_ms, ctx->ev0, ctx->ev1));
    TLHIP_CHECK_HIP(hipEventRecord(ctx->ev0, ctx->stream));
    TLHIP_TRY(decode_steps(m, n_decode, use_graph != 0));
    TLHIP_CHECK_HIP(hipEventRecord(ctx->ev1, ctx->stream));
    TLHIP_CHECK_HIP(hipEventSynchronize(ctx->ev1));
    TLHIP_CHECK_HIP(hipEventElapsedTime(decode_ms, ctx->ev0, ctx->ev1));
    TLHIP_CHECK_HIP(hipMemcpy(tokens_out, m->d_tokens, sizeof(int32_t) * (n_decode + 1), hipMemcpyDeviceToHost));
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

}  // extern "C"
