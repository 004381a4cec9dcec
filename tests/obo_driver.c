/* obo_driver.c -- debug/chat_demo_with_kvcache.tl run op by op from C.
 *
 * The same call sequence as tensorlogic_amd/program.py (ChatDemoKVCache):
 * one tlhip_* entry point per TL builtin of the program's prefill
 * (chat_demo_with_kvcache.tl:130-186) and decode loop (:208-296), each op's
 * output allocated by the caller from the library's pool and freed after
 * its last use, with no Python in between.  Its per-token wall time is the
 * C ABI's own cost for an interpreter that calls the library one builtin at
 * a time; bench.py reports it beside the Python figure, and the tokens must
 * equal the Python runner's and the fused runner's in literal mode.
 *
 * Test and benchmark infrastructure: built by __graft_entry__.build() into
 * tests/libobo_driver.so (linked against tensorlogic_amd/libtlhip.so) and
 * called through ctypes (tests/obo.py).  Not part of the library.
 */
#include <stdio.h>
#include <string.h>
#include <time.h>

#include "../include/tl_hip.h"

static char g_err[1024];
static tlhip_ctx C;

#define CK(expr)                                                                     \
    do {                                                                             \
        tlhip_status s_ = (expr);                                                    \
        if (s_ != TLHIP_OK) {                                                        \
            snprintf(g_err, sizeof g_err, "%s: %s", #expr, tlhip_last_error());      \
            return -1;                                                               \
        }                                                                            \
    } while (0)

typedef struct {
    tlhip_tensor attn_norm, q, k, v, o, ffn_norm, gate, up, down;
} Layer;

typedef struct {
    int n_layers, hidden, n_heads, n_kv, head_dim, vocab, max_ctx, pos, rope_abs;
    float eps, scale;
    tlhip_tensor emb, out_norm, out;
    Layer L[128];
    tlhip_kvcache cache;
} Prog;

static int t_new(int nd, int64_t a, int64_t b, int64_t c, int64_t d, tlhip_tensor* out) {
    const int64_t s[4] = {a, b, c, d};
    CK(tlhip_tensor_alloc(C, TLHIP_F16, nd, s, out));
    return 0;
}

static int t_view(tlhip_tensor x, int nd, int64_t a, int64_t b, int64_t c, int64_t d, tlhip_tensor* out) {
    const int64_t s[4] = {a, b, c, d};
    CK(tlhip_tensor_reshape(x, nd, s, out));
    return 0;
}

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

/* x [rows, hidden] -> rms_norm(x, w, eps) */
static int rmsn(Prog* p, tlhip_tensor x, int rows, tlhip_tensor w, tlhip_tensor* y) {
    if (t_new(2, rows, p->hidden, 0, 0, y)) return -1;
    CK(tlhip_rms_norm(C, x, w, p->eps, *y));
    return 0;
}

static int lin(tlhip_tensor x, int rows, tlhip_tensor w, int n, tlhip_tensor* y) {
    if (t_new(2, rows, n, 0, 0, y)) return -1;
    CK(tlhip_linear(C, x, w, NULL, *y));
    return 0;
}

/* reshape [n, Hkv, 1, D] -> broadcast_to [n, Hkv, H/Hkv, D] -> reshape [n, H, D] */
static int expand(Prog* p, tlhip_tensor t, int n, tlhip_tensor* out) {
    tlhip_tensor g1, bc;
    const int grp = p->n_heads / p->n_kv;
    if (t_view(t, 4, n, p->n_kv, 1, p->head_dim, &g1)) return -1;
    if (t_new(4, n, p->n_kv, grp, p->head_dim, &bc)) return -1;
    CK(tlhip_broadcast_to(C, g1, bc));
    if (t_view(bc, 3, n, p->n_heads, p->head_dim, 0, out)) return -1;
    tlhip_tensor_free(g1);
    tlhip_tensor_free(bc);
    return 0;
}

/* silu(gate) * up -> down, as swiglu_ffn */
static int swiglu_ffn(Prog* p, Layer* L, tlhip_tensor x, int rows, tlhip_tensor* y) {
    tlhip_tensor gate, sg, ga, up, inter;
    int64_t shp[8];
    tlhip_dtype dt;
    int nd;
    CK(tlhip_tensor_info(L->gate, &dt, &nd, shp));
    const int inter_n = (int)shp[0];
    if (lin(x, rows, L->gate, inter_n, &gate)) return -1;
    if (t_new(2, rows, inter_n, 0, 0, &sg)) return -1;
    CK(tlhip_sigmoid(C, gate, sg));
    if (t_new(2, rows, inter_n, 0, 0, &ga)) return -1;
    CK(tlhip_mul(C, gate, sg, ga));
    if (lin(x, rows, L->up, inter_n, &up)) return -1;
    if (t_new(2, rows, inter_n, 0, 0, &inter)) return -1;
    CK(tlhip_mul(C, ga, up, inter));
    if (lin(inter, rows, L->down, p->hidden, y)) return -1;
    tlhip_tensor_free(gate);
    tlhip_tensor_free(sg);
    tlhip_tensor_free(ga);
    tlhip_tensor_free(up);
    tlhip_tensor_free(inter);
    return 0;
}

/* One layer's attention for S query rows at rope offset `off` against the
 * keys K_all / V_all [J, Hkv, D], causal mask [S, S] (prefill) or [1, 1]
 * (decode); returns attn_output.reshape([S, hidden]).linear(W_o). */
static int attention(Prog* p, Layer* L, tlhip_tensor q_rope, tlhip_tensor K_all, tlhip_tensor V_all, int S, int J,
                     tlhip_tensor* y) {
    const int NH = p->n_heads, D = p->head_dim;
    tlhip_tensor kx, vx, sc, ssc, cm, cm3, mb, masked, w, ao, aor;
    if (expand(p, K_all, J, &kx)) return -1;
    if (t_new(3, S, NH, J, 0, &sc)) return -1;
    CK(tlhip_einsum_scores(C, q_rope, kx, sc));
    if (t_new(3, S, NH, J, 0, &ssc)) return -1;
    CK(tlhip_mul_scalar(C, sc, p->scale, ssc));
    if (t_new(2, S, S, 0, 0, &cm)) return -1;
    CK(tlhip_causal_mask(C, cm));
    if (t_view(cm, 3, S, 1, S, 0, &cm3)) return -1;
    if (t_new(3, S, NH, J, 0, &mb)) return -1;
    CK(tlhip_broadcast_to(C, cm3, mb));
    if (t_new(3, S, NH, J, 0, &masked)) return -1;
    CK(tlhip_apply_attention_mask(C, ssc, mb, masked));
    if (t_new(3, S, NH, J, 0, &w)) return -1;
    CK(tlhip_softmax_lastdim(C, masked, w));
    if (expand(p, V_all, J, &vx)) return -1;
    if (t_new(3, S, NH, D, 0, &ao)) return -1;
    CK(tlhip_einsum_context(C, w, vx, ao));
    if (t_view(ao, 2, S, p->hidden, 0, 0, &aor)) return -1;
    if (lin(aor, S, L->o, p->hidden, y)) return -1;
    tlhip_tensor arr[] = {kx, sc, ssc, cm, cm3, mb, masked, w, vx, ao, aor};
    for (size_t i = 0; i < sizeof arr / sizeof arr[0]; i++) tlhip_tensor_free(arr[i]);
    return 0;
}

/* rows [S, Hx*D] -> reshape [S, Hx, D] -> rope(off) */
static int rope_rows(Prog* p, tlhip_tensor t, int S, int Hx, int off, tlhip_tensor* y) {
    tlhip_tensor r;
    if (t_view(t, 3, S, Hx, p->head_dim, 0, &r)) return -1;
    if (t_new(3, S, Hx, p->head_dim, 0, y)) return -1;
    CK(tlhip_rope(C, r, off, 10000.0f, TLHIP_ROPE_INTERLEAVED, 0, *y));
    tlhip_tensor_free(r);
    return 0;
}

/* the last rows' logits: rms_norm(x_last, output_norm).linear(output) */
static int head(Prog* p, tlhip_tensor x_last, tlhip_tensor* logits) {
    tlhip_tensor xn;
    if (rmsn(p, x_last, 1, p->out_norm, &xn)) return -1;
    if (lin(xn, 1, p->out, p->vocab, logits)) return -1;
    tlhip_tensor_free(xn);
    return 0;
}

static int layer_step(Prog* p, int li, tlhip_tensor* x, int S, int off, int decode) {
    Layer* L = &p->L[li];
    const int NKV = p->n_kv, D = p->head_dim, kvd = p->n_kv * p->head_dim;
    tlhip_tensor xn1, q, k, v, q_rope, k_rope, vh, K_all, V_all, attn_out, x1, xn2, ffn, x2;
    if (rmsn(p, *x, S, L->attn_norm, &xn1)) return -1;
    if (lin(xn1, S, L->q, p->hidden, &q)) return -1;
    if (decode && rope_rows(p, q, S, p->n_heads, off, &q_rope)) return -1;
    if (lin(xn1, S, L->k, kvd, &k)) return -1;
    if (lin(xn1, S, L->v, kvd, &v)) return -1;
    if (rope_rows(p, k, S, NKV, off, &k_rope)) return -1;
    if (t_view(v, 3, S, NKV, D, 0, &vh)) return -1;
    int J;
    if (decode) {
        CK(tlhip_kvcache_append(C, p->cache, li, k_rope, vh));
        CK(tlhip_kvcache_get(p->cache, li, 0, &K_all));
        CK(tlhip_kvcache_get(p->cache, li, 1, &V_all));
        J = tlhip_kvcache_len(p->cache, li);
    } else {
        /* prefill: cache.set, then tinyllama_gqa_attention(Q, K, V, W_o, S),
         * which rotates Q and K itself and reshapes V again */
        CK(tlhip_kvcache_set(C, p->cache, li, k_rope, vh));
        if (rope_rows(p, q, S, p->n_heads, off, &q_rope)) return -1;
        if (rope_rows(p, k, S, NKV, off, &K_all)) return -1;
        if (t_view(v, 3, S, NKV, D, 0, &V_all)) return -1;
        J = S;
    }
    if (attention(p, L, q_rope, K_all, V_all, S, J, &attn_out)) return -1;
    if (t_new(2, S, p->hidden, 0, 0, &x1)) return -1;
    CK(tlhip_add(C, *x, attn_out, x1));
    if (rmsn(p, x1, S, L->ffn_norm, &xn2)) return -1;
    if (swiglu_ffn(p, L, xn2, S, &ffn)) return -1;
    if (t_new(2, S, p->hidden, 0, 0, &x2)) return -1;
    CK(tlhip_add(C, x1, ffn, x2));
    tlhip_tensor arr[] = {xn1, q, k, v, q_rope, k_rope, vh, K_all, V_all, attn_out, x1, xn2, ffn, *x};
    for (size_t i = 0; i < sizeof arr / sizeof arr[0]; i++) tlhip_tensor_free(arr[i]);
    *x = x2;
    return 0;
}

static int prefill(Prog* p, const int32_t* ids, int S, int32_t* tok) {
    tlhip_tensor x, last, lastr, logits;
    if (t_new(2, S, p->hidden, 0, 0, &x)) return -1;
    CK(tlhip_embedding(C, p->emb, ids, S, x));
    for (int li = 0; li < p->n_layers; li++)
        if (layer_step(p, li, &x, S, 0, 0)) return -1;
    p->pos = S;
    if (t_new(1, p->hidden, 0, 0, 0, &last)) return -1;
    CK(tlhip_slice_last(C, x, 0, last));
    if (t_view(last, 2, 1, p->hidden, 0, 0, &lastr)) return -1;
    if (head(p, lastr, &logits)) return -1;
    CK(tlhip_argmax(C, logits, tok));   /* temperature_sample(logits, 0) */
    tlhip_tensor arr[] = {x, last, lastr, logits};
    for (size_t i = 0; i < sizeof arr / sizeof arr[0]; i++) tlhip_tensor_free(arr[i]);
    return 0;
}

static int decode(Prog* p, int32_t token, int32_t* tok, tlhip_tensor* logits_out) {
    tlhip_tensor x;
    if (p->pos >= p->max_ctx) {
        snprintf(g_err, sizeof g_err, "cache full");
        return -1;
    }
    const int off = p->rope_abs ? p->pos : 0;
    if (t_new(2, 1, p->hidden, 0, 0, &x)) return -1;
    CK(tlhip_embedding(C, p->emb, &token, 1, x));
    for (int li = 0; li < p->n_layers; li++)
        if (layer_step(p, li, &x, 1, off, 1)) return -1;
    p->pos++;
    if (head(p, x, logits_out)) return -1;
    CK(tlhip_argmax(C, *logits_out, tok));
    tlhip_tensor_free(x);
    return 0;
}

static int load(Prog* p, const char* path) {
    tlhip_gguf g;
    uint32_t u;
    CK(tlhip_gguf_open(path, &g));
    CK(tlhip_gguf_kv_u32(g, "llama.block_count", &u));
    p->n_layers = (int)u;
    CK(tlhip_gguf_kv_u32(g, "llama.embedding_length", &u));
    p->hidden = (int)u;
    CK(tlhip_gguf_kv_u32(g, "llama.attention.head_count", &u));
    p->n_heads = (int)u;
    CK(tlhip_gguf_kv_u32(g, "llama.attention.head_count_kv", &u));
    p->n_kv = (int)u;
    p->head_dim = p->hidden / p->n_heads;
    if (p->n_layers > 128) {
        snprintf(g_err, sizeof g_err, "more than 128 layers");
        return -1;
    }
    CK(tlhip_gguf_load_tensor(C, g, "token_embd.weight", &p->emb));
    CK(tlhip_gguf_load_tensor(C, g, "output_norm.weight", &p->out_norm));
    CK(tlhip_gguf_load_tensor(C, g, "output.weight", &p->out));
    static const char* names[9] = {"attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                   "ffn_norm", "ffn_gate", "ffn_up", "ffn_down"};
    for (int i = 0; i < p->n_layers; i++) {
        tlhip_tensor* dst[9] = {&p->L[i].attn_norm, &p->L[i].q, &p->L[i].k, &p->L[i].v, &p->L[i].o,
                                &p->L[i].ffn_norm, &p->L[i].gate, &p->L[i].up, &p->L[i].down};
        for (int k = 0; k < 9; k++) {
            char nm[96];
            snprintf(nm, sizeof nm, "blk.%d.%s.weight", i, names[k]);
            CK(tlhip_gguf_load_tensor(C, g, nm, dst[k]));
        }
    }
    CK(tlhip_gguf_close(g));
    int64_t shp[8];
    tlhip_dtype dt;
    int nd;
    CK(tlhip_tensor_info(p->emb, &dt, &nd, shp));
    p->vocab = (int)shp[0];
    return 0;
}

static void unload(Prog* p) {
    tlhip_tensor_free(p->emb);
    tlhip_tensor_free(p->out_norm);
    tlhip_tensor_free(p->out);
    for (int i = 0; i < p->n_layers; i++) {
        Layer* L = &p->L[i];
        tlhip_tensor arr[] = {L->attn_norm, L->q, L->k, L->v, L->o, L->ffn_norm, L->gate, L->up, L->down};
        for (int k = 0; k < 9; k++) tlhip_tensor_free(arr[k]);
    }
    if (p->cache) tlhip_kvcache_free(p->cache);
}

/* Prefill `prompt`, then warmup + steps greedy decode steps; tokens[0 ..
 * 1 + warmup + steps) receives the chosen ids, logits (vocab f16 values,
 * when not NULL) the last decode step's logits; ms[0] = prefill wall ms,
 * ms[1] = mean wall ms per timed decode step (ending with a device sync).
 * rope_abs = 0 keeps the program's literal semantics (decode rows rotated as
 * position 0).  Returns 0, or -1 with the message in obo_error(). */
int obo_run(const char* path, const int32_t* prompt, int n_prompt, int warmup, int steps, int max_ctx,
            int rope_abs, float eps, float scale, int32_t* tokens, uint16_t* logits, double* ms) {
    static Prog P;
    memset(&P, 0, sizeof P);
    Prog* p = &P;
    g_err[0] = 0;
    p->max_ctx = max_ctx;
    p->rope_abs = rope_abs;
    p->eps = eps;
    p->scale = scale;
    CK(tlhip_init(0, &C));
    int rc = load(p, path);
    if (!rc) {
        tlhip_status s = tlhip_kvcache_create(C, p->n_layers, max_ctx, p->n_kv, p->head_dim, &p->cache);
        if (s != TLHIP_OK) {
            snprintf(g_err, sizeof g_err, "kvcache_create: %s", tlhip_last_error());
            rc = -1;
        }
    }
    int32_t tok = 0;
    double t0 = now_ms();
    if (!rc) rc = prefill(p, prompt, n_prompt, &tok);
    ms[0] = now_ms() - t0;
    tokens[0] = tok;
    tlhip_tensor lg = NULL;
    for (int i = 0; !rc && i < warmup; i++) {
        rc = decode(p, tok, &tok, &lg);
        tokens[1 + i] = tok;
        if (lg) tlhip_tensor_free(lg);
        lg = NULL;
    }
    if (!rc && tlhip_sync(C) != TLHIP_OK) rc = -1;
    t0 = now_ms();
    for (int i = 0; !rc && i < steps; i++) {
        if (lg) tlhip_tensor_free(lg);
        lg = NULL;
        rc = decode(p, tok, &tok, &lg);
        tokens[1 + warmup + i] = tok;
    }
    if (!rc && tlhip_sync(C) != TLHIP_OK) rc = -1;
    ms[1] = steps > 0 ? (now_ms() - t0) / steps : 0.0;
    if (!rc && logits && lg && tlhip_tensor_download(C, lg, logits, (size_t)p->vocab * 2) != TLHIP_OK) {
        snprintf(g_err, sizeof g_err, "download logits: %s", tlhip_last_error());
        rc = -1;
    }
    if (lg) tlhip_tensor_free(lg);
    unload(p);
    tlhip_shutdown(C);
    return rc;
}

const char* obo_error(void) { return g_err; }

/* Config-3 elementwise legs timed from C (no Python between the calls):
 * rms_norm over [S, 2048] (eps 1e-5, w = 1 + small noise) and rope of the
 * query [S, 32, 64] and key [S, 4, 64] blocks, `iters` back-to-back calls of
 * each between hipEvents on the context stream; us[0] = us per rms_norm,
 * us[1] = us per query rope, us[2] = us per key rope.  Inputs are fixed
 * pseudo-random f16 bit patterns: x, q, k of magnitude in [0.25, 2), w in
 * [1, 1.04). */
static int upload_rand(int nd, int64_t a, int64_t b, int64_t c, uint32_t seed, int weight, tlhip_tensor* t) {
    int64_t n = a * (b ? b : 1) * (c ? c : 1);
    static uint16_t buf[2048 * 2048 * 2];
    if (n > (int64_t)(sizeof buf / 2)) {
        snprintf(g_err, sizeof g_err, "upload_rand: %lld elements", (long long)n);
        return -1;
    }
    uint32_t s = seed * 2654435761u + 1u;
    for (int64_t i = 0; i < n; i++) {
        s = s * 1664525u + 1013904223u;
        const uint32_t r = s >> 8;
        buf[i] = weight ? (uint16_t)(0x3C00u + r % 41u)
                        : (uint16_t)(((r & 1u) << 15) | ((13u + (r >> 1) % 3u) << 10) | ((r >> 3) & 0x3FFu));
    }
    if (t_new(nd, a, b, c, 0, t)) return -1;
    CK(tlhip_tensor_upload(C, *t, buf, (size_t)n * 2));
    return 0;
}

int obo_time_legs(int S, int iters, double* us) {
    tlhip_tensor x = NULL, w = NULL, y = NULL, q = NULL, k = NULL, qo = NULL, ko = NULL;
    g_err[0] = 0;
    CK(tlhip_init(0, &C));
    int rc = upload_rand(2, S, 2048, 0, 1, 0, &x);
    if (!rc) rc = upload_rand(1, 2048, 0, 0, 2, 1, &w);
    if (!rc) rc = upload_rand(3, S, 32, 64, 3, 0, &q);
    if (!rc) rc = upload_rand(3, S, 4, 64, 4, 0, &k);
    if (!rc) rc = t_new(2, S, 2048, 0, 0, &y);
    if (!rc) rc = t_new(3, S, 32, 64, 0, &qo);
    if (!rc) rc = t_new(3, S, 4, 64, 0, &ko);
    for (int leg = 0; !rc && leg < 3; leg++) {
        for (int pass = 0; !rc && pass < 2; pass++) {   /* warm-up pass, then the timed one */
            const int n = pass ? iters : 8;
            if (pass && tlhip_timer_start(C) != TLHIP_OK) rc = -1;
            for (int i = 0; !rc && i < n; i++) {
                tlhip_status st = leg == 0 ? tlhip_rms_norm(C, x, w, 1e-5f, y)
                                  : leg == 1 ? tlhip_rope(C, q, 0, 10000.0f, TLHIP_ROPE_INTERLEAVED, 0, qo)
                                             : tlhip_rope(C, k, 0, 10000.0f, TLHIP_ROPE_INTERLEAVED, 0, ko);
                if (st != TLHIP_OK) rc = -1;
            }
            float ms = 0.0f;
            if (!rc && pass && tlhip_timer_stop(C, &ms) != TLHIP_OK) rc = -1;
            if (!rc && pass) us[leg] = ms * 1000.0 / n;
        }
    }
    if (rc && !g_err[0]) snprintf(g_err, sizeof g_err, "%s", tlhip_last_error());
    tlhip_tensor arr[] = {x, w, y, q, k, qo, ko};
    for (size_t i = 0; i < sizeof arr / sizeof arr[0]; i++)
        if (arr[i]) tlhip_tensor_free(arr[i]);
    tlhip_shutdown(C);
    return rc;
}
