// runtime.cpp -- context, errors, tensors and the stream-ordered pool.
//
// Replaces the reference's Metal device singleton (src/device/metal_device.rs
// :9-74), its per-thread command batching (commands.rs:44-200) and its
// size-class buffer pool (buffer_pool.rs:104-660): one HIP stream per context,
// allocations from the device's default memory pool via hipMallocAsync on
// that stream, frees stream-ordered via hipFreeAsync.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <mutex>
#include <new>

#include "internal.hpp"

namespace tlhip {

// The last error of the calling thread.  A fixed buffer, so that recording
// an error allocates nothing (it is also what reports a failed host
// allocation).
static thread_local char g_last_error[1280];

void set_error(tlhip_status st, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    static const char* names[] = {"OK", "ShapeMismatch", "InvalidDimension", "InvalidOperation",
                                  "AllocationError", "IndexOutOfBounds", "LoadError",
                                  "DeviceError", "DtypeError", "InvalidArgument"};
    const char* nm = (st >= 0 && st <= 9) ? names[st] : "Error";
    snprintf(g_last_error, sizeof g_last_error, "%s: %s", nm, buf);
}

tlhip_status fail(tlhip_status st, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    set_error(st, "%s", buf);
    return st;
}

// The exception barrier of the C ABI (every exported function ends in
// TLHIP_CATCH_STATUS or an equivalent handler): an exception thrown by host
// code -- std::bad_alloc from a container, anything else -- becomes a status
// and a message instead of unwinding through extern "C" into the caller.
tlhip_status abi_exception() noexcept {
    try {
        throw;
    } catch (const std::bad_alloc&) {
        return fail(TLHIP_ERR_ALLOCATION, "host memory allocation failed (std::bad_alloc)");
    } catch (const std::exception& e) {
        return fail(TLHIP_ERR_INVALID_OPERATION, "internal error: %s", e.what());
    } catch (...) {
        return fail(TLHIP_ERR_INVALID_OPERATION, "internal error: unknown exception");
    }
}

size_t payload_bytes(tlhip_dtype d, const int64_t* shape, int ndim) {
    int64_t n = 1;
    for (int i = 0; i < ndim; i++) n *= shape[i];
    switch (d) {
        case TLHIP_F16: return (size_t)n * 2;
        case TLHIP_F32: return (size_t)n * 4;
        case TLHIP_I32: return (size_t)n * 4;
        case TLHIP_Q4_0: return (size_t)n / 32 * 18;
        case TLHIP_Q8_0: return (size_t)n / 32 * 34;
        case TLHIP_Q6_K: return (size_t)n / 256 * 210;
    }
    return 0;
}

std::string shape_str(const tlhip_tensor_s* t) {
    std::string s = "[";
    for (int i = 0; i < t->ndim; i++) {
        if (i) s += ", ";
        s += std::to_string(t->shape[i]);
    }
    return s + "]";
}

static std::mutex g_ctx_mu;

tlhip_status check_ctx(tlhip_ctx ctx) {
    if (!ctx || !ctx->stream) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null context");
    return TLHIP_OK;
}

void ctx_release(tlhip_ctx ctx) {
    {
        std::lock_guard<std::mutex> lk(g_ctx_mu);
        if (--ctx->refs > 0) return;
    }
    (void)hipSetDevice(ctx->device);
    for (auto& kv : ctx->block_cache)
        for (void* b : kv.second) (void)hipFreeAsync(b, ctx->stream);
    ctx->block_cache.clear();
    (void)hipStreamSynchronize(ctx->stream);
    for (auto& r : ctx->rope_tables) (void)hipFree(r.dev);
    (void)hipFree(ctx->d_scratch_i32);
    (void)hipFree(ctx->d_tile_flags);
    if (ctx->d_ws) {
        (void)hipFreeAsync(ctx->d_ws, ctx->stream);
        (void)hipStreamSynchronize(ctx->stream);
    }
    (void)hipHostFree(ctx->h_pinned_i32);
    (void)hipEventDestroy(ctx->ev0);
    (void)hipEventDestroy(ctx->ev1);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

static void ctx_retain(tlhip_ctx ctx) {
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    ctx->refs++;
}

tlhip_status check_t(tlhip_tensor t, const char* what) {
    if (!t || !t->data) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null tensor (%s)", what);
    return TLHIP_OK;
}

tlhip_status check_dtype(tlhip_tensor t, tlhip_dtype d, const char* op) {
    if (t->dtype != d)
        return fail(TLHIP_ERR_DTYPE, "%s: unsupported dtype %d (expected %d)", op, (int)t->dtype,
                    (int)d);
    return TLHIP_OK;
}

tlhip_status after_launch(tlhip_ctx ctx, const char* op) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TLHIP_ERR_DEVICE, "%s launch failed: %s", op, hipGetErrorString(e));
    if (ctx->sync_every_op) {
        e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return fail(TLHIP_ERR_DEVICE, "%s failed: %s", op, hipGetErrorString(e));
    }
    return TLHIP_OK;
}

// The context's block cache: a tensor's block is rounded up to its size
// class -- a quarter power of two, at most 25 % over, from 256 bytes -- and
// blocks of freed tensors up to kCacheBlockMax are kept (up to kCacheCap per
// context) for the next allocation of that class.  A hipMallocAsync /
// hipFreeAsync pair costs ~7.7 us of host time on MI355X, ~3x a small
// kernel's launch, and an interpreter that calls the library one builtin at
// a time allocates an output per call.
constexpr size_t kCacheBlockMax = (size_t)32 << 20;
constexpr size_t kCacheCap = (size_t)512 << 20;

static size_t block_class(size_t n) {
    if (n <= 256) return 256;
    const int k = 63 - __builtin_clzll((unsigned long long)n);   // 2^k <= n < 2^(k+1)
    const size_t step = (size_t)1 << (k - 2);
    return (n + step - 1) / step * step;
}

tlhip_status alloc_tensor(tlhip_ctx ctx, tlhip_dtype dtype, int ndim, const int64_t* shape,
                          tlhip_tensor* out) {
    TLHIP_TRY(check_ctx(ctx));
    if (!out) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null output handle");
    *out = nullptr;
    if (ndim < 1 || ndim > 8 || !shape)
        return fail(TLHIP_ERR_INVALID_DIMENSION, "rank %d not in 1..8", ndim);
    for (int i = 0; i < ndim; i++)
        if (shape[i] < 0) return fail(TLHIP_ERR_INVALID_DIMENSION, "negative dim %lld", (long long)shape[i]);
    if ((int)dtype < 0 || (int)dtype > 5) return fail(TLHIP_ERR_INVALID_ARGUMENT, "bad dtype %d", (int)dtype);
    size_t bytes = payload_bytes(dtype, shape, ndim);
    size_t qs_bytes = 0;
    if (is_quant(dtype)) {
        if (ndim != 2 || shape[1] % quant_group(dtype) != 0)
            return fail(TLHIP_ERR_INVALID_DIMENSION, "quantized tensors must be 2-D [N, K] with K %% %d == 0",
                        (int)quant_group(dtype));
        qs_bytes = quant_data_bytes(dtype, shape[0], shape[1]);
        bytes = qs_bytes + (size_t)quant_scale_count(dtype, shape[0], shape[1]) * 2;
    }
    auto* t = new tlhip_tensor_s();
    t->ctx = ctx;
    t->dtype = dtype;
    t->ndim = ndim;
    for (int i = 0; i < ndim; i++) t->shape[i] = shape[i];
    size_t abytes = bytes ? bytes : 256;
    if (abytes <= kCacheBlockMax) {
        abytes = block_class(abytes);
        std::lock_guard<std::mutex> lk(ctx->cache_mu);
        auto it = ctx->block_cache.find(abytes);
        if (it != ctx->block_cache.end() && !it->second.empty()) {
            t->data = it->second.back();
            it->second.pop_back();
            ctx->cached_bytes -= abytes;
        }
    }
    if (!t->data) {
        hipError_t e = hipMallocAsync(&t->data, abytes, ctx->stream);
        if (e != hipSuccess) {
            delete t;
            (void)hipGetLastError();
            return fail(TLHIP_ERR_ALLOCATION, "hipMallocAsync(%zu) failed: %s", abytes, hipGetErrorString(e));
        }
    }
    t->alloc_bytes = abytes;
    if (is_quant(dtype)) t->scales = (uint16_t*)((uint8_t*)t->data + qs_bytes);
    ctx_retain(ctx);
    *out = t;
    return TLHIP_OK;
}

static std::mutex g_rope_mu;

tlhip_status rope_table(tlhip_ctx ctx, float theta, int rot_dims, int need_pos, const float** dev) {
    std::lock_guard<std::mutex> lk(g_rope_mu);
    RopeTable* rt = nullptr;
    for (auto& r : ctx->rope_tables)
        if (r.theta == theta && r.rot_dims == rot_dims) rt = &r;
    if (rt && rt->max_pos >= need_pos) {
        *dev = rt->dev;
        return TLHIP_OK;
    }
    int maxp = 4096;
    while (maxp < need_pos) maxp *= 2;
    const int half = rot_dims / 2;
    // The reference's frequency formula (rope_f16, unified.metal:2355-2418):
    // freq_i = 1 / pow(theta, 2i / D) in f32, angle = f32(pos) * freq_i.
    // cos/sin of that f32 angle are evaluated in double and rounded to f32.
    std::vector<float> h((size_t)maxp * half * 2);
    for (int i = 0; i < half; i++) {
        float expo = (float)(2 * i) / (float)rot_dims;
        float freq = 1.0f / powf(theta, expo);
        for (int p = 0; p < maxp; p++) {
            volatile float ang = (float)p * freq;
            h[2 * ((size_t)p * half + i) + 0] = (float)std::cos((double)ang);
            h[2 * ((size_t)p * half + i) + 1] = (float)std::sin((double)ang);
        }
    }
    float* d = nullptr;
    TLHIP_CHECK_HIP(hipMalloc(&d, h.size() * sizeof(float)));
    TLHIP_CHECK_HIP(hipMemcpy(d, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
    if (rt) {
        // Old table may still be read by queued work: free after the stream drains.
        TLHIP_CHECK_HIP(hipStreamSynchronize(ctx->stream));
        TLHIP_CHECK_HIP(hipFree(rt->dev));
        rt->dev = d;
        rt->max_pos = maxp;
    } else {
        RopeTable r;
        r.theta = theta;
        r.rot_dims = rot_dims;
        r.max_pos = maxp;
        r.dev = d;
        ctx->rope_tables.push_back(r);
    }
    *dev = d;
    return TLHIP_OK;
}

}  // namespace tlhip

using namespace tlhip;

extern "C" {

const char* tlhip_last_error(void) { return g_last_error; }

tlhip_status tlhip_init(int device, tlhip_ctx* out) try {
    if (!out) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null output");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
        return fail(TLHIP_ERR_DEVICE, "no HIP device available (%s)", hipGetErrorString(e));
    if (device < 0) device = 0;
    if (device >= n) return fail(TLHIP_ERR_DEVICE, "device %d out of range (%d devices)", device, n);
    TLHIP_CHECK_HIP(hipSetDevice(device));
    // the no-allocation entry point's workspace address on this device; a
    // failure here concerns only that entry point, which resolves it again
    // on its first call and reports the error there
    if (noalloc_setup(device) != TLHIP_OK) (void)hipGetLastError();
    auto* c = new tlhip_ctx_s();
    c->device = device;
    hipError_t e1 = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e1 != hipSuccess) {
        delete c;
        return fail(TLHIP_ERR_DEVICE, "hipStreamCreate failed: %s", hipGetErrorString(e1));
    }
    TLHIP_CHECK_HIP(hipEventCreate(&c->ev0));
    TLHIP_CHECK_HIP(hipEventCreate(&c->ev1));
    TLHIP_CHECK_HIP(hipMalloc(&c->d_scratch_i32, 256 * sizeof(int32_t)));
    TLHIP_CHECK_HIP(hipMalloc(&c->d_tile_flags, CTX_FLAG_WORDS * sizeof(uint32_t)));
    // (on the context's own stream, which does not wait for the null stream)
    TLHIP_CHECK_HIP(hipMemsetAsync(c->d_tile_flags, 0, CTX_FLAG_WORDS * sizeof(uint32_t), c->stream));
    TLHIP_CHECK_HIP(hipStreamSynchronize(c->stream));
    TLHIP_CHECK_HIP(hipHostMalloc(&c->h_pinned_i32, 256 * sizeof(int32_t), hipHostMallocDefault));
    // Keep freed pool memory cached in the pool instead of returning it to
    // the driver at every synchronisation.
    hipMemPool_t pool;
    if (hipDeviceGetDefaultMemPool(&pool, device) == hipSuccess) {
        uint64_t thr = UINT64_MAX;
        (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &thr);
    }
    const char* env = getenv("TLHIP_SYNC_EVERY_OP");
    c->sync_every_op = env && env[0] == '1';
    *out = c;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_shutdown(tlhip_ctx ctx) try {
    TLHIP_TRY(check_ctx(ctx));
    // releases the caller's reference; tensors still alive keep the stream
    ctx_release(ctx);
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_sync(tlhip_ctx ctx) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_CHECK_HIP(hipStreamSynchronize(ctx->stream));
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_device_name(tlhip_ctx ctx, char* buf, size_t len) try {
    TLHIP_TRY(check_ctx(ctx));
    if (!buf || !len) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null buffer");
    hipDeviceProp_t p;
    TLHIP_CHECK_HIP(hipGetDeviceProperties(&p, ctx->device));
    snprintf(buf, len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_set_sync_every_op(tlhip_ctx ctx, int on) try {
    TLHIP_TRY(check_ctx(ctx));
    ctx->sync_every_op = on != 0;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_tensor_alloc(tlhip_ctx ctx, tlhip_dtype dtype, int ndim, const int64_t* shape,
                                tlhip_tensor* out) try {
    return alloc_tensor(ctx, dtype, ndim, shape, out);
} TLHIP_CATCH_STATUS

size_t tlhip_tensor_nbytes(tlhip_tensor t) try {
    if (!t) return 0;
    return payload_bytes(t->dtype, t->shape, t->ndim);
} TLHIP_CATCH_VALUE(0)

tlhip_status tlhip_tensor_upload(tlhip_ctx ctx, tlhip_tensor t, const void* host, size_t bytes) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(check_t(t, "upload"));
    if (!host && bytes) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null host pointer");
    size_t need = tlhip_tensor_nbytes(t);
    if (bytes != need)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "upload of %zu bytes into a tensor of %zu bytes", bytes, need);
    if (!bytes) return TLHIP_OK;
    if (!is_quant(t->dtype)) {
        TLHIP_CHECK_HIP(hipMemcpyAsync(t->data, host, bytes, hipMemcpyHostToDevice, ctx->stream));
        TLHIP_CHECK_HIP(hipStreamSynchronize(ctx->stream));
        return TLHIP_OK;
    }
    // new contents: a dequantised copy made from the old ones is stale
    if (t->f16_copy) {
        tlhip_tensor_free(t->f16_copy);
        t->f16_copy = nullptr;
    }
    // Packed GGUF blocks -> staging -> structure-of-arrays repack on device.
    void* stage = nullptr;
    TLHIP_CHECK_HIP(hipMallocAsync(&stage, bytes, ctx->stream));
    TLHIP_CHECK_HIP(hipMemcpyAsync(stage, host, bytes, hipMemcpyHostToDevice, ctx->stream));
    int64_t N = t->shape[0], K = t->shape[1];
    tlhip_status st = launch_repack_rows(ctx->stream, t->dtype, (const uint8_t*)stage, t->data, t->scales,
                                         N, K, N, 0, 1, 0);
    (void)hipFreeAsync(stage, ctx->stream);
    TLHIP_TRY(st);
    TLHIP_TRY(after_launch(ctx, "upload/repack"));
    TLHIP_CHECK_HIP(hipStreamSynchronize(ctx->stream));
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_tensor_download(tlhip_ctx ctx, tlhip_tensor t, void* host, size_t bytes) try {
    TLHIP_TRY(check_ctx(ctx));
    TLHIP_TRY(check_t(t, "download"));
    size_t need = tlhip_tensor_nbytes(t);
    if (bytes != need)
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "download of %zu bytes from a tensor of %zu bytes", bytes, need);
    if (!host && bytes) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null host pointer");
    if (!bytes) return TLHIP_OK;
    if (!is_quant(t->dtype)) {
        TLHIP_CHECK_HIP(hipMemcpyAsync(host, t->data, bytes, hipMemcpyDeviceToHost, ctx->stream));
        TLHIP_CHECK_HIP(hipStreamSynchronize(ctx->stream));
        return TLHIP_OK;
    }
    void* stage = nullptr;
    TLHIP_CHECK_HIP(hipMallocAsync(&stage, bytes, ctx->stream));
    int64_t N = t->shape[0], K = t->shape[1];
    tlhip_status st = launch_repack_rows(ctx->stream, t->dtype, (uint8_t*)stage, t->data, t->scales,
                                         N, K, N, 0, 1, 1);
    if (st == TLHIP_OK) {
        hipError_t e = hipMemcpyAsync(host, stage, bytes, hipMemcpyDeviceToHost, ctx->stream);
        if (e != hipSuccess) st = fail(TLHIP_ERR_DEVICE, "hipMemcpyAsync: %s", hipGetErrorString(e));
    }
    (void)hipFreeAsync(stage, ctx->stream);
    TLHIP_CHECK_HIP(hipStreamSynchronize(ctx->stream));
    return st;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_tensor_retain(tlhip_tensor t) try {
    if (!t) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null tensor");
    t->refcount++;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_tensor_free(tlhip_tensor t) try {
    if (!t) return TLHIP_OK;
    if (--t->refcount > 0) return TLHIP_OK;
    if (t->base) {
        tlhip_tensor_free(t->base);
    } else if (t->data) {
        if (t->f16_copy) tlhip_tensor_free(t->f16_copy);
        tlhip_ctx c = t->ctx;
        bool kept = false;
        if (t->alloc_bytes <= kCacheBlockMax) {
            std::lock_guard<std::mutex> lk(c->cache_mu);
            if (c->cached_bytes + t->alloc_bytes <= kCacheCap) {
                c->block_cache[t->alloc_bytes].push_back(t->data);
                c->cached_bytes += t->alloc_bytes;
                kept = true;
            }
        }
        if (!kept) {
            (void)hipSetDevice(c->device);
            (void)hipFreeAsync(t->data, c->stream);
        }
        ctx_release(c);
    }
    delete t;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_tensor_info(tlhip_tensor t, tlhip_dtype* dtype, int* ndim, int64_t* shape) try {
    if (!t) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null tensor");
    if (dtype) *dtype = t->dtype;
    if (ndim) *ndim = t->ndim;
    if (shape)
        for (int i = 0; i < t->ndim; i++) shape[i] = t->shape[i];
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

tlhip_status tlhip_tensor_reshape(tlhip_tensor t, int ndim, const int64_t* shape, tlhip_tensor* out) try {
    TLHIP_TRY(check_t(t, "reshape"));
    if (!out || !shape) return fail(TLHIP_ERR_INVALID_ARGUMENT, "null argument");
    if (is_quant(t->dtype)) return fail(TLHIP_ERR_INVALID_OPERATION, "reshape of a quantized tensor");
    if (ndim < 1 || ndim > 8) return fail(TLHIP_ERR_INVALID_DIMENSION, "rank %d", ndim);
    int64_t n = 1;
    for (int i = 0; i < ndim; i++) {
        if (shape[i] < 0) return fail(TLHIP_ERR_INVALID_DIMENSION, "negative dim");
        n *= shape[i];
    }
    if (n != numel(t))
        return fail(TLHIP_ERR_SHAPE_MISMATCH, "reshape %s -> %lld elements", shape_str(t).c_str(),
                    (long long)n);
    auto* v = new tlhip_tensor_s();
    *v = *t;
    v->refcount = 1;
    v->f16_copy = nullptr;
    v->ndim = ndim;
    for (int i = 0; i < 8; i++) v->shape[i] = i < ndim ? shape[i] : 0;
    tlhip_tensor owner = t->base ? t->base : t;
    owner->refcount++;
    v->base = owner;
    *out = v;
    return TLHIP_OK;
} TLHIP_CATCH_STATUS

}  // extern "C"
