// noalloc.hip -- tlhip_linear_noalloc: linear(x, W[, b]) that allocates
// nothing, for callers that cannot call hipMalloc (code under HIP graph
// capture, tight serving loops, harnesses that forbid allocation).
//
// tlhip_linear takes the split-K partials of its MFMA GEMM from the
// stream-ordered pool.  This variant takes them from `scratch`, a file-scope
// device array of kScratchBytes that each GPU holds from the library's load
// until the process ends.  Its device address is resolved once per device by
// noalloc_setup (called from tlhip_init with that device current) and kept
// per device; host code only ever passes that address, never the array's
// name, to kernels.
//
// The split is the one tlhip_linear picks (gemm_splits), so both entry points
// run the same kernels and produce the same bits.  Every partial a reduction
// reads is written by the GEMM of the same call (each slice covers every
// output element of its tiles), so the contents a previous call left behind
// never matter and nothing is cleared.  The skinny GEMM's arrival counters
// live in the context (allocated by tlhip_init) and every launch leaves them
// at zero.  All calls on one GPU share the array:
// calls that overlap in time on one GPU (two contexts' streams, two host
// threads) race on it and must be serialised by the caller.
#include <mutex>

#include "internal.hpp"

namespace {

// Largest split-K partial set gemm_splits can ask for (GEMM_SPLIT_PARTIALS_MAX,
// 20 MiB: M > 64 keeps at most 320 tiles of 128 x 128 over all slices, e.g.
// Q4_0 [512 x 10240] @ [2560 x 10240]^T in 4 slices; the skinny GEMM's
// splits stay within 16 MiB).
constexpr size_t kScratchBytes = tlhip::GEMM_SPLIT_PARTIALS_MAX;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_mu;
float* g_scratch_dev[kMaxDevices] = {};

}  // namespace

namespace tlhip {

tlhip_status noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices)
        return fail(TLHIP_ERR_DEVICE, "device %d beyond the %d the library tracks", device, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_scratch_dev[device]) return TLHIP_OK;
    int prev = -1;
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    // the symbol's address is per device: resolve it with that device current
    if (prev != device && hipSetDevice(device) != hipSuccess)
        return fail(TLHIP_ERR_DEVICE, "linear_noalloc: cannot make device %d current", device);
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
    if (e != hipSuccess || !ptr) {
        (void)hipGetLastError();
        return fail(TLHIP_ERR_DEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    }
    g_scratch_dev[device] = (float*)ptr;
    return TLHIP_OK;
}

}  // namespace tlhip

extern "C" tlhip_status tlhip_linear_noalloc(tlhip_ctx ctx, tlhip_tensor x, tlhip_tensor w, tlhip_tensor bias,
                                             tlhip_tensor y) try {
    using namespace tlhip;
    TLHIP_TRY(check_ctx(ctx));
    float* ws = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (ctx->device >= 0 && ctx->device < kMaxDevices) ws = g_scratch_dev[ctx->device];
    }
    if (!ws) {   // tlhip_init could not resolve it: once more, here, or report why not
        TLHIP_TRY(noalloc_setup(ctx->device));
        std::lock_guard<std::mutex> lk(g_mu);
        ws = g_scratch_dev[ctx->device];
    }
    return linear_impl(ctx, x, w, bias, y, ws, kScratchBytes);
} TLHIP_CATCH_STATUS
