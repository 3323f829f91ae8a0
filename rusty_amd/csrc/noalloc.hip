// rq_mlp_swiglu_noalloc: the SwiGLU MLP of rq_mlp_swiglu with its fp16
// intermediate h in a file-scope device array instead of a caller workspace,
// for callers that cannot allocate device memory (code under HIP graph
// capture, serving loops that forbid hipMalloc).  The entry point allocates
// nothing and calls no allocating routine: the array exists once per device
// for the life of the process, and its device address is looked up once per
// device at context creation.
//
// Every call on one device shares that device's array, so calls that overlap
// on one device (two streams, two host threads) race on it.  Nothing in the
// array has to start at zero: the gate/up pass writes every h value the down
// projection reads.
#include <mutex>

#include "common.hpp"

// h of the no-alloc SwiGLU: 2*m*I fp16 values of at most kNoAllocScratchBytes.
// In host code `scratch` names a host-side stand-in, not device memory: host
// code uses only the per-device address from hipGetSymbolAddress.
static constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace rq {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];       // device address of `scratch`, per device
hipError_t g_scratch_err[kMaxDevices];  // the lookup's error, per device

}  // namespace

void noalloc_init(int device) {
    if (device < 0 || device >= kMaxDevices) return;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device]) return;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && p) {
        g_scratch_ptr[device] = p;
        g_scratch_err[device] = hipSuccess;
    } else {
        g_scratch_err[device] = e != hipSuccess ? e : hipErrorInvalidSymbol;
        (void)hipGetLastError();  // reported by the entry point, not left for the next call
    }
}

}  // namespace rq

using namespace rq;

extern "C" int rq_mlp_swiglu_noalloc(rq_ctx *ctx, const rq_qweight *gate, const rq_qweight *up,
                                     const rq_qweight *down, const void *x, rq_dtype x_dtype, void *y,
                                     rq_dtype y_dtype, int64_t m, rq_stream stream) {
    RQ_ENTER(ctx);
    int st = swiglu_check(gate, up, down, x_dtype, y_dtype, m);
    if (st != RQ_OK || m == 0 || gate->k_in == 0) return st;
    if (!y || !x) return fail(RQ_ERR_INVALID_ARGUMENT, "null activation pointer");
    const int64_t I = gate->n_out;
    // h = 2*m*I fp16 values; mul_ok bounds m*2I (swiglu_check)
    if ((uint64_t)m * (uint64_t)(2 * I) * 2u > kNoAllocScratchBytes)
        return fail(RQ_ERR_SHAPE, "m * intermediate = %lld * %lld needs %llu bytes of scratch; the no-alloc MLP has %zu "
                    "(m * intermediate <= %zu)", (long long)m, (long long)I,
                    (unsigned long long)((uint64_t)m * (uint64_t)(2 * I) * 2u), kNoAllocScratchBytes,
                    kNoAllocScratchBytes / 4);
    void *h = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (ctx->device >= 0 && ctx->device < kMaxDevices) h = g_scratch_ptr[ctx->device];
        if (!h)
            return fail(RQ_ERR_HIP, "device %d: the scratch array's address was not found at context creation (%s)",
                        ctx->device,
                        ctx->device >= 0 && ctx->device < kMaxDevices ? hipGetErrorString(g_scratch_err[ctx->device])
                                                                      : "device ordinal out of range");
    }
    // no workspace for any of its GEMMs (gate/up and down): the context's
    // split-K partials and preparation area are not shared with these calls
    const GemmWorkspace none{nullptr, nullptr, 0, 0};
    return swiglu_run(ctx, *gate, *up, *down, x, x_dtype, h, y, y_dtype, m, none, pick(ctx, stream));
}
