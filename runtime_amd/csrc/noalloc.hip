// packed_linear for decode batches without any device allocation.
//
// mfh_packed_linear_noalloc runs the same matrix-core GEMV as
// mfh_packed_linear for m <= 8, but its activation-fragment scratch is a
// fixed array in this library's device image instead of a block from the
// context's pool, and it refuses weights whose private tile copies do not
// exist yet rather than building them.  So the call performs no hipMalloc,
// hipFree or allocating library call: it serves callers that must not
// allocate (code under stream capture, serving loops, harnesses that forbid
// it).
//
// Each GPU holds one copy of the array for the life of the process, and every
// call on that GPU uses it: calls whose work overlaps on one GPU (two
// contexts' streams, or host threads) race on it.  Every byte a call's
// kernels read from it is written earlier in the same call's stream order,
// so no clearing is needed between calls.
#include <mutex>

#include "internal.hpp"
#include "kernels.hpp"

namespace mfh {
namespace {

// Widest K served: the fragments take k_pad * 32 bytes (two 4-row integer
// fragments, or one binary16 hi/lo NF4 fragment pair), plus 8 factors and 8
// correction pairs per 128-group (gemv_mfma_scratch_bytes).
constexpr uint32_t kNoAllocMaxK = 16384;
constexpr size_t kNoAllocScratchBytes =
    size_t(kNoAllocMaxK) * 32 + size_t(8) * (kNoAllocMaxK / 128) * sizeof(float) +
    size_t(8) * (kNoAllocMaxK / 128) * 4 * sizeof(int);

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_lock;
void *g_address[kMaxDevices] = {};

}  // namespace

// The device address of this GPU's copy of `scratch`, looked up once per
// device with that device current (the caller's DeviceGuard).  The array's
// name is only a host-side stand-in; kernels must be given this address.
mfh_status noalloc_scratch(int device, void **out)
{
    if (device < 0 || device >= kMaxDevices)
        return MFH_UNSUPPORTED;
    std::lock_guard<std::mutex> hold(g_lock);
    if (!g_address[device]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
            (void)hipGetLastError();
            return MFH_BACKEND_FAILURE;
        }
        g_address[device] = ptr;
    }
    *out = g_address[device];
    return MFH_OK;
}

}  // namespace mfh

using namespace mfh;

extern "C" {

mfh_status mfh_packed_linear_noalloc(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                                     const mfh_buf *codes, const mfh_buf *scales)
{
    PackedCall call;
    mfh_status s = admit_packed_linear(ctx, output, input, codes, scales, &call);
    if (s)
        return s;
    if (call.m > 8 || ctx->kernel_path == 1)
        return fail(ctx, MFH_UNSUPPORTED,
                    "allocation-free packed linear serves at most 8 rows on the matrix-core GEMV");
    if (call.k > kNoAllocMaxK)
        return fail(ctx, MFH_RESOURCE_LIMIT,
                    "packed linear input width exceeds the allocation-free scratch limit");
    if (!prepared_stream(codes, scales, call.format, &call.a))
        return fail(ctx, MFH_UNSUPPORTED,
                    "allocation-free packed linear needs weights prepared by mfh_prepare_packed");
    if (!ctx->noalloc_scratch)
        return fail(ctx, MFH_BACKEND_FAILURE, "allocation-free scratch is unavailable");
    if (gemv_mfma_scratch_bytes(call) > kNoAllocScratchBytes)
        return fail(ctx, MFH_RESOURCE_LIMIT,
                    "packed linear input width exceeds the allocation-free scratch limit");
    DeviceGuard guard(ctx->device);
    // Drops only derived copies of the output (pool blocks return to the
    // pool; nothing is freed).
    mark_written(output);
    if (call.m == 0 || call.n == 0)
        return MFH_OK;
    if (call.k == 0) {
        launch_fill_f32(ctx->stream, call.out_a, size_t(call.m) * call.n, 0.0f);
    } else {
        call.separate_prologue = ctx->kernel_path == 2;
        launch_gemv_mfma(ctx->stream, call, ctx->noalloc_scratch);
    }
    if (hipGetLastError() != hipSuccess)
        return fail(ctx, MFH_BACKEND_FAILURE, "packed kernel launch failed");
    return MFH_OK;
}

}  // extern "C"
