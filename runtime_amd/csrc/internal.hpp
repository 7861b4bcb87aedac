// Internal types of the HIP backend: context, buffers, pooled device memory.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <initializer_list>
#include <map>
#include <memory>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/minifield_hip.h"

namespace mfh {

// Packed stream formats (crates/kernels-simd/src/lib.rs:87-108).
enum class Format : int { Ternary = 0, Nf4 = 1, Int8 = 2 };

__host__ __device__ constexpr int weights_per_byte(Format f)
{
    return f == Format::Ternary ? 4 : f == Format::Nf4 ? 2 : 1;
}

// Error carrier: the status plus a static message, like ExecutorError's
// `&'static str` payloads.
struct Error {
    mfh_status status;
    const char *message;
};

// Size-bucketed caching allocator over hipMalloc.  All device work of a
// context runs on one stream, so a block released by the host can be handed
// to the next allocation immediately: any later use is stream-ordered after
// every use already queued.  Every block it holds, handed out or idle, counts
// as the context's device footprint (`reserved`).
class Pool {
public:
    explicit Pool(int device) : device_(device) {}
    ~Pool();
    // An idle block of bucket(bytes) .. 1.25 x that, or null.
    void *take(size_t bytes, size_t *capacity);
    // A new block of bucket(bytes) from the driver, or null.
    void *grow(size_t bytes, size_t *capacity);
    void release(void *ptr, size_t capacity);
    // Return every idle block to the driver.  The caller first makes sure no
    // queued work still uses them.
    void evict_idle();
    size_t reserved() const { return reserved_; }
    size_t idle() const { return idle_; }

private:
    int device_;
    size_t reserved_ = 0;
    size_t idle_ = 0;
    std::multimap<size_t, void *> free_;
    std::unordered_set<void *> all_;
};

size_t pool_bucket(size_t bytes);

}  // namespace mfh

struct mfh_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    mfh_backend_identity identity{};
    mfh_limits limits{};
    // Logical device bytes held per allocation class: each live buffer's
    // byte extent plus the sizes of its backend-private derived copies
    // (binary16 shadow, repacked tiles, tiled scales), charged to the
    // buffer's class.  The rest of the pool's reserve (bucket slack, context
    // scratch, idle pooled blocks) counts as scratch.
    uint64_t held_by_class[4] = {0, 0, 0, 0};
    // The logical bytes charged for each pool block a buffer holds (its own
    // storage or a derived copy), uncharged when the block is released.
    std::unordered_map<void *, uint64_t> charged;
    uint64_t peak_bytes = 0;
    uint64_t pending_result_bytes = 0;
    uint32_t pending_operations = 0;
    bool cancel_requested = false;
    const char *last_error = "no error";
    int kernel_path = 0;
    // Prefill GEMM activations: 0 = binary16 hi + lo halves, 1 = one half.
    int gemm_activations = 0;
    int cu_count = 256;
    std::unique_ptr<mfh::Pool> pool;
    // Small device scratch for staged host token ids and per-call partials;
    // reused in stream order.
    void *ids_scratch = nullptr;
    size_t ids_scratch_capacity = 0;
    void *work_scratch = nullptr;
    size_t work_scratch_capacity = 0;
    void *digits_scratch = nullptr;
    size_t digits_scratch_capacity = 0;
    // This device's address of the allocation-free entry point's fixed
    // scratch array (noalloc.hip), looked up at mfh_create; null if the
    // lookup failed.
    void *noalloc_scratch = nullptr;
    // Live handles, orphaned (their ctx pointer cleared) when the context is
    // destroyed first, so a late release or free stays safe.
    std::unordered_set<mfh_buf *> live_buffers;
    std::unordered_set<mfh_fence *> live_fences;
    std::unordered_set<mfh_readback *> live_readbacks;
};

struct mfh_buf {
    mfh_ctx *ctx = nullptr;
    uint64_t generation = 0;
    mfh_dtype dtype = MFH_DTYPE_F32;
    uint32_t rank = 0;
    uint64_t dims[4] = {0, 0, 0, 0};
    uint64_t elements = 0;
    uint64_t bytes = 0;
    mfh_alloc_class cls = MFH_CLASS_SCRATCH;
    void *dev = nullptr;
    size_t capacity = 0;  // device bytes of `dev` (the pool block)
    // U8 streams: whether any byte equals 0x80 (the reserved INT8 code),
    // scanned once at upload (backend-cpu/src/packed.rs:205 scans per call).
    bool has_int8_reserved = false;
    // F32 uploads whose every value is exactly representable in binary16 keep
    // a binary16 copy; packed kernels read scales from it.  Any write to the
    // buffer by an operation drops it.
    void *f16_shadow = nullptr;
    size_t f16_capacity = 0;
    // Backend-private repacked copy of a U8 code stream for one format, built
    // by prepare_packed (mfh_prepare_packed, or the first packed operation
    // that fixes the format).
    void *repacked = nullptr;
    size_t repacked_capacity = 0;
    int repacked_format = -1;
    // F32 scale streams: the scales in tile order for one format's padding,
    // built with the repacked codes; dropped when the buffer is written.
    void *tiled_scales = nullptr;
    size_t tiled_capacity = 0;
    int tiled_format = -1;
    bool tiled_half = false;
};

struct mfh_fence {
    mfh_ctx *ctx = nullptr;
    hipEvent_t event = nullptr;
    bool cancelled = false;
    bool consumed = false;
};

struct mfh_readback {
    mfh_ctx *ctx = nullptr;
    hipEvent_t event = nullptr;
    float *host = nullptr;
    size_t count = 0;
    bool consumed = false;
    bool cancelled = false;
};

namespace mfh {

// Record an error on the context and return its status.
mfh_status fail(mfh_ctx *ctx, mfh_status status, const char *message);
inline mfh_status fail(mfh_ctx *ctx, const Error &e) { return fail(ctx, e.status, e.message); }

// Buffer admission (backend-cpu/src/storage.rs:295-375, minus the per-call
// finite scan, which deferred device backends do not perform).
mfh_status check_buffer(mfh_ctx *ctx, const mfh_buf *buf);
mfh_status check_f32(mfh_ctx *ctx, const mfh_buf *buf);
mfh_status check_u8(mfh_ctx *ctx, const mfh_buf *buf);
mfh_status check_output(mfh_ctx *ctx, const mfh_buf *buf, const uint64_t *dims, uint32_t rank);
mfh_status check_operation(mfh_ctx *ctx, mfh_operation op);

// Drop derived copies of a buffer whose contents an operation overwrites.
void mark_written(mfh_buf *buf);

// Make the context's device current for the scope of one call.  When it
// already is (the common case: one device per process), the call costs one
// hipGetDevice and nothing is restored.
struct DeviceGuard {
    int previous = -1;
    explicit DeviceGuard(int device)
    {
        int current = device;
        (void)hipGetDevice(&current);
        if (current != device) {
            previous = current;
            (void)hipSetDevice(device);
        }
    }
    ~DeviceGuard()
    {
        if (previous >= 0)
            (void)hipSetDevice(previous);
    }
};

inline bool same_shape(const mfh_buf *a, const mfh_buf *b)
{
    if (!a || !b || a->rank != b->rank)
        return false;
    for (uint32_t i = 0; i < a->rank; ++i)
        if (a->dims[i] != b->dims[i])
            return false;
    return true;
}

// Whether `out` shares storage with any of `inputs` (null entries skipped).
inline bool aliases(const mfh_buf *out, std::initializer_list<const mfh_buf *> inputs)
{
    for (const mfh_buf *in : inputs)
        if (in && out->dev && in->dev == out->dev)
            return true;
    return false;
}

// Device memory for the context: an idle pool block, else a new one when the
// context's footprint (every pooled block plus pending readback staging)
// stays within max_total_bytes, after returning idle blocks to the driver
// if that makes room.  On failure records the reason and returns
// MFH_RESOURCE_LIMIT; nothing is allocated.
mfh_status acquire(mfh_ctx *ctx, size_t bytes, void **out, size_t *capacity);
// The same for a derived copy of `owner`, charged to the owner's class.
mfh_status acquire_for(mfh_ctx *ctx, mfh_buf *owner, size_t bytes, void **out, size_t *capacity);
// Return a block (null is ignored); `owner` non-null uncharges its class.
void release_block(mfh_ctx *ctx, mfh_buf *owner, void *ptr, size_t capacity);

// Device scratch owned by the context, grown on demand (stream ordered).
// Null when the allocation is refused; acquire() recorded why, and
// allocation_failed() is the status to return.
void *ids_scratch(mfh_ctx *ctx, size_t bytes);
void *work_scratch(mfh_ctx *ctx, size_t bytes);
void *digits_scratch(mfh_ctx *ctx, size_t bytes);
inline mfh_status allocation_failed(mfh_ctx *) { return MFH_RESOURCE_LIMIT; }

// An F32 rank-2 buffer of binary16 file values: the 2-byte values are
// uploaded into the buffer's binary16 shadow and decoded to f32 on the
// device (exact; the loader's f16 -> f32 rule).  The caller has checked that
// every value is finite.
mfh_status upload_scales_f16(mfh_ctx *ctx, const uint64_t *dims, const uint16_t *bits,
                             size_t count, mfh_alloc_class cls, mfh_buf **out);

// The device address of the allocation-free scratch array on `device`
// (which must be current), looked up once per device.
mfh_status noalloc_scratch(int device, void **out);

// Build (once, stream ordered) the tile-order copies the matrix-core
// kernels read for the format the two streams' widths select: repacked
// codes on `codes`, tiled scales on `scales`.  Admits the pair like every
// packed operation.
mfh_status prepare_packed(mfh_ctx *ctx, const mfh_buf *codes, const mfh_buf *scales);

// Fill `count` floats with `value` on the context stream (a kernel, so the
// call is capturable; no hipMemsetAsync).
void launch_fill_f32(hipStream_t stream, float *dst, size_t count, float value);

}  // namespace mfh
