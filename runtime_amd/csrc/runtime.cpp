// Context lifetime, buffer storage and accounting, completions.
//
// Mirrors the reference's backend storage contract
// (crates/backend-cpu/src/storage.rs, crates/engine-api/src/resources.rs,
// crates/engine-api/src/inference.rs:39-111) on one HIP stream per context.
#include <cstdlib>
#include <cstring>
#include <new>

#include "internal.hpp"
#include "kernels.hpp"
#include "../../include/minifield_convert.h"

namespace mfh {

size_t pool_bucket(size_t bytes)
{
    // 256-byte granularity up to 1 MiB, then 1/8-octave buckets so a
    // released block serves requests of nearly the same size.
    if (bytes == 0)
        return 256;
    if (bytes <= (1u << 20))
        return (bytes + 255) & ~size_t(255);
    size_t top = size_t(1) << (63 - __builtin_clzll(bytes));
    size_t step = top / 8;
    return (bytes + step - 1) / step * step;
}

Pool::~Pool()
{
    int previous = 0;
    (void)hipGetDevice(&previous);
    (void)hipSetDevice(device_);
    for (void *p : all_)
        (void)hipFree(p);
    (void)hipSetDevice(previous);
}

void *Pool::take(size_t bytes, size_t *capacity)
{
    const size_t want = pool_bucket(bytes);
    auto it = free_.lower_bound(want);
    // Reuse a block up to 25% larger than needed.
    if (it == free_.end() || it->first > want + want / 4)
        return nullptr;
    void *p = it->second;
    *capacity = it->first;
    idle_ -= it->first;
    free_.erase(it);
    return p;
}

void *Pool::grow(size_t bytes, size_t *capacity)
{
    const size_t want = pool_bucket(bytes);
    void *p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    all_.insert(p);
    reserved_ += want;
    *capacity = want;
    return p;
}

void Pool::release(void *ptr, size_t capacity)
{
    if (!ptr)
        return;
    free_.emplace(capacity, ptr);
    idle_ += capacity;
}

void Pool::evict_idle()
{
    for (auto &entry : free_) {
        (void)hipFree(entry.second);
        all_.erase(entry.second);
        reserved_ -= entry.first;
    }
    free_.clear();
    idle_ = 0;
}

namespace {

void note_peak(mfh_ctx *ctx)
{
    const uint64_t total = ctx->pool->reserved() + ctx->pending_result_bytes;
    if (total > ctx->peak_bytes)
        ctx->peak_bytes = total;
}

// Return the idle blocks to the driver once the stream has drained (a block
// the host released may still be read by queued work).
void evict(mfh_ctx *ctx)
{
    if (!ctx->pool->idle())
        return;
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipGetLastError();
    ctx->pool->evict_idle();
}

}  // namespace

mfh_status acquire(mfh_ctx *ctx, size_t bytes, void **out, size_t *capacity)
{
    *out = ctx->pool->take(bytes, capacity);
    if (*out)
        return MFH_OK;
    // resources.rs:27-43 on the physical footprint: every pooled block, idle
    // ones included, plus pending readback staging.
    const uint64_t want = pool_bucket(bytes);
    const uint64_t limit = ctx->limits.max_total_bytes;
    auto fits = [&] {
        const uint64_t owned = ctx->pool->reserved() + ctx->pending_result_bytes;
        return owned + want >= owned && owned + want <= limit;
    };
    if (!fits())
        evict(ctx);
    if (!fits())
        return fail(ctx, MFH_RESOURCE_LIMIT, "allocation exceeds configured total resource limit");
    *out = ctx->pool->grow(bytes, capacity);
    if (!*out) {
        evict(ctx);
        *out = ctx->pool->grow(bytes, capacity);
    }
    if (!*out)
        return fail(ctx, MFH_RESOURCE_LIMIT, "device allocation failed");
    note_peak(ctx);
    return MFH_OK;
}

mfh_status acquire_for(mfh_ctx *ctx, mfh_buf *owner, size_t bytes, void **out, size_t *capacity)
{
    mfh_status s = acquire(ctx, bytes, out, capacity);
    if (!s) {
        ctx->held_by_class[owner->cls] += bytes;
        ctx->charged[*out] = bytes;
    }
    return s;
}

void release_block(mfh_ctx *ctx, mfh_buf *owner, void *ptr, size_t capacity)
{
    if (!ptr)
        return;
    if (owner) {
        auto it = ctx->charged.find(ptr);
        if (it != ctx->charged.end()) {
            ctx->held_by_class[owner->cls] -= it->second;
            ctx->charged.erase(it);
        }
    }
    ctx->pool->release(ptr, capacity);
}

mfh_status fail(mfh_ctx *ctx, mfh_status status, const char *message)
{
    if (ctx)
        ctx->last_error = message;
    return status;
}

mfh_status check_buffer(mfh_ctx *ctx, const mfh_buf *buf)
{
    if (!buf)
        return fail(ctx, MFH_INVALID_ARGUMENT, "buffer handle is null");
    if (buf->ctx != ctx)
        return fail(ctx, MFH_WRONG_BACKEND, "buffer belongs to another backend");
    if (buf->generation != ctx->identity.generation)
        return fail(ctx, MFH_STALE_BUFFER, "buffer belongs to an earlier backend generation");
    return MFH_OK;
}

mfh_status check_f32(mfh_ctx *ctx, const mfh_buf *buf)
{
    mfh_status s = check_buffer(ctx, buf);
    if (s)
        return s;
    if (buf->dtype != MFH_DTYPE_F32)
        return fail(ctx, MFH_INVALID_DTYPE, "expected an f32 operand");
    return MFH_OK;
}

mfh_status check_u8(mfh_ctx *ctx, const mfh_buf *buf)
{
    mfh_status s = check_buffer(ctx, buf);
    if (s)
        return s;
    if (buf->dtype != MFH_DTYPE_U8)
        return fail(ctx, MFH_INVALID_DTYPE, "expected a u8 operand");
    return MFH_OK;
}

// check_output_shape, backend-cpu/src/storage.rs:363-375.
mfh_status check_output(mfh_ctx *ctx, const mfh_buf *buf, const uint64_t *dims, uint32_t rank)
{
    mfh_status s = check_f32(ctx, buf);
    if (s)
        return s;
    bool same = buf->rank == rank;
    for (uint32_t i = 0; same && i < rank; ++i)
        same = buf->dims[i] == dims[i];
    if (!same)
        return fail(ctx, MFH_INVALID_SHAPE, "output layout differs from required contiguous shape");
    return MFH_OK;
}

// check_operation, backend-cpu/src/storage.rs:284-293.
mfh_status check_operation(mfh_ctx *ctx, mfh_operation op)
{
    (void)op;  // every OperationKind this ABI exposes is implemented
    if (ctx->cancel_requested)
        return fail(ctx, MFH_CANCELLED, "operation cancelled");
    return MFH_OK;
}

void mark_written(mfh_buf *buf)
{
    mfh_ctx *ctx = buf->ctx;
    if (buf->f16_shadow) {
        release_block(ctx, buf, buf->f16_shadow, buf->f16_capacity);
        buf->f16_shadow = nullptr;
        buf->f16_capacity = 0;
    }
    if (buf->tiled_scales) {
        release_block(ctx, buf, buf->tiled_scales, buf->tiled_capacity);
        buf->tiled_scales = nullptr;
        buf->tiled_capacity = 0;
        buf->tiled_format = -1;
    }
}

// Scratch blocks only grow; a replaced block returns to the pool, where
// stream order keeps it from being reused before the work queued on it ran.
static void *grow(mfh_ctx *ctx, void **slot, size_t *capacity, size_t bytes)
{
    if (bytes > *capacity) {
        size_t want = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
        void *p = nullptr;
        size_t got = 0;
        if (acquire(ctx, want, &p, &got))
            return nullptr;
        release_block(ctx, nullptr, *slot, *capacity);
        *slot = p;
        *capacity = got;
    }
    return *slot;
}

void *ids_scratch(mfh_ctx *ctx, size_t bytes)
{
    return grow(ctx, &ctx->ids_scratch, &ctx->ids_scratch_capacity, bytes);
}

void *work_scratch(mfh_ctx *ctx, size_t bytes)
{
    return grow(ctx, &ctx->work_scratch, &ctx->work_scratch_capacity, bytes);
}

void *digits_scratch(mfh_ctx *ctx, size_t bytes)
{
    return grow(ctx, &ctx->digits_scratch, &ctx->digits_scratch_capacity, bytes);
}

}  // namespace mfh

using namespace mfh;

namespace {

const uint64_t kOperations = (1ull << MFH_OP_COPY) | (1ull << MFH_OP_RECT_COPY_2D) |
                             (1ull << MFH_OP_GATHER_ROWS) | (1ull << MFH_OP_ADD) |
                             (1ull << MFH_OP_MULTIPLY) | (1ull << MFH_OP_LINEAR) |
                             (1ull << MFH_OP_ROW_RMS_NORM) | (1ull << MFH_OP_ROTARY) |
                             (1ull << MFH_OP_GROUPED_QUERY_ATTENTION) |
                             (1ull << MFH_OP_GATED_SHORT_CONVOLUTION) |
                             (1ull << MFH_OP_SWIGLU) | (1ull << MFH_OP_PACKED_GATHER_ROWS) |
                             (1ull << MFH_OP_PACKED_LINEAR) | (1ull << MFH_OP_ADD_ROW_RMS_NORM) |
                             (1ull << MFH_OP_PACKED_LINEAR_PAIR) |
                             (1ull << MFH_OP_PACKED_SWIGLU_LINEAR) |
                             (1ull << MFH_OP_PACKED_SWIGLU_PAIR) | (1ull << MFH_OP_QK_NORM_ROPE) |
                             (1ull << MFH_OP_ARGMAX) | (1ull << MFH_OP_GATHER_COLUMNS);

// Shape admission shared by the allocation entry points: rank <= 4, element
// count and byte size without overflow, capability and limit checks
// (storage.rs:381-420, backend.rs:397-431, resources.rs:27-43).
mfh_status admit_shape(mfh_ctx *ctx, const uint64_t *dims, uint32_t rank, size_t elem,
                       uint64_t *elements, uint64_t *bytes)
{
    if (rank > 4)
        return fail(ctx, MFH_INVALID_SHAPE, "rank exceeds portable descriptor limit");
    if (rank > 0 && !dims)
        return fail(ctx, MFH_INVALID_ARGUMENT, "dims pointer is null");
    uint64_t count = 1;
    for (uint32_t i = 0; i < rank; ++i) {
        if (dims[i] != 0 && count > UINT64_MAX / dims[i])
            return fail(ctx, MFH_OVERFLOW, "element count overflows u64");
        count *= dims[i];
    }
    if (count > UINT64_MAX / elem)
        return fail(ctx, MFH_OVERFLOW, "byte extent overflows u64");
    uint64_t b = count * elem;
    if (count > ctx->limits.max_total_bytes / 4)
        return fail(ctx, MFH_RESOURCE_LIMIT, "element count exceeds backend capability");
    if (b > ctx->limits.max_allocation_bytes)
        return fail(ctx, MFH_RESOURCE_LIMIT, "allocation exceeds configured per-buffer limit");
    *elements = count;
    *bytes = b;
    return MFH_OK;
}

mfh_status make_buffer(mfh_ctx *ctx, const uint64_t *dims, uint32_t rank, mfh_dtype dtype,
                       mfh_alloc_class cls, mfh_buf **out)
{
    if (!out)
        return fail(ctx, MFH_INVALID_ARGUMENT, "output handle pointer is null");
    *out = nullptr;
    if (ctx->cancel_requested)
        return fail(ctx, MFH_CANCELLED, "operation cancelled");
    if (cls < MFH_CLASS_WEIGHT || cls > MFH_CLASS_BRANCH)
        return fail(ctx, MFH_INVALID_ARGUMENT, "unknown allocation class");
    uint64_t elements = 0, bytes = 0;
    mfh_status s = admit_shape(ctx, dims, rank, dtype == MFH_DTYPE_F32 ? 4 : 1, &elements, &bytes);
    if (s)
        return s;
    auto *buf = new (std::nothrow) mfh_buf();
    if (!buf)
        return fail(ctx, MFH_RESOURCE_LIMIT, "host allocation failed");
    buf->ctx = ctx;
    buf->generation = ctx->identity.generation;
    buf->dtype = dtype;
    buf->rank = rank;
    for (uint32_t i = 0; i < rank; ++i)
        buf->dims[i] = dims[i];
    buf->elements = elements;
    buf->bytes = bytes;
    buf->cls = cls;
    if (bytes > 0) {
        if (acquire(ctx, bytes, &buf->dev, &buf->capacity)) {
            delete buf;
            return MFH_RESOURCE_LIMIT;
        }
    }
    ctx->live_buffers.insert(buf);
    if (buf->dev) {
        ctx->held_by_class[cls] += bytes;
        ctx->charged[buf->dev] = bytes;
    }
    *out = buf;
    return MFH_OK;
}

bool f16_exact(float v, uint16_t *h)
{
    // Exact when binary16 round-trips the value bit for bit.
    uint16_t bits = mfc_f32_to_f16(v);
    float back = mfc_f16_to_f32(bits);
    uint32_t a, b;
    std::memcpy(&a, &v, 4);
    std::memcpy(&b, &back, 4);
    *h = bits;
    return a == b;
}

}  // namespace

extern "C" {

const char *mfh_status_message(mfh_status status)
{
    switch (status) {
    case MFH_OK: return "ok";
    case MFH_INVALID_ARGUMENT: return "invalid argument";
    case MFH_INVALID_SHAPE: return "invalid shape";
    case MFH_INVALID_LAYOUT: return "invalid layout";
    case MFH_INVALID_DTYPE: return "invalid dtype";
    case MFH_OVERFLOW: return "overflow";
    case MFH_OUT_OF_BOUNDS: return "out of bounds";
    case MFH_UNSUPPORTED: return "unsupported";
    case MFH_RESOURCE_LIMIT: return "resource limit";
    case MFH_WRONG_BACKEND: return "buffer belongs to another backend";
    case MFH_STALE_BUFFER: return "buffer belongs to an earlier backend generation";
    case MFH_DUPLICATE_NAME: return "duplicate name";
    case MFH_MISSING_REQUIRED_TENSOR: return "required tensor is missing";
    case MFH_UNEXPECTED_TENSOR: return "undeclared tensor is present";
    case MFH_INVALID_TIE: return "invalid tied tensor declaration";
    case MFH_CANCELLED: return "operation cancelled";
    case MFH_COMPLETION_CONSUMED: return "completion result was already consumed";
    case MFH_BACKEND_FAILURE: return "backend failure";
    }
    return "unknown status";
}

mfh_status mfh_create(uint32_t ordinal, uint64_t owner, const mfh_limits *limits, mfh_ctx **out)
{
    if (!out || !limits)
        return MFH_INVALID_ARGUMENT;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
        (void)hipGetLastError();
        return MFH_UNSUPPORTED;
    }
    if (ordinal >= uint32_t(count))
        return MFH_OUT_OF_BOUNDS;
    auto *ctx = new (std::nothrow) mfh_ctx();
    if (!ctx)
        return MFH_RESOURCE_LIMIT;
    ctx->device = int(ordinal);
    DeviceGuard guard(ctx->device);
    // Default priority, non-blocking with respect to the legacy null stream.
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return MFH_BACKEND_FAILURE;
    }
    hipDeviceProp_t props;
    if (hipGetDeviceProperties(&props, ctx->device) == hipSuccess)
        ctx->cu_count = props.multiProcessorCount;
    ctx->identity.kind = MFH_BACKEND_KIND_HIP;
    ctx->identity.ordinal = ordinal;
    ctx->identity.owner = owner;
    ctx->identity.generation = 1;
    ctx->limits = *limits;
    ctx->pool.reset(new mfh::Pool(ctx->device));
    if (noalloc_scratch(ctx->device, &ctx->noalloc_scratch))
        ctx->noalloc_scratch = nullptr;
    *out = ctx;
    return MFH_OK;
}

void mfh_destroy(mfh_ctx *ctx)
{
    if (!ctx)
        return;
    {
        DeviceGuard guard(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        // Orphan every handle still alive: its memory goes with the pool and
        // its later release/free only deletes the host-side record.
        for (mfh_buf *buf : ctx->live_buffers) {
            buf->ctx = nullptr;
            buf->dev = buf->f16_shadow = buf->repacked = buf->tiled_scales = nullptr;
        }
        for (mfh_fence *fence : ctx->live_fences) {
            (void)hipEventDestroy(fence->event);
            fence->event = nullptr;
            fence->ctx = nullptr;
        }
        for (mfh_readback *rb : ctx->live_readbacks) {
            (void)hipEventDestroy(rb->event);
            if (rb->host)
                (void)hipHostFree(rb->host);
            rb->event = nullptr;
            rb->host = nullptr;
            rb->ctx = nullptr;
        }
        ctx->pool.reset();
        (void)hipStreamDestroy(ctx->stream);
    }
    delete ctx;
}

const char *mfh_last_error(const mfh_ctx *ctx) { return ctx ? ctx->last_error : "null context"; }

mfh_status mfh_identity(const mfh_ctx *ctx, mfh_backend_identity *out)
{
    if (!ctx || !out)
        return MFH_INVALID_ARGUMENT;
    *out = ctx->identity;
    return MFH_OK;
}

mfh_status mfh_capabilities(const mfh_ctx *ctx, mfh_backend_capabilities *out)
{
    if (!ctx || !out)
        return MFH_INVALID_ARGUMENT;
    out->dtypes = (1u << MFH_DTYPE_F32) | (1u << MFH_DTYPE_U8);
    out->operations = kOperations;
    out->max_rank = 4;
    out->max_elements = ctx->limits.max_total_bytes / 4;
    out->max_allocation_bytes = ctx->limits.max_allocation_bytes;
    out->supports_nonblocking_completion = 1;
    return MFH_OK;
}

mfh_status mfh_resource_report(const mfh_ctx *ctx, mfh_report *out)
{
    if (!ctx || !out)
        return MFH_INVALID_ARGUMENT;
    // Every pooled device byte is reported once: the logical bytes of live
    // buffers and their derived copies under the buffer's class, everything
    // else the pool holds (bucket slack, context scratch, idle blocks) as
    // scratch, as backend-wgpu/src/lib.rs:340-370 charges byte extents per
    // class and the physical remainder as scratch.  The total is the
    // context's device footprint plus pending readback staging.
    const uint64_t *held = ctx->held_by_class;
    const uint64_t attributed = held[0] + held[1] + held[2] + held[3];
    out->resident_weight_bytes = held[MFH_CLASS_WEIGHT];
    out->cache_bytes = held[MFH_CLASS_CACHE];
    out->scratch_bytes = held[MFH_CLASS_SCRATCH] + (ctx->pool->reserved() - attributed);
    out->staged_branch_bytes = held[MFH_CLASS_BRANCH];
    out->pending_operation_bytes = ctx->pending_result_bytes;
    out->pending_operations = ctx->pending_operations;
    return MFH_OK;
}

mfh_status mfh_peak_accounted_bytes(const mfh_ctx *ctx, uint64_t *out)
{
    if (!ctx || !out)
        return MFH_INVALID_ARGUMENT;
    *out = ctx->peak_bytes;
    return MFH_OK;
}

mfh_status mfh_advance_generation(mfh_ctx *ctx)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    if (ctx->identity.generation == UINT64_MAX)
        return fail(ctx, MFH_OVERFLOW, "backend generation overflows u64");
    ctx->identity.generation += 1;
    ctx->cancel_requested = false;
    return MFH_OK;
}

mfh_status mfh_request_cancel(mfh_ctx *ctx)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    ctx->cancel_requested = true;
    return MFH_OK;
}

mfh_status mfh_clear_cancel(mfh_ctx *ctx)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    ctx->cancel_requested = false;
    return MFH_OK;
}

mfh_status mfh_poll_retired_fences(mfh_ctx *ctx)
{
    // Fences own their HIP events and free them on mfh_fence_free; nothing
    // is retained behind an abandoned fence, so there is nothing to retire.
    return ctx ? MFH_OK : MFH_INVALID_ARGUMENT;
}

mfh_status mfh_alloc_f32(mfh_ctx *ctx, const uint64_t *dims, uint32_t rank, mfh_alloc_class cls,
                         int zeroed, mfh_buf **out)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    mfh_status s = make_buffer(ctx, dims, rank, MFH_DTYPE_F32, cls, out);
    if (s)
        return s;
    // Weight and Cache classes are always zeroed (executor/storage.rs:8-18).
    if ((zeroed || cls == MFH_CLASS_WEIGHT || cls == MFH_CLASS_CACHE) && (*out)->elements)
        launch_fill_f32(ctx->stream, static_cast<float *>((*out)->dev), (*out)->elements, 0.0f);
    return MFH_OK;
}

mfh_status mfh_upload_f32(mfh_ctx *ctx, const uint64_t *dims, uint32_t rank, const float *values,
                          size_t count, mfh_alloc_class cls, mfh_buf **out)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    mfh_status s = make_buffer(ctx, dims, rank, MFH_DTYPE_F32, cls, out);
    if (s)
        return s;
    mfh_buf *buf = *out;
    if (count != buf->elements || (count && !values)) {
        mfh_release(buf);
        *out = nullptr;
        return fail(ctx, MFH_INVALID_SHAPE, "upload length differs from shape element count");
    }
    if (!count)
        return MFH_OK;
    if (hipMemcpyAsync(buf->dev, values, buf->bytes, hipMemcpyHostToDevice, ctx->stream) !=
        hipSuccess) {
        (void)hipGetLastError();
        mfh_release(buf);
        *out = nullptr;
        return fail(ctx, MFH_BACKEND_FAILURE, "host to device copy failed");
    }
    // Rank-2 uploads whose values all round-trip through binary16 (packed
    // scale streams decoded from F16 files) also get a binary16 copy.
    if (rank == 2) {
        std::vector<uint16_t> half(count);
        bool exact = true;
        for (size_t i = 0; i < count && exact; ++i)
            exact = f16_exact(values[i], &half[i]);
        if (exact) {
            // The shadow is optional: where the limit leaves no room for it
            // the kernels read the f32 scales.
            if (acquire_for(ctx, buf, count * 2, &buf->f16_shadow, &buf->f16_capacity))
                buf->f16_shadow = nullptr;
            if (buf->f16_shadow &&
                hipMemcpyAsync(buf->f16_shadow, half.data(), count * 2, hipMemcpyHostToDevice,
                               ctx->stream) != hipSuccess) {
                (void)hipGetLastError();
                release_block(ctx, buf, buf->f16_shadow, buf->f16_capacity);
                buf->f16_shadow = nullptr;
            }
        }
        if (hipStreamSynchronize(ctx->stream) != hipSuccess) {
            (void)hipGetLastError();
            return fail(ctx, MFH_BACKEND_FAILURE, "host to device copy failed");
        }
        return MFH_OK;
    }
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        return fail(ctx, MFH_BACKEND_FAILURE, "host to device copy failed");
    }
    return MFH_OK;
}

mfh_status mfh_upload_u8(mfh_ctx *ctx, const uint64_t *dims, uint32_t rank, const uint8_t *bytes,
                         size_t count, mfh_alloc_class cls, mfh_buf **out)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    mfh_status s = make_buffer(ctx, dims, rank, MFH_DTYPE_U8, cls, out);
    if (s)
        return s;
    mfh_buf *buf = *out;
    if (count != buf->elements || (count && !bytes)) {
        mfh_release(buf);
        *out = nullptr;
        return fail(ctx, MFH_INVALID_SHAPE, "upload length differs from shape element count");
    }
    if (!count)
        return MFH_OK;
    buf->has_int8_reserved = std::memchr(bytes, 0x80, count) != nullptr;
    if (hipMemcpyAsync(buf->dev, bytes, count, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        mfh_release(buf);
        *out = nullptr;
        return fail(ctx, MFH_BACKEND_FAILURE, "host to device copy failed");
    }
    return MFH_OK;
}

}  // extern "C"

namespace mfh {

mfh_status upload_scales_f16(mfh_ctx *ctx, const uint64_t *dims, const uint16_t *bits,
                             size_t count, mfh_alloc_class cls, mfh_buf **out)
{
    DeviceGuard guard(ctx->device);
    mfh_status s = make_buffer(ctx, dims, 2, MFH_DTYPE_F32, cls, out);
    if (s)
        return s;
    mfh_buf *buf = *out;
    if (count != buf->elements || (count && !bits)) {
        mfh_release(buf);
        *out = nullptr;
        return fail(ctx, MFH_INVALID_SHAPE, "upload length differs from shape element count");
    }
    if (!count)
        return MFH_OK;
    if ((s = acquire_for(ctx, buf, count * 2, &buf->f16_shadow, &buf->f16_capacity))) {
        buf->f16_shadow = nullptr;
        mfh_release(buf);
        *out = nullptr;
        return s;
    }
    if (hipMemcpyAsync(buf->f16_shadow, bits, count * 2, hipMemcpyHostToDevice, ctx->stream) !=
        hipSuccess) {
        (void)hipGetLastError();
        mfh_release(buf);
        *out = nullptr;
        return fail(ctx, MFH_BACKEND_FAILURE, "host to device copy failed");
    }
    launch_f16_to_f32(ctx->stream, static_cast<float *>(buf->dev),
                      static_cast<const uint16_t *>(buf->f16_shadow), count);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        return fail(ctx, MFH_BACKEND_FAILURE, "host to device copy failed");
    }
    return MFH_OK;
}

}  // namespace mfh

extern "C" {

void mfh_release(mfh_buf *buf)
{
    if (!buf)
        return;
    mfh_ctx *ctx = buf->ctx;
    if (ctx) {
        release_block(ctx, buf, buf->dev, buf->capacity);
        release_block(ctx, buf, buf->f16_shadow, buf->f16_capacity);
        release_block(ctx, buf, buf->repacked, buf->repacked_capacity);
        release_block(ctx, buf, buf->tiled_scales, buf->tiled_capacity);
        ctx->live_buffers.erase(buf);
    }
    delete buf;
}

mfh_status mfh_buf_desc(const mfh_buf *buf, mfh_dtype *dtype, uint32_t *rank, uint64_t *dims)
{
    if (!buf)
        return MFH_INVALID_ARGUMENT;
    if (dtype)
        *dtype = buf->dtype;
    if (rank)
        *rank = buf->rank;
    if (dims)
        for (uint32_t i = 0; i < buf->rank; ++i)
            dims[i] = buf->dims[i];
    return MFH_OK;
}

mfh_status mfh_fence_submit(mfh_ctx *ctx, mfh_fence **out)
{
    if (!ctx || !out)
        return MFH_INVALID_ARGUMENT;
    *out = nullptr;
    if (ctx->cancel_requested)
        return fail(ctx, MFH_CANCELLED, "operation cancelled");
    DeviceGuard guard(ctx->device);
    auto *fence = new (std::nothrow) mfh_fence();
    if (!fence)
        return fail(ctx, MFH_RESOURCE_LIMIT, "host allocation failed");
    fence->ctx = ctx;
    if (hipEventCreateWithFlags(&fence->event, hipEventDisableTiming) != hipSuccess ||
        hipEventRecord(fence->event, ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        if (fence->event)
            (void)hipEventDestroy(fence->event);
        delete fence;
        return fail(ctx, MFH_BACKEND_FAILURE, "fence submission failed");
    }
    ctx->live_fences.insert(fence);
    *out = fence;
    return MFH_OK;
}

mfh_status mfh_fence_poll(mfh_fence *fence, int *ready)
{
    if (!fence || !ready)
        return MFH_INVALID_ARGUMENT;
    *ready = 0;
    if (fence->cancelled) {
        *ready = 1;
        return MFH_CANCELLED;
    }
    if (fence->consumed) {
        *ready = 1;
        return MFH_COMPLETION_CONSUMED;
    }
    if (!fence->ctx) {
        *ready = 1;
        return MFH_WRONG_BACKEND;  // its backend was destroyed
    }
    DeviceGuard guard(fence->ctx->device);
    hipError_t e = hipEventQuery(fence->event);
    if (e == hipErrorNotReady)
        return MFH_OK;
    *ready = 1;
    fence->consumed = true;
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(fence->ctx, MFH_BACKEND_FAILURE, "device work failed before the fence");
    }
    return MFH_OK;
}

mfh_status mfh_fence_cancel(mfh_fence *fence)
{
    if (!fence)
        return MFH_INVALID_ARGUMENT;
    // The work is already submitted; cancellation only drops the result.
    fence->cancelled = true;
    return MFH_OK;
}

void mfh_fence_free(mfh_fence *fence)
{
    if (!fence)
        return;
    if (fence->ctx) {
        DeviceGuard guard(fence->ctx->device);
        (void)hipEventDestroy(fence->event);
        fence->ctx->live_fences.erase(fence);
    }
    delete fence;
}

mfh_status mfh_read_f32_async(mfh_ctx *ctx, const mfh_buf *buf, mfh_readback **out)
{
    if (!ctx || !out)
        return MFH_INVALID_ARGUMENT;
    *out = nullptr;
    if (ctx->cancel_requested)
        return fail(ctx, MFH_CANCELLED, "operation cancelled");
    mfh_status s = check_f32(ctx, buf);
    if (s)
        return s;
    DeviceGuard guard(ctx->device);
    // The staging the completion owns until it is polled counts against the
    // total limit like device blocks do.  As for a device allocation, the
    // idle pooled blocks are returned to the driver before a request that
    // does not fit is refused (backend-wgpu/src/device.rs:657-676 clears its
    // free pools before the budget check of readback staging).
    auto fits = [&] {
        const uint64_t owned = ctx->pool->reserved() + ctx->pending_result_bytes;
        return owned + buf->bytes >= owned && owned + buf->bytes <= ctx->limits.max_total_bytes;
    };
    if (!fits())
        evict(ctx);
    if (!fits())
        return fail(ctx, MFH_RESOURCE_LIMIT, "allocation exceeds configured total resource limit");
    auto *rb = new (std::nothrow) mfh_readback();
    if (!rb)
        return fail(ctx, MFH_RESOURCE_LIMIT, "host allocation failed");
    rb->ctx = ctx;
    rb->count = buf->elements;
    if (rb->count) {
        if (hipHostMalloc(reinterpret_cast<void **>(&rb->host), buf->bytes, hipHostMallocDefault) !=
            hipSuccess) {
            (void)hipGetLastError();
            delete rb;
            return fail(ctx, MFH_RESOURCE_LIMIT, "pinned readback allocation failed");
        }
        if (hipMemcpyAsync(rb->host, buf->dev, buf->bytes, hipMemcpyDeviceToHost, ctx->stream) !=
            hipSuccess) {
            (void)hipGetLastError();
            (void)hipHostFree(rb->host);
            delete rb;
            return fail(ctx, MFH_BACKEND_FAILURE, "device to host copy failed");
        }
    }
    if (hipEventCreateWithFlags(&rb->event, hipEventDisableTiming) != hipSuccess ||
        hipEventRecord(rb->event, ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipStreamSynchronize(ctx->stream);
        if (rb->host)
            (void)hipHostFree(rb->host);
        delete rb;
        return fail(ctx, MFH_BACKEND_FAILURE, "readback submission failed");
    }
    ctx->pending_result_bytes += buf->bytes;
    note_peak(ctx);
    ctx->live_readbacks.insert(rb);
    *out = rb;
    return MFH_OK;
}

mfh_status mfh_readback_poll(mfh_readback *rb, int *ready, float *dst, size_t capacity,
                             size_t *count)
{
    if (!rb || !ready)
        return MFH_INVALID_ARGUMENT;
    *ready = 0;
    if (rb->cancelled) {
        *ready = 1;
        return MFH_CANCELLED;
    }
    if (rb->consumed) {
        *ready = 1;
        return MFH_COMPLETION_CONSUMED;
    }
    if (!rb->ctx) {
        *ready = 1;
        return MFH_WRONG_BACKEND;  // its backend was destroyed
    }
    DeviceGuard guard(rb->ctx->device);
    hipError_t e = hipEventQuery(rb->event);
    if (e == hipErrorNotReady)
        return MFH_OK;
    *ready = 1;
    rb->consumed = true;
    rb->ctx->pending_result_bytes -= rb->count * 4;
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(rb->ctx, MFH_BACKEND_FAILURE, "device work failed before the readback");
    }
    size_t n = rb->count < capacity ? rb->count : capacity;
    if (n && dst)
        std::memcpy(dst, rb->host, n * 4);
    if (count)
        *count = rb->count;
    return MFH_OK;
}

mfh_status mfh_readback_cancel(mfh_readback *rb)
{
    if (!rb)
        return MFH_INVALID_ARGUMENT;
    rb->cancelled = true;
    return MFH_OK;
}

void mfh_readback_free(mfh_readback *rb)
{
    if (!rb)
        return;
    if (rb->ctx) {
        DeviceGuard guard(rb->ctx->device);
        // The copy may still be in flight: wait for it before freeing the
        // pinned destination.
        (void)hipEventSynchronize(rb->event);
        (void)hipEventDestroy(rb->event);
        if (rb->host)
            (void)hipHostFree(rb->host);
        if (!rb->consumed)
            rb->ctx->pending_result_bytes -= rb->count * 4;
        rb->ctx->live_readbacks.erase(rb);
    }
    delete rb;
}

mfh_status mfh_synchronize(mfh_ctx *ctx)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    DeviceGuard guard(ctx->device);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        return fail(ctx, MFH_BACKEND_FAILURE, "device work failed");
    }
    return MFH_OK;
}

void *mfh_stream(const mfh_ctx *ctx) { return ctx ? static_cast<void *>(ctx->stream) : nullptr; }

int mfh_set_kernel_path(mfh_ctx *ctx, int path)
{
    if (!ctx)
        return -1;
    int previous = ctx->kernel_path;
    ctx->kernel_path = path;
    return previous;
}

int mfh_set_gemm_activations(mfh_ctx *ctx, int mode)
{
    if (!ctx)
        return -1;
    int previous = ctx->gemm_activations;
    ctx->gemm_activations = mode == 1 ? 1 : 0;
    return previous;
}

int mfh_supports_ternary_lut2(const mfh_ctx *ctx)
{
    (void)ctx;
    return 0;
}

}  // extern "C"
