// Packed-weight operations: admission and kernel selection.
//
// Admission restates CpuBackend's checks in the reference's order and with
// its messages (crates/backend-cpu/src/packed.rs:11-466): every operand is
// validated before anything is enqueued, so a rejected call writes nothing.
#include <vector>

#include "internal.hpp"
#include "kernels.hpp"

namespace mfh {
namespace {

struct Packed {
    uint32_t rows = 0;
    uint32_t inner = 0;
    Format format = Format::Ternary;
};

// check_packed_operands, backend-cpu/src/packed.rs:177-220.
mfh_status check_packed(mfh_ctx *ctx, const mfh_buf *codes, const mfh_buf *scales, Packed *out)
{
    mfh_status s = check_u8(ctx, codes);
    if (!s)
        s = check_f32(ctx, scales);
    if (s)
        return s;
    if (codes->rank != 2 || scales->rank != 2)
        return fail(ctx, MFH_INVALID_SHAPE, "packed weight streams must be rank two");
    uint64_t code_width = codes->dims[1];
    uint64_t groups = scales->dims[1];
    if (groups > UINT64_MAX / 128)
        return fail(ctx, MFH_OVERFLOW, "packed inner width overflows usize");
    uint64_t inner = groups * 128;
    if (code_width == inner / 4) {
        out->format = Format::Ternary;
    } else if (code_width == inner / 2) {
        out->format = Format::Nf4;
    } else if (code_width == inner) {
        if (codes->has_int8_reserved)
            return fail(ctx, MFH_INVALID_ARGUMENT, "INT8 -128 code is reserved");
        out->format = Format::Int8;
    } else {
        return fail(ctx, MFH_INVALID_SHAPE,
                    "packed code width must be inner/4 (ternary), inner/2 (nf4), or inner (int8)");
    }
    if (scales->dims[0] != codes->dims[0])
        return fail(ctx, MFH_INVALID_SHAPE, "packed codes and scales disagree on row count");
    if (codes->dims[0] > UINT32_MAX || inner > UINT32_MAX)
        return fail(ctx, MFH_OVERFLOW, "packed stream exceeds the 32-bit kernel index range");
    out->rows = uint32_t(codes->dims[0]);
    out->inner = uint32_t(inner);
    return MFH_OK;
}

PackedStream stream_of(const mfh_buf *codes, const mfh_buf *scales)
{
    PackedStream s;
    s.codes = static_cast<const uint8_t *>(codes->dev);
    s.scales = static_cast<const float *>(scales->dev);
    s.scales16 = static_cast<const uint16_t *>(scales->f16_shadow);
    return s;
}

// Build (once) the tile-order copies the matrix-core kernels read: the
// repacked codes live on the code buffer, the tiled scales on the scale
// buffer, each charged to its buffer's allocation class and bounded by the
// context's limits.  Both are stream-ordered kernels; nothing synchronizes.
// Nothing is replaced unless both new copies could be allocated.
mfh_status prepare_tiles(mfh_ctx *ctx, const mfh_buf *codes_c, const mfh_buf *scales_c,
                         const Packed &p, PackedStream *stream)
{
    // Derived copies are caches on immutable inputs; the handles stay const
    // to callers.
    mfh_buf *codes = const_cast<mfh_buf *>(codes_c);
    mfh_buf *scales = const_cast<mfh_buf *>(scales_c);
    const int fmt = int(p.format);
    const bool half = scales->f16_shadow != nullptr;
    const bool need_codes = !codes->repacked || codes->repacked_format != fmt;
    const bool need_scales =
        !scales->tiled_scales || scales->tiled_format != fmt || scales->tiled_half != half;
    void *tiles = nullptr, *tiled = nullptr;
    size_t tiles_cap = 0, tiled_cap = 0;
    mfh_status s = MFH_OK;
    if (need_codes)
        s = acquire_for(ctx, codes, repacked_bytes(p.format, p.rows, p.inner), &tiles, &tiles_cap);
    if (!s && need_scales) {
        s = acquire_for(ctx, scales, tiled_scales_bytes(p.format, p.rows, p.inner, half), &tiled,
                        &tiled_cap);
        if (s)
            release_block(ctx, codes, tiles, tiles_cap);
    }
    if (s)
        return s;
    if (need_codes) {
        release_block(ctx, codes, codes->repacked, codes->repacked_capacity);
        codes->repacked = tiles;
        codes->repacked_capacity = tiles_cap;
        codes->repacked_format = fmt;
        launch_repack(ctx->stream, p.format, static_cast<const uint8_t *>(codes->dev),
                      static_cast<uint8_t *>(codes->repacked), p.rows, p.inner);
    }
    if (need_scales) {
        release_block(ctx, scales, scales->tiled_scales, scales->tiled_capacity);
        scales->tiled_scales = tiled;
        scales->tiled_capacity = tiled_cap;
        scales->tiled_format = fmt;
        scales->tiled_half = half;
        launch_tile_scales(ctx->stream, p.format, static_cast<const float *>(scales->dev),
                           scales->tiled_scales, p.rows, p.inner, half);
    }
    if ((need_codes || need_scales) && hipGetLastError() != hipSuccess)
        return fail(ctx, MFH_BACKEND_FAILURE, "packed kernel launch failed");
    if (stream) {
        stream->tiles = static_cast<const uint8_t *>(codes->repacked);
        stream->tiled_scales = scales->tiled_scales;
        stream->tiled_half = half;
    }
    return MFH_OK;
}

// Whether the matrix-core decode GEMV serves this call.
bool use_mfma_gemv(const mfh_ctx *ctx, const PackedCall &call)
{
    return call.m <= 8 && ctx->kernel_path != 1 && gemv_mfma_supported(call.format);
}

// Enqueue the kernels of one admitted packed product.  `a`/`b` are the
// weight operands (b only for two-stream calls).
mfh_status run_packed(mfh_ctx *ctx, PackedCall call, const mfh_buf *codes_a,
                      const mfh_buf *scales_a, const mfh_buf *codes_b = nullptr,
                      const mfh_buf *scales_b = nullptr)
{
    hipStream_t stream = ctx->stream;
    if (call.m == 0 || call.n == 0)
        return MFH_OK;
    if (call.k == 0) {
        // An empty contraction: every row dot is 0, silu(0) * 0 is 0.
        launch_fill_f32(stream, call.out_a, size_t(call.m) * call.n, 0.0f);
        if (call.epilogue == Epilogue::Pair)
            launch_fill_f32(stream, call.out_b, size_t(call.m) * call.n, 0.0f);
        return MFH_OK;
    }
    if (use_mfma_gemv(ctx, call)) {
        Packed p{call.n, call.k, call.format};
        mfh_status s = prepare_tiles(ctx, codes_a, scales_a, p, &call.a);
        if (!s && codes_b)
            s = prepare_tiles(ctx, codes_b, scales_b, p, &call.b);
        if (s)
            return s;
        void *scratch = digits_scratch(ctx, gemv_mfma_scratch_bytes(call));
        if (!scratch)
            return allocation_failed(ctx);
        call.separate_prologue = ctx->kernel_path == 2;
        launch_gemv_mfma(stream, call, scratch);
    } else if (call.m <= 8) {
        launch_gemv_fma(stream, call);
    } else if (ctx->kernel_path != 1) {
        // The GEMM reads the same repacked tiles as the decode GEMV.
        Packed p{call.n, call.k, call.format};
        mfh_status s = prepare_tiles(ctx, codes_a, scales_a, p, &call.a);
        if (!s && codes_b)
            s = prepare_tiles(ctx, codes_b, scales_b, p, &call.b);
        if (s)
            return s;
        void *scratch = digits_scratch(ctx, gemm_mfma_scratch_bytes(call));
        if (!scratch)
            return allocation_failed(ctx);
        call.single_half = ctx->gemm_activations == 1;
        launch_gemm_mfma(stream, call, scratch);
    } else {
        launch_gemm_fma(stream, call);
    }
    if (hipGetLastError() != hipSuccess)
        return fail(ctx, MFH_BACKEND_FAILURE, "packed kernel launch failed");
    return MFH_OK;
}

}  // namespace

mfh_status packed_xform(mfh_ctx *ctx, Epilogue epilogue, const XForm &xform, uint32_t m,
                        uint32_t n, uint32_t k, const mfh_buf *codes_a, const mfh_buf *scales_a,
                        const mfh_buf *codes_b, const mfh_buf *scales_b, float *out_a,
                        float *out_b, Candidate *argmax, uint32_t *argmax_count)
{
    Packed p;
    mfh_status s = check_packed(ctx, codes_a, scales_a, &p);
    if (s)
        return s;
    if (codes_b) {
        Packed q;
        if ((s = check_packed(ctx, codes_b, scales_b, &q)))
            return s;
        if (q.format != p.format || q.rows != p.rows || q.inner != p.inner)
            return fail(ctx, MFH_INVALID_SHAPE,
                        "packed linear pair requires equal weight and output shapes");
    }
    if (p.rows != n || p.inner != k)
        return fail(ctx, MFH_INVALID_SHAPE, "packed linear input width differs from weight width");
    // Every operand the transform reads must be present (the kernels do not
    // check): a, plus b for SwiGLU and w for the norm.
    bool operands = out_a && xform.a && (epilogue != Epilogue::Pair || out_b);
    switch (xform.kind) {
    case XKind::Plain: break;
    case XKind::AddRms: operands = operands && xform.w; break;
    case XKind::Swiglu: operands = operands && xform.b; break;
    case XKind::GqaMerge: break;
    }
    if (!operands)
        return fail(ctx, MFH_INVALID_ARGUMENT, "fused decode product is missing an operand");
    PackedCall call;
    call.format = p.format;
    call.epilogue = epilogue;
    call.m = m;
    call.n = n;
    call.k = k;
    call.a = stream_of(codes_a, scales_a);
    if (codes_b)
        call.b = stream_of(codes_b, scales_b);
    call.out_a = out_a;
    call.out_b = out_b;
    call.xform = xform;
    call.argmax = argmax;
    call.argmax_count = argmax_count;
    if (xform.kind == XKind::Plain)
        call.x = xform.a;  // the GEMV reads a Plain source from call.x
    const bool mfma = use_mfma_gemv(ctx, call) && m >= 1 && m <= 2;
    if (xform.kind == XKind::GqaMerge) {
        // A merge the one-row wide kernel cannot serve is the caller's
        // ordinary case (it combines the ranges and projects plainly), so
        // it leaves no error message.
        call.separate_prologue = ctx->kernel_path == 2;
        if (!mfma || !gqa_merge_supported(call))
            return MFH_UNSUPPORTED;
    }
    if (!mfma)
        return fail(ctx, MFH_UNSUPPORTED, "fused decode product needs the matrix-core GEMV");
    DeviceGuard guard(ctx->device);
    return run_packed(ctx, call, codes_a, scales_a, codes_b, scales_b);
}

mfh_status packed_xform_conv(mfh_ctx *ctx, const XForm &xform, uint32_t k,
                             const mfh_buf *codes, const mfh_buf *scales, const ConvStep &conv)
{
    Packed p;
    mfh_status s = check_packed(ctx, codes, scales, &p);
    if (s)
        return s;
    if (p.rows != 3 * uint64_t(conv.hidden) || p.inner != k)
        return fail(ctx, MFH_INVALID_SHAPE, "packed linear input width differs from weight width");
    if (xform.kind != XKind::AddRms || !xform.a || !xform.w || !conv.kernel || !conv.history ||
        !conv.next || !conv.out || conv.width < 1 || ctx->kernel_path != 0)
        return fail(ctx, MFH_UNSUPPORTED, "fused convolution needs the one-row decode kernels");
    PackedCall call;
    call.format = p.format;
    call.epilogue = Epilogue::Single;
    call.m = 1;
    call.n = p.rows;
    call.k = k;
    call.a = stream_of(codes, scales);
    call.xform = xform;
    DeviceGuard guard(ctx->device);
    if (wide_conv_supported(call, conv)) {
        if ((s = prepare_tiles(ctx, codes, scales, p, &call.a)))
            return s;
        try_wide_conv(ctx->stream, call, conv);
    } else if (!try_vgemv_conv(ctx->stream, call, conv)) {
        return fail(ctx, MFH_UNSUPPORTED, "fused convolution needs the one-row decode kernels");
    }
    if (hipGetLastError() != hipSuccess)
        return fail(ctx, MFH_BACKEND_FAILURE, "packed kernel launch failed");
    return MFH_OK;
}

mfh_status packed_xform_segments(mfh_ctx *ctx, const XForm &xform, uint32_t m, uint32_t k,
                                 uint32_t count, const mfh_buf *const *codes,
                                 const mfh_buf *const *scales, const uint32_t *n,
                                 float *const *out)
{
    if (count == 0 || count > kMaxSegments || m == 0 || m > 2 ||
        !xform.a || (xform.kind == XKind::AddRms && !xform.w) ||
        (xform.kind == XKind::Swiglu && !xform.b))
        return fail(ctx, MFH_UNSUPPORTED, "fused decode product needs the matrix-core GEMV");
    PackedCall call;
    call.epilogue = Epilogue::Single;
    call.m = m;
    call.k = k;
    call.xform = xform;
    if (xform.kind == XKind::Plain)
        call.x = xform.a;
    call.segments = count;
    Packed first;
    for (uint32_t i = 0; i < count; ++i) {
        Packed p;
        mfh_status s = check_packed(ctx, codes[i], scales[i], &p);
        if (s)
            return s;
        if (i == 0)
            first = p;
        if (p.format != first.format || p.inner != k || p.rows != n[i] || !out[i])
            return fail(ctx, MFH_INVALID_SHAPE,
                        "packed linear input width differs from weight width");
        call.seg[i] = stream_of(codes[i], scales[i]);
        call.seg_out[i] = out[i];
        call.seg_n[i] = n[i];
    }
    call.format = first.format;
    call.n = n[0];
    if (!use_mfma_gemv(ctx, call))
        return fail(ctx, MFH_UNSUPPORTED, "fused decode product needs the matrix-core GEMV");
    DeviceGuard guard(ctx->device);
    for (uint32_t i = 0; i < count; ++i) {
        Packed p{n[i], k, first.format};
        mfh_status s = prepare_tiles(ctx, codes[i], scales[i], p, &call.seg[i]);
        if (s)
            return s;
        if (call.seg[i].tiled_half != call.seg[0].tiled_half)
            return fail(ctx, MFH_UNSUPPORTED, "segment scales differ in width");
    }
    call.a.tiled_half = call.seg[0].tiled_half;
    void *scratch = digits_scratch(ctx, gemv_mfma_scratch_bytes(call));
    if (!scratch)
        return allocation_failed(ctx);
    call.separate_prologue = ctx->kernel_path == 2;
    launch_gemv_mfma(ctx->stream, call, scratch);
    if (hipGetLastError() != hipSuccess)
        return fail(ctx, MFH_BACKEND_FAILURE, "packed kernel launch failed");
    return MFH_OK;
}

mfh_status admit_packed_linear(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                               const mfh_buf *codes, const mfh_buf *scales, PackedCall *call)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_PACKED_LINEAR);
    if (!s)
        s = check_f32(ctx, input);
    if (s)
        return s;
    Packed p;
    if ((s = check_packed(ctx, codes, scales, &p)))
        return s;
    if (input->rank != 2)
        return fail(ctx, MFH_INVALID_SHAPE, "packed linear input must be rank two");
    if (input->dims[1] != p.inner)
        return fail(ctx, MFH_INVALID_SHAPE, "packed linear input width differs from weight width");
    uint64_t dims[2] = {input->dims[0], p.rows};
    if ((s = check_output(ctx, output, dims, 2)))
        return s;
    if (aliases(output, {input, codes, scales}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    if (input->dims[0] > UINT32_MAX)
        return fail(ctx, MFH_OVERFLOW, "packed linear row count exceeds the kernel index range");
    call->format = p.format;
    call->epilogue = Epilogue::Single;
    call->m = uint32_t(input->dims[0]);
    call->n = p.rows;
    call->k = p.inner;
    call->x = static_cast<const float *>(input->dev);
    call->a = stream_of(codes, scales);
    call->out_a = static_cast<float *>(output->dev);
    return MFH_OK;
}

bool prepared_stream(const mfh_buf *codes, const mfh_buf *scales, Format format,
                     PackedStream *stream)
{
    const bool half = scales->f16_shadow != nullptr;
    if (!codes->repacked || codes->repacked_format != int(format) || !scales->tiled_scales ||
        scales->tiled_format != int(format) || scales->tiled_half != half)
        return false;
    stream->tiles = static_cast<const uint8_t *>(codes->repacked);
    stream->tiled_scales = scales->tiled_scales;
    stream->tiled_half = half;
    return true;
}

mfh_status prepare_packed(mfh_ctx *ctx, const mfh_buf *codes, const mfh_buf *scales)
{
    Packed p;
    mfh_status s = check_packed(ctx, codes, scales, &p);
    if (s)
        return s;
    if (p.rows == 0 || p.inner == 0)
        return MFH_OK;
    DeviceGuard guard(ctx->device);
    return prepare_tiles(ctx, codes, scales, p, nullptr);
}

}  // namespace mfh

using namespace mfh;

extern "C" {

mfh_status mfh_prepare_packed(mfh_ctx *ctx, const mfh_buf *codes, const mfh_buf *scales)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    if (ctx->cancel_requested)
        return fail(ctx, MFH_CANCELLED, "operation cancelled");
    return prepare_packed(ctx, codes, scales);
}

int mfh_packed_prepared(const mfh_ctx *ctx, const mfh_buf *codes, const mfh_buf *scales)
{
    if (!ctx || !codes || !scales || codes->ctx != ctx || scales->ctx != ctx)
        return 0;
    Packed p;
    if (check_packed(const_cast<mfh_ctx *>(ctx), codes, scales, &p))
        return 0;
    PackedStream unused;
    return prepared_stream(codes, scales, p.format, &unused) ? 1 : 0;
}

mfh_status mfh_packed_gather_rows(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *codes,
                                  const mfh_buf *scales, const uint32_t *host_ids,
                                  size_t host_count, const mfh_buf *device_ids)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_PACKED_GATHER_ROWS);
    if (s)
        return s;
    Packed p;
    if ((s = check_packed(ctx, codes, scales, &p)))
        return s;
    if ((s = check_f32(ctx, output)))
        return s;
    if (device_ids && host_ids)
        return fail(ctx, MFH_INVALID_ARGUMENT, "token ids must be either host or device ids");
    uint64_t count = 0;
    if (device_ids) {
        if ((s = check_f32(ctx, device_ids)))
            return s;
        if (device_ids->rank != 1)
            return fail(ctx, MFH_INVALID_SHAPE, "device token-id buffer must be rank one");
        count = device_ids->dims[0];
    } else {
        if (host_count && !host_ids)
            return fail(ctx, MFH_INVALID_ARGUMENT, "host id pointer is null");
        for (size_t i = 0; i < host_count; ++i)
            if (host_ids[i] >= p.rows || host_ids[i] >= (1u << 24))
                return fail(ctx, MFH_OUT_OF_BOUNDS, "gather identifier exceeds row count");
        count = host_count;
    }
    uint64_t dims[2] = {count, p.inner};
    if (output->rank != 2 || output->dims[0] != dims[0] || output->dims[1] != dims[1])
        return fail(ctx, MFH_INVALID_SHAPE, "packed gather output layout differs from required shape");
    if (aliases(output, {codes, scales, device_ids}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    if (count > UINT32_MAX)
        return fail(ctx, MFH_OVERFLOW, "gather id count exceeds the kernel index range");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    if (count == 0 || p.inner == 0)
        return MFH_OK;
    const float *ids = nullptr;
    if (device_ids) {
        ids = static_cast<const float *>(device_ids->dev);
    } else {
        // Host ids travel as exact f32 row selectors (< 2^24 by admission).
        std::vector<float> staged(host_count);
        for (size_t i = 0; i < host_count; ++i)
            staged[i] = float(host_ids[i]);
        void *dst = ids_scratch(ctx, host_count * sizeof(float));
        if (!dst)
            return allocation_failed(ctx);
        if (hipMemcpyAsync(dst, staged.data(), host_count * sizeof(float), hipMemcpyHostToDevice,
                           ctx->stream) != hipSuccess) {
            (void)hipGetLastError();
            return fail(ctx, MFH_BACKEND_FAILURE, "host to device copy failed");
        }
        ids = static_cast<const float *>(dst);
    }
    launch_packed_gather(ctx->stream, p.format, static_cast<float *>(output->dev),
                         static_cast<const uint8_t *>(codes->dev),
                         static_cast<const float *>(scales->dev), ids, uint32_t(count), p.rows,
                         p.inner);
    if (hipGetLastError() != hipSuccess)
        return fail(ctx, MFH_BACKEND_FAILURE, "packed kernel launch failed");
    return MFH_OK;
}

mfh_status mfh_packed_linear(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                             const mfh_buf *codes, const mfh_buf *scales)
{
    PackedCall call;
    mfh_status s = admit_packed_linear(ctx, output, input, codes, scales, &call);
    if (s)
        return s;
    DeviceGuard guard(ctx->device);
    mark_written(output);
    return run_packed(ctx, call, codes, scales);
}

mfh_status mfh_packed_linear_pair(mfh_ctx *ctx, mfh_buf *out_a, mfh_buf *out_b,
                                  const mfh_buf *input, const mfh_buf *codes_a,
                                  const mfh_buf *scales_a, const mfh_buf *codes_b,
                                  const mfh_buf *scales_b)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_PACKED_LINEAR_PAIR);
    if (s)
        return s;
    if (!same_shape(codes_a, codes_b) || !same_shape(scales_a, scales_b) ||
        !same_shape(out_a, out_b))
        return fail(ctx, MFH_INVALID_SHAPE,
                    "packed linear pair requires equal weight and output shapes");
    // Both projections pass admission before either output is written.
    if ((s = check_f32(ctx, input)))
        return s;
    Packed p, q;
    if ((s = check_packed(ctx, codes_a, scales_a, &p)) || (s = check_packed(ctx, codes_b, scales_b, &q)))
        return s;
    if (input->rank != 2)
        return fail(ctx, MFH_INVALID_SHAPE, "packed linear input must be rank two");
    if (input->dims[1] != p.inner)
        return fail(ctx, MFH_INVALID_SHAPE, "packed linear input width differs from weight width");
    uint64_t dims[2] = {input->dims[0], p.rows};
    if ((s = check_output(ctx, out_a, dims, 2)) || (s = check_output(ctx, out_b, dims, 2)))
        return s;
    if (out_a->dev && out_a->dev == out_b->dev)
        return fail(ctx, MFH_INVALID_ARGUMENT, "pair outputs alias each other");
    if (aliases(out_a, {input, codes_a, scales_a, codes_b, scales_b}) ||
        aliases(out_b, {input, codes_a, scales_a, codes_b, scales_b}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    if (input->dims[0] > UINT32_MAX)
        return fail(ctx, MFH_OVERFLOW, "packed linear row count exceeds the kernel index range");
    DeviceGuard guard(ctx->device);
    mark_written(out_a);
    mark_written(out_b);
    PackedCall call;
    call.format = p.format;
    call.epilogue = Epilogue::Pair;
    call.m = uint32_t(input->dims[0]);
    call.n = p.rows;
    call.k = p.inner;
    call.x = static_cast<const float *>(input->dev);
    call.a = stream_of(codes_a, scales_a);
    call.b = stream_of(codes_b, scales_b);
    call.out_a = static_cast<float *>(out_a->dev);
    call.out_b = static_cast<float *>(out_b->dev);
    return run_packed(ctx, call, codes_a, scales_a, codes_b, scales_b);
}

mfh_status mfh_packed_swiglu_linear(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *gate,
                                    const mfh_buf *up, const mfh_buf *codes,
                                    const mfh_buf *scales)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_PACKED_SWIGLU_LINEAR);
    if (!s)
        s = check_f32(ctx, gate);
    if (!s)
        s = check_f32(ctx, up);
    if (s)
        return s;
    Packed p;
    if ((s = check_packed(ctx, codes, scales, &p)))
        return s;
    if (gate->rank != 2 || !same_shape(gate, up))
        return fail(ctx, MFH_INVALID_SHAPE,
                    "packed SwiGLU gate and up layouts must match and be rank two");
    if (gate->dims[1] != p.inner)
        return fail(ctx, MFH_INVALID_SHAPE, "packed SwiGLU input width differs from weight width");
    uint64_t dims[2] = {gate->dims[0], p.rows};
    if ((s = check_output(ctx, output, dims, 2)))
        return s;
    if (aliases(output, {gate, up, codes, scales}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    if (gate->dims[0] > UINT32_MAX)
        return fail(ctx, MFH_OVERFLOW, "packed SwiGLU row count exceeds the kernel index range");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    PackedCall call;
    call.format = p.format;
    call.epilogue = Epilogue::Single;
    call.m = uint32_t(gate->dims[0]);
    call.n = p.rows;
    call.k = p.inner;
    call.a = stream_of(codes, scales);
    call.out_a = static_cast<float *>(output->dev);
    if (use_mfma_gemv(ctx, call)) {
        // The GEMV's activation prologue forms silu(gate) * up as it reads them.
        call.xform.kind = XKind::Swiglu;
        call.xform.a = static_cast<const float *>(gate->dev);
        call.xform.b = static_cast<const float *>(up->dev);
        return run_packed(ctx, call, codes, scales);
    }
    const size_t count = size_t(gate->dims[0]) * p.inner;
    // Stage silu(gate) * up once, then run the plain packed product on it
    // (backend-cpu/src/packed.rs:425-455).
    float *activated = static_cast<float *>(work_scratch(ctx, count * sizeof(float)));
    if (count && !activated)
        return allocation_failed(ctx);
    launch_swiglu(ctx->stream, activated, static_cast<const float *>(gate->dev),
                  static_cast<const float *>(up->dev), count);
    call.x = activated;
    return run_packed(ctx, call, codes, scales);
}

mfh_status mfh_packed_swiglu_pair(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                                  const mfh_buf *codes_a, const mfh_buf *scales_a,
                                  const mfh_buf *codes_b, const mfh_buf *scales_b)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_PACKED_SWIGLU_PAIR);
    if (!s)
        s = check_f32(ctx, input);
    if (s)
        return s;
    if (!same_shape(codes_a, codes_b) || !same_shape(scales_a, scales_b))
        return fail(ctx, MFH_INVALID_SHAPE, "packed SwiGLU pair requires equal weight shapes");
    Packed p, q;
    if ((s = check_packed(ctx, codes_a, scales_a, &p)) || (s = check_packed(ctx, codes_b, scales_b, &q)))
        return s;
    if (input->rank != 2)
        return fail(ctx, MFH_INVALID_SHAPE, "packed SwiGLU pair input must be rank two");
    if (input->dims[1] != p.inner)
        return fail(ctx, MFH_INVALID_SHAPE,
                    "packed SwiGLU pair input width differs from weight width");
    uint64_t dims[2] = {input->dims[0], p.rows};
    if ((s = check_output(ctx, output, dims, 2)))
        return s;
    if (aliases(output, {input, codes_a, scales_a, codes_b, scales_b}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    if (input->dims[0] > UINT32_MAX)
        return fail(ctx, MFH_OVERFLOW, "packed SwiGLU row count exceeds the kernel index range");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    PackedCall call;
    call.format = p.format;
    call.epilogue = Epilogue::SwigluPair;
    call.m = uint32_t(input->dims[0]);
    call.n = p.rows;
    call.k = p.inner;
    call.x = static_cast<const float *>(input->dev);
    call.a = stream_of(codes_a, scales_a);
    call.b = stream_of(codes_b, scales_b);
    call.out_a = static_cast<float *>(output->dev);
    return run_packed(ctx, call, codes_a, scales_a, codes_b, scales_b);
}

}  // extern "C"
