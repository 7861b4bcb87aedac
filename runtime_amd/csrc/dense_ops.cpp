// Dense LFM2 operations: admission and launches.
//
// Admission restates CpuBackend's checks in the reference's order and with
// its messages (crates/backend-cpu/src/{dense,normalization_rotary,
// attention_convolution}.rs, spec constructors in
// crates/engine-api/src/backend.rs:128-383).  Every operand is validated
// before anything is enqueued, so a rejected call writes nothing; the
// reference's CPU backend can leave earlier rows or the `sum` of a fused
// add-and-norm written when a later check fails.
//
// Two behaviours differ because device work is deferred: values are not
// inspected on the host, so a non-finite result propagates instead of
// raising BackendFailure, and a device token id outside the table gives a
// NaN row instead of OutOfBounds.  Outputs may not share storage with an
// input (the trait's `&mut` / `&` operands cannot alias).
#include <cmath>
#include <cstring>
#include <vector>

#include "internal.hpp"
#include "kernels.hpp"

namespace mfh {
namespace {

const float *dev_f32(const mfh_buf *b) { return static_cast<const float *>(b->dev); }
float *dev_f32(mfh_buf *b) { return static_cast<float *>(b->dev); }

// Copy `bytes` of host data into the context's staging scratch (stream
// ordered; pageable sources are consumed before the call returns).
const void *stage(mfh_ctx *ctx, const void *host, size_t bytes, mfh_status *status)
{
    void *dst = ids_scratch(ctx, bytes ? bytes : 4);
    if (!dst) {
        *status = allocation_failed(ctx);
        return nullptr;
    }
    if (bytes && hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, ctx->stream) != hipSuccess) {
        (void)hipGetLastError();
        *status = fail(ctx, MFH_BACKEND_FAILURE, "host to device copy failed");
        return nullptr;
    }
    *status = MFH_OK;
    return dst;
}

mfh_status launched(mfh_ctx *ctx)
{
    if (hipGetLastError() != hipSuccess)
        return fail(ctx, MFH_BACKEND_FAILURE, "dense kernel launch failed");
    return MFH_OK;
}

// PackedHeadSpec::new (backend.rs:240-247).
mfh_status head_spec(mfh_ctx *ctx, uint32_t heads, uint32_t head_dim)
{
    if (heads == 0 || head_dim == 0)
        return fail(ctx, MFH_INVALID_ARGUMENT, "head count and head dimension must be nonzero");
    return MFH_OK;
}

// PackedHeadSpec::validate_packed (backend.rs:264-276).
mfh_status validate_packed(mfh_ctx *ctx, const mfh_buf *buf, uint32_t heads, uint32_t head_dim,
                           uint64_t *tokens)
{
    if (buf->rank != 2)
        return fail(ctx, MFH_INVALID_SHAPE, "packed head tensor must be rank two");
    if (buf->dims[1] != uint64_t(heads) * head_dim)
        return fail(ctx, MFH_INVALID_SHAPE, "packed head tensor width differs from descriptor");
    *tokens = buf->dims[0];
    return MFH_OK;
}

// RotarySpec::new (backend.rs:287-300).
mfh_status rotary_spec(mfh_ctx *ctx, uint32_t heads, uint32_t head_dim, float theta)
{
    mfh_status s = head_spec(ctx, heads, head_dim);
    if (s)
        return s;
    if (head_dim % 2 != 0)
        return fail(ctx, MFH_INVALID_SHAPE, "split-half RoPE requires an even head dimension");
    if (!std::isfinite(theta) || theta <= 0.0f)
        return fail(ctx, MFH_INVALID_ARGUMENT, "RoPE theta must be finite and positive");
    return MFH_OK;
}

mfh_status check_epsilon(mfh_ctx *ctx, float epsilon)
{
    if (!std::isfinite(epsilon) || epsilon <= 0.0f)
        return fail(ctx, MFH_INVALID_ARGUMENT, "RMS epsilon must be finite and positive");
    return MFH_OK;
}

// Positions for the rotary kernels.  Consecutive positions (every decode and
// prefill pass of the executor) travel as their base in the kernel
// arguments; anything else is staged as f32 values converted like the
// reference's `position as f32` (round to nearest).
Positions stage_positions(mfh_ctx *ctx, const uint64_t *positions, size_t count,
                          mfh_status *status)
{
    Positions p;
    *status = MFH_OK;
    bool consecutive = count > 0 && positions[0] <= UINT64_MAX - count;
    for (size_t i = 1; consecutive && i < count; ++i)
        consecutive = positions[i] == positions[0] + i;
    if (consecutive) {
        p.base = positions[0];
        return p;
    }
    std::vector<float> staged(count);
    for (size_t i = 0; i < count; ++i)
        staged[i] = float(positions[i]);
    p.staged = static_cast<const float *>(stage(ctx, staged.data(), count * sizeof(float), status));
    return p;
}

// Element-wise add/multiply admission (dense.rs:166-182).
mfh_status check_elementwise(mfh_ctx *ctx, mfh_operation op, const mfh_buf *output,
                             const mfh_buf *left, const mfh_buf *right)
{
    mfh_status s = check_operation(ctx, op);
    if (!s)
        s = check_f32(ctx, left);
    if (!s)
        s = check_f32(ctx, right);
    if (s)
        return s;
    if (!same_shape(left, right))
        return fail(ctx, MFH_INVALID_SHAPE, "elementwise operands have different layouts");
    return check_output(ctx, output, left->dims, left->rank);
}

// row_rms_norm admission after the operation check (normalization_rotary.rs:19-52).
// Sets *width (0 means a no-op).
mfh_status check_row_rms(mfh_ctx *ctx, const mfh_buf *output, const mfh_buf *input,
                         const mfh_buf *weight, float epsilon, uint32_t *width)
{
    mfh_status s = check_epsilon(ctx, epsilon);
    if (!s)
        s = check_f32(ctx, input);
    if (!s)
        s = check_f32(ctx, weight);
    if (s)
        return s;
    if (input->rank != 2 || weight->rank != 1)
        return fail(ctx, MFH_INVALID_SHAPE, "RMS input must be rank two and weight rank one");
    if (input->dims[1] != weight->dims[0])
        return fail(ctx, MFH_INVALID_SHAPE, "RMS input width differs from weight width");
    if ((s = check_output(ctx, output, input->dims, 2)))
        return s;
    if (input->dims[1] > (uint64_t(1) << 24))
        return fail(ctx, MFH_UNSUPPORTED, "RMS width exceeds exact f32 divisor range");
    *width = uint32_t(input->dims[1]);
    return MFH_OK;
}

mfh_status check_argmax_input(mfh_ctx *ctx, const mfh_buf *output, const mfh_buf *input,
                              bool masked, const uint64_t *mask, size_t mask_words)
{
    mfh_status s = check_operation(ctx, MFH_OP_ARGMAX);
    if (!s)
        s = check_f32(ctx, input);
    if (s)
        return s;
    if (input->rank != 2)
        return fail(ctx, MFH_INVALID_SHAPE,
                    masked ? "masked argmax input must be rank two" : "argmax input must be rank two");
    const uint64_t width = input->dims[1];
    if (width == 0 || width > (uint64_t(1) << 24))
        return fail(ctx, MFH_UNSUPPORTED,
                    masked ? "masked argmax width must be in [1, 2^24] for exact f32 indices"
                           : "argmax width must be in [1, 2^24] for exact f32 indices");
    if (masked) {
        if (mask_words != (width + 63) / 64 || (mask_words && !mask))
            return fail(ctx, MFH_INVALID_ARGUMENT,
                        "masked argmax mask length must be ceil(width / 64)");
    }
    uint64_t dims[1] = {input->dims[0]};
    if ((s = check_output(ctx, output, dims, 1)))
        return s;
    if (aliases(output, {input}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    if (input->dims[0] > UINT32_MAX)
        return fail(ctx, MFH_OVERFLOW, "argmax row count exceeds the kernel index range");
    return MFH_OK;
}

mfh_status run_argmax(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input, const uint64_t *mask,
                      size_t mask_words)
{
    DeviceGuard guard(ctx->device);
    mark_written(output);
    const uint64_t *dev_mask = nullptr;
    if (mask) {
        mfh_status s;
        dev_mask = static_cast<const uint64_t *>(stage(ctx, mask, mask_words * 8, &s));
        if (s)
            return s;
    }
    const uint32_t rows = uint32_t(input->dims[0]), width = uint32_t(input->dims[1]);
    void *partials = nullptr;
    if (const size_t bytes = argmax_scratch_bytes(rows, width)) {
        partials = work_scratch(ctx, bytes);
        if (!partials)
            return allocation_failed(ctx);
    }
    launch_argmax(ctx->stream, dev_f32(output), dev_f32(input), rows, width, dev_mask, partials);
    return launched(ctx);
}

}  // namespace
}  // namespace mfh

using namespace mfh;

extern "C" {

mfh_status mfh_copy(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_COPY);
    if (!s)
        s = check_f32(ctx, input);
    if (!s)
        s = check_output(ctx, output, input->dims, input->rank);
    if (s)
        return s;
    if (aliases(output, {input}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    launch_copy(ctx->stream, dev_f32(output), dev_f32(input), size_t(input->elements));
    return launched(ctx);
}

mfh_status mfh_copy_rect_2d(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                            uint64_t source_row, uint64_t source_column,
                            uint64_t destination_row, uint64_t destination_column,
                            uint64_t rows, uint64_t columns)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_RECT_COPY_2D);
    if (!s)
        s = check_f32(ctx, input);
    if (!s)
        s = check_f32(ctx, output);
    if (s)
        return s;
    if (input->dev == output->dev)
        return fail(ctx, MFH_UNSUPPORTED,
                    "rectangular copy does not permit overlapping source and destination allocation");
    // RectCopy2d::validate (backend.rs:189-230).
    if (input->rank != 2 || output->rank != 2)
        return fail(ctx, MFH_INVALID_SHAPE,
                    "rectangular copy requires rank-two source and destination");
    if (source_row > UINT64_MAX - rows)
        return fail(ctx, MFH_OVERFLOW, "rectangular source row end overflows u64");
    if (source_column > UINT64_MAX - columns)
        return fail(ctx, MFH_OVERFLOW, "rectangular source column end overflows u64");
    if (destination_row > UINT64_MAX - rows)
        return fail(ctx, MFH_OVERFLOW, "rectangular destination row end overflows u64");
    if (destination_column > UINT64_MAX - columns)
        return fail(ctx, MFH_OVERFLOW, "rectangular destination column end overflows u64");
    if (source_row + rows > input->dims[0] || source_column + columns > input->dims[1] ||
        destination_row + rows > output->dims[0] ||
        destination_column + columns > output->dims[1])
        return fail(ctx, MFH_OUT_OF_BOUNDS,
                    "rectangular copy range exceeds source or destination shape");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    RectCopy rect{input->dims[1], output->dims[1], source_row,  source_column,
                  destination_row, destination_column, rows,   columns};
    launch_rect_copy(ctx->stream, dev_f32(output), dev_f32(input), rect);
    return launched(ctx);
}

mfh_status mfh_argmax(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_argmax_input(ctx, output, input, false, nullptr, 0);
    if (s)
        return s;
    return run_argmax(ctx, output, input, nullptr, 0);
}

mfh_status mfh_argmax_masked(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                             const uint64_t *mask, size_t mask_words)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_argmax_input(ctx, output, input, true, mask, mask_words);
    if (s)
        return s;
    return run_argmax(ctx, output, input, mask, mask_words);
}

mfh_status mfh_gather_rows(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *table,
                           const uint32_t *host_ids, size_t host_count,
                           const mfh_buf *device_ids)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_GATHER_ROWS);
    if (!s)
        s = check_f32(ctx, table);
    if (s)
        return s;
    if (table->rank != 2)
        return fail(ctx, MFH_INVALID_SHAPE, "gather table must be rank two");
    if (device_ids && host_ids)
        return fail(ctx, MFH_INVALID_ARGUMENT, "token ids must be either host or device ids");
    uint64_t count = host_count;
    if (device_ids) {
        if ((s = check_f32(ctx, device_ids)))
            return s;
        if (device_ids->rank != 1)
            return fail(ctx, MFH_INVALID_SHAPE, "device token-id buffer must be rank one");
        count = device_ids->dims[0];
    } else if (host_count && !host_ids) {
        return fail(ctx, MFH_INVALID_ARGUMENT, "host id pointer is null");
    }
    uint64_t dims[2] = {count, table->dims[1]};
    if ((s = check_output(ctx, output, dims, 2)))
        return s;
    for (size_t i = 0; !device_ids && i < host_count; ++i) {
        if (host_ids[i] >= table->dims[0])
            return fail(ctx, MFH_OUT_OF_BOUNDS, "gather identifier exceeds row count");
        if (host_ids[i] >= (1u << 24))
            return fail(ctx, MFH_UNSUPPORTED, "gather identifier exceeds the exact f32 selector range");
    }
    if (aliases(output, {table, device_ids}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    if (count > UINT32_MAX || table->dims[0] > UINT32_MAX)
        return fail(ctx, MFH_OVERFLOW, "gather extent exceeds the kernel index range");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    if (count == 0 || table->dims[1] == 0)
        return MFH_OK;
    const float *ids = nullptr;
    if (device_ids) {
        ids = dev_f32(device_ids);
    } else {
        // Host ids travel as exact f32 row selectors (< 2^24 by admission).
        std::vector<float> staged(host_count);
        for (size_t i = 0; i < host_count; ++i)
            staged[i] = float(host_ids[i]);
        ids = static_cast<const float *>(stage(ctx, staged.data(), host_count * 4, &s));
        if (s)
            return s;
    }
    launch_gather_rows(ctx->stream, dev_f32(output), dev_f32(table), ids, uint32_t(count),
                       uint32_t(table->dims[0]), table->dims[1]);
    return launched(ctx);
}

mfh_status mfh_gather_columns(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                              const uint32_t *columns, size_t count)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_GATHER_COLUMNS);
    if (!s)
        s = check_f32(ctx, input);
    if (s)
        return s;
    if (input->rank != 2)
        return fail(ctx, MFH_INVALID_SHAPE, "column gather input must be rank two");
    if (count && !columns)
        return fail(ctx, MFH_INVALID_ARGUMENT, "column pointer is null");
    for (size_t k = 0; k < count; ++k)
        if (columns[k] >= input->dims[1])
            return fail(ctx, MFH_OUT_OF_BOUNDS, "column gather identifier exceeds input width");
    uint64_t dims[2] = {input->dims[0], count};
    if ((s = check_output(ctx, output, dims, 2)))
        return s;
    if (aliases(output, {input}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    if (count > UINT32_MAX)
        return fail(ctx, MFH_OVERFLOW, "column count exceeds the kernel index range");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    if (count == 0 || input->dims[0] == 0)
        return MFH_OK;
    const uint32_t *cols = static_cast<const uint32_t *>(stage(ctx, columns, count * 4, &s));
    if (s)
        return s;
    launch_gather_columns(ctx->stream, dev_f32(output), dev_f32(input), cols, input->dims[0],
                          input->dims[1], uint32_t(count));
    return launched(ctx);
}

mfh_status mfh_add(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *left, const mfh_buf *right)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_elementwise(ctx, MFH_OP_ADD, output, left, right);
    if (s)
        return s;
    if (aliases(output, {left, right}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    launch_binary(ctx->stream, 0, dev_f32(output), dev_f32(left), dev_f32(right),
                  size_t(left->elements));
    return launched(ctx);
}

mfh_status mfh_multiply(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *left,
                        const mfh_buf *right)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_elementwise(ctx, MFH_OP_MULTIPLY, output, left, right);
    if (s)
        return s;
    if (aliases(output, {left, right}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    launch_binary(ctx->stream, 1, dev_f32(output), dev_f32(left), dev_f32(right),
                  size_t(left->elements));
    return launched(ctx);
}

mfh_status mfh_linear(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                      const mfh_buf *weight)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_LINEAR);
    if (!s)
        s = check_f32(ctx, input);
    if (!s)
        s = check_f32(ctx, weight);
    if (s)
        return s;
    if (input->rank != 2 || weight->rank != 2)
        return fail(ctx, MFH_INVALID_SHAPE, "linear input and weight must be rank two");
    if (input->dims[1] != weight->dims[1])
        return fail(ctx, MFH_INVALID_SHAPE, "linear input width differs from weight width");
    uint64_t dims[2] = {input->dims[0], weight->dims[0]};
    if ((s = check_output(ctx, output, dims, 2)))
        return s;
    if (aliases(output, {input, weight}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    if (dims[0] > UINT32_MAX || dims[1] > UINT32_MAX || input->dims[1] > UINT32_MAX)
        return fail(ctx, MFH_OVERFLOW, "linear extent exceeds the kernel index range");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    launch_linear(ctx->stream, dev_f32(output), dev_f32(input), dev_f32(weight),
                  uint32_t(dims[0]), uint32_t(dims[1]), uint32_t(input->dims[1]));
    return launched(ctx);
}

mfh_status mfh_row_rms_norm(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                            const mfh_buf *weight, float epsilon)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_ROW_RMS_NORM);
    uint32_t width = 0;
    if (!s)
        s = check_row_rms(ctx, output, input, weight, epsilon, &width);
    if (s)
        return s;
    if (aliases(output, {input, weight}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    launch_row_rms(ctx->stream, dev_f32(output), nullptr, dev_f32(input), nullptr,
                   dev_f32(weight), input->dims[0], width, epsilon);
    return launched(ctx);
}

mfh_status mfh_head_rms_norm(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                             const mfh_buf *weight, uint32_t heads, uint32_t head_dim,
                             float epsilon)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = head_spec(ctx, heads, head_dim);
    if (!s)
        s = check_operation(ctx, MFH_OP_ROW_RMS_NORM);
    if (!s)
        s = check_epsilon(ctx, epsilon);
    if (!s)
        s = check_f32(ctx, input);
    if (!s)
        s = check_f32(ctx, weight);
    uint64_t tokens = 0;
    if (!s)
        s = validate_packed(ctx, input, heads, head_dim, &tokens);
    if (s)
        return s;
    if (weight->rank != 1 || weight->dims[0] != head_dim)
        return fail(ctx, MFH_INVALID_SHAPE, "head RMS weight must have head_dim entries");
    if ((s = check_output(ctx, output, input->dims, 2)))
        return s;
    if (head_dim > (1u << 24))
        return fail(ctx, MFH_UNSUPPORTED, "RMS width exceeds exact f32 divisor range");
    if (aliases(output, {input, weight}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    launch_head_rms(ctx->stream, dev_f32(output), dev_f32(input), dev_f32(weight),
                    tokens * heads, head_dim, epsilon);
    return launched(ctx);
}

mfh_status mfh_split_half_rotary(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                                 const uint64_t *positions, size_t position_count,
                                 uint32_t heads, uint32_t head_dim, float theta)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = rotary_spec(ctx, heads, head_dim, theta);
    if (!s)
        s = check_operation(ctx, MFH_OP_ROTARY);
    if (!s)
        s = check_f32(ctx, input);
    uint64_t tokens = 0;
    if (!s)
        s = validate_packed(ctx, input, heads, head_dim, &tokens);
    if (s)
        return s;
    if (position_count != tokens)
        return fail(ctx, MFH_INVALID_SHAPE, "RoPE position count differs from token count");
    if (position_count && !positions)
        return fail(ctx, MFH_INVALID_ARGUMENT, "position pointer is null");
    if ((s = check_output(ctx, output, input->dims, 2)))
        return s;
    if (aliases(output, {input}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    if (tokens == 0)
        return MFH_OK;
    const Positions pos = stage_positions(ctx, positions, position_count, &s);
    if (s)
        return s;
    launch_rotary(ctx->stream, dev_f32(output), dev_f32(input), pos, tokens, heads, head_dim,
                  theta);
    return launched(ctx);
}

mfh_status mfh_add_row_rms_norm(mfh_ctx *ctx, mfh_buf *sum, mfh_buf *normed,
                                const mfh_buf *left, const mfh_buf *right,
                                const mfh_buf *weight, float epsilon)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_ADD_ROW_RMS_NORM);
    if (!s)
        s = check_elementwise(ctx, MFH_OP_ADD, sum, left, right);
    uint32_t width = 0;
    if (!s)
        s = check_row_rms(ctx, normed, sum, weight, epsilon, &width);
    if (s)
        return s;
    if (sum->dev == normed->dev)
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    if (aliases(sum, {left, right, weight}) || aliases(normed, {left, right, weight}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    DeviceGuard guard(ctx->device);
    mark_written(sum);
    mark_written(normed);
    const uint64_t rows = left->dims[0];
    if (width == 0) {
        // The add still runs; the norm of an empty row is a no-op.
        launch_binary(ctx->stream, 0, dev_f32(sum), dev_f32(left), dev_f32(right),
                      size_t(left->elements));
        return launched(ctx);
    }
    launch_row_rms(ctx->stream, dev_f32(normed), dev_f32(sum), dev_f32(left), dev_f32(right),
                   dev_f32(weight), rows, width, epsilon);
    return launched(ctx);
}

mfh_status mfh_qk_norm_rope(mfh_ctx *ctx, mfh_buf *query_out, mfh_buf *key_out,
                            const mfh_buf *query, const mfh_buf *key,
                            const mfh_buf *query_weight, const mfh_buf *key_weight,
                            const uint64_t *positions, size_t position_count,
                            uint32_t query_heads, uint32_t head_dim, float theta,
                            uint32_t key_value_heads, uint32_t key_value_head_dim,
                            float epsilon)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = rotary_spec(ctx, query_heads, head_dim, theta);
    if (!s)
        s = head_spec(ctx, key_value_heads, key_value_head_dim);
    if (!s)
        s = check_operation(ctx, MFH_OP_QK_NORM_ROPE);
    if (!s)
        s = check_epsilon(ctx, epsilon);
    if (!s)
        s = check_f32(ctx, query);
    if (!s)
        s = check_f32(ctx, key);
    if (!s)
        s = check_f32(ctx, query_weight);
    if (!s)
        s = check_f32(ctx, key_weight);
    if (s)
        return s;
    if (key_value_head_dim != head_dim)
        return fail(ctx, MFH_INVALID_SHAPE, "RoPE head dimensions must match for query and key");
    uint64_t query_tokens = 0, key_tokens = 0;
    if ((s = validate_packed(ctx, query, query_heads, head_dim, &query_tokens)) ||
        (s = validate_packed(ctx, key, key_value_heads, head_dim, &key_tokens)))
        return s;
    if (query_tokens != key_tokens)
        return fail(ctx, MFH_INVALID_SHAPE, "RoPE query and key token counts differ");
    if (position_count != query_tokens)
        return fail(ctx, MFH_INVALID_SHAPE, "RoPE position count differs from token count");
    if (position_count && !positions)
        return fail(ctx, MFH_INVALID_ARGUMENT, "position pointer is null");
    if ((s = check_output(ctx, query_out, query->dims, 2)) ||
        (s = check_output(ctx, key_out, key->dims, 2)))
        return s;
    if (query_weight->rank != 1 || query_weight->dims[0] != head_dim)
        return fail(ctx, MFH_INVALID_SHAPE, "query");
    if (key_weight->rank != 1 || key_weight->dims[0] != head_dim)
        return fail(ctx, MFH_INVALID_SHAPE, "key");
    if (head_dim > (1u << 24))
        return fail(ctx, MFH_UNSUPPORTED, "RMS width exceeds exact f32 divisor range");
    if (query_out->dev == key_out->dev ||
        aliases(query_out, {query, key, query_weight, key_weight}) ||
        aliases(key_out, {query, key, query_weight, key_weight}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    DeviceGuard guard(ctx->device);
    mark_written(query_out);
    mark_written(key_out);
    if (query_tokens == 0)
        return MFH_OK;
    const Positions pos = stage_positions(ctx, positions, position_count, &s);
    if (s)
        return s;
    launch_qk_norm_rope(ctx->stream, dev_f32(query_out), dev_f32(key_out), dev_f32(query),
                        dev_f32(key), dev_f32(query_weight), dev_f32(key_weight), pos,
                        query_tokens, query_heads, key_value_heads, head_dim, theta, epsilon);
    return launched(ctx);
}

mfh_status mfh_causal_gqa(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *query,
                          const mfh_buf *key, const mfh_buf *value, mfh_buf *key_cache,
                          mfh_buf *value_cache, uint64_t *cache_len, uint32_t query_heads,
                          uint32_t key_value_heads, uint32_t head_dim)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    // GqaSpec::new (backend.rs:320-335).
    if (key_value_heads == 0 || query_heads == 0 || query_heads % key_value_heads != 0)
        return fail(ctx, MFH_INVALID_SHAPE,
                    "query heads must be a nonzero multiple of key/value heads");
    mfh_status s = head_spec(ctx, query_heads, head_dim);
    if (!s)
        s = check_operation(ctx, MFH_OP_GROUPED_QUERY_ATTENTION);
    if (!s)
        s = check_f32(ctx, query);
    if (!s)
        s = check_f32(ctx, key);
    if (!s)
        s = check_f32(ctx, value);
    if (!s)
        s = check_f32(ctx, key_cache);
    if (!s)
        s = check_f32(ctx, value_cache);
    if (s)
        return s;
    if (!cache_len)
        return fail(ctx, MFH_INVALID_ARGUMENT, "cache length pointer is null");
    if (key_cache->dev == value_cache->dev)
        return fail(ctx, MFH_INVALID_ARGUMENT, "key and value caches must have distinct storage");
    uint64_t tokens = 0, key_tokens = 0, value_tokens = 0;
    if ((s = validate_packed(ctx, query, query_heads, head_dim, &tokens)))
        return s;
    if ((s = validate_packed(ctx, key, key_value_heads, head_dim, &key_tokens)))
        return s;
    if (key_tokens == tokens &&
        (s = validate_packed(ctx, value, key_value_heads, head_dim, &value_tokens)))
        return s;
    if (key_tokens != tokens || value_tokens != tokens)
        return fail(ctx, MFH_INVALID_SHAPE, "GQA query, key, and value token counts differ");
    if ((s = check_output(ctx, output, query->dims, 2)))
        return s;
    const uint64_t kv_width = uint64_t(key_value_heads) * head_dim;
    if (key_cache->rank != 2 || key_cache->dims[1] != kv_width ||
        !same_shape(key_cache, value_cache))
        return fail(ctx, MFH_INVALID_SHAPE,
                    "GQA caches must have matching [capacity, kv_heads * head_dim] shape");
    const uint64_t capacity = key_cache->dims[0];
    if (*cache_len > UINT64_MAX - tokens)
        return fail(ctx, MFH_OVERFLOW, "GQA cache length overflows u64");
    const uint64_t new_len = *cache_len + tokens;
    if (*cache_len > capacity || new_len > capacity)
        return fail(ctx, MFH_OUT_OF_BOUNDS, "GQA append exceeds cache capacity");
    if (head_dim > kMaxGqaHeadDim)
        return fail(ctx, MFH_UNSUPPORTED, "GQA head dimension exceeds the device kernel limit");
    if (tokens * query_heads > uint64_t(INT32_MAX) / 256)
        return fail(ctx, MFH_OVERFLOW, "GQA token count exceeds the kernel index range");
    if (aliases(output, {query, key, value, key_cache, value_cache}) ||
        aliases(key_cache, {query, key, value}) || aliases(value_cache, {query, key, value}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    mark_written(key_cache);
    mark_written(value_cache);
    GqaShape g;
    g.tokens = tokens;
    g.initial_len = *cache_len;
    g.query_heads = query_heads;
    g.key_value_heads = key_value_heads;
    g.head_dim = head_dim;
    g.group = query_heads / key_value_heads;
    g.scale = 1.0f / std::sqrt(float(head_dim));
    float *partials = nullptr;
    if (const size_t bytes = gqa_scratch_bytes(g)) {
        partials = static_cast<float *>(work_scratch(ctx, bytes));
        if (!partials)
            return allocation_failed(ctx);
    }
    launch_gqa(ctx->stream, dev_f32(output), dev_f32(query), dev_f32(key), dev_f32(value),
               dev_f32(key_cache), dev_f32(value_cache), g, partials);
    if ((s = launched(ctx)))
        return s;
    *cache_len = new_len;
    return MFH_OK;
}

mfh_status mfh_gated_short_convolution(mfh_ctx *ctx, mfh_buf *output,
                                       const mfh_buf *projection, const mfh_buf *kernel,
                                       mfh_buf *history, uint32_t hidden, uint32_t width)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    // GatedShortConvSpec::new (backend.rs:356-364).
    if (hidden == 0 || width == 0)
        return fail(ctx, MFH_INVALID_ARGUMENT,
                    "short convolution hidden width and kernel width must be nonzero");
    mfh_status s = check_operation(ctx, MFH_OP_GATED_SHORT_CONVOLUTION);
    if (!s)
        s = check_f32(ctx, projection);
    if (!s)
        s = check_f32(ctx, kernel);
    if (!s)
        s = check_f32(ctx, history);
    if (s)
        return s;
    if (projection->rank != 2 || projection->dims[1] != uint64_t(hidden) * 3)
        return fail(ctx, MFH_INVALID_SHAPE,
                    "short convolution projection must be [tokens, 3 * hidden]");
    const uint64_t tokens = projection->dims[0];
    uint64_t out_dims[2] = {tokens, hidden};
    if ((s = check_output(ctx, output, out_dims, 2)))
        return s;
    if (kernel->rank != 2 || kernel->dims[0] != hidden || kernel->dims[1] != width)
        return fail(ctx, MFH_INVALID_SHAPE, "short convolution kernel must be [hidden, width]");
    if (history->rank != 2 || history->dims[0] != uint64_t(width) - 1 ||
        history->dims[1] != hidden)
        return fail(ctx, MFH_INVALID_SHAPE,
                    "short convolution history must be [width - 1, hidden]");
    if (aliases(output, {projection, kernel, history}) ||
        aliases(history, {projection, kernel}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    mark_written(history);
    launch_short_conv(ctx->stream, dev_f32(output), dev_f32(projection), dev_f32(kernel),
                      dev_f32(history), tokens, hidden, width);
    return launched(ctx);
}

mfh_status mfh_swiglu(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *gate, const mfh_buf *up)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    mfh_status s = check_operation(ctx, MFH_OP_SWIGLU);
    if (!s)
        s = check_f32(ctx, gate);
    if (!s)
        s = check_f32(ctx, up);
    if (s)
        return s;
    if (!same_shape(gate, up))
        return fail(ctx, MFH_INVALID_SHAPE, "SwiGLU gate and up layouts differ");
    if ((s = check_output(ctx, output, gate->dims, gate->rank)))
        return s;
    if (aliases(output, {gate, up}))
        return fail(ctx, MFH_INVALID_ARGUMENT, "output aliases an input");
    DeviceGuard guard(ctx->device);
    mark_written(output);
    launch_swiglu(ctx->stream, dev_f32(output), dev_f32(gate), dev_f32(up),
                  size_t(gate->elements));
    return launched(ctx);
}

}  // extern "C"
