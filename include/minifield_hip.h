/*
 * minifield_hip.h - C ABI of the MI355X (gfx950) backend for Minifield's
 * packed-weight matmul path.
 *
 * The ABI mirrors the `InferenceOps` trait of the reference
 * (crates/engine-api/src/inference.rs:33-425) one entry point per trait
 * method, with the same operand order.  A Rust `crates/backend-hip` binds
 * these symbols one-to-one from an `extern "C"` block.  Every entry point
 * takes plain pointers, sizes and opaque handles; no C++ or torch types cross
 * the boundary.
 *
 * Threading: one context is single-threaded and cooperative, like the
 * reference's `Rc`/`RefCell` backends (engine-api/src/resources.rs:90-99).
 * All device work of one context is ordered on one HIP stream.
 *
 * Errors: every fallible call returns `mfh_status`, whose non-zero values map
 * 1:1 onto `ExecutorError` (engine-api/src/error.rs:10-28).  The static
 * message of the most recent failure is available from `mfh_last_error`.
 * Operations validate every operand before enqueueing anything, so a rejected
 * call leaves every output untouched
 * (backend-cpu/tests/packed_pair_validation.rs:57-92).
 */
#ifndef MINIFIELD_HIP_H
#define MINIFIELD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ExecutorError variants, engine-api/src/error.rs:10-28, in declaration order. */
typedef enum mfh_status {
    MFH_OK = 0,
    MFH_INVALID_ARGUMENT = 1,
    MFH_INVALID_SHAPE = 2,
    MFH_INVALID_LAYOUT = 3,
    MFH_INVALID_DTYPE = 4,
    MFH_OVERFLOW = 5,
    MFH_OUT_OF_BOUNDS = 6,
    MFH_UNSUPPORTED = 7,
    MFH_RESOURCE_LIMIT = 8,
    MFH_WRONG_BACKEND = 9,
    MFH_STALE_BUFFER = 10,
    MFH_DUPLICATE_NAME = 11,
    MFH_MISSING_REQUIRED_TENSOR = 12,
    MFH_UNEXPECTED_TENSOR = 13,
    MFH_INVALID_TIE = 14,
    MFH_CANCELLED = 15,
    MFH_COMPLETION_CONSUMED = 16,
    MFH_BACKEND_FAILURE = 17
} mfh_status;

/* AllocationClass, engine-api/src/resources.rs:19-24. */
typedef enum mfh_alloc_class {
    MFH_CLASS_WEIGHT = 0,
    MFH_CLASS_CACHE = 1,
    MFH_CLASS_SCRATCH = 2,
    MFH_CLASS_BRANCH = 3
} mfh_alloc_class;

/* DType subset the backend stores (engine-api/src/tensor.rs). */
typedef enum mfh_dtype {
    MFH_DTYPE_F32 = 0,
    MFH_DTYPE_U8 = 1
} mfh_dtype;

/* OperationKind bit positions, engine-api/src/backend.rs:76-99 (repr(u8)). */
typedef enum mfh_operation {
    MFH_OP_COPY = 0,
    MFH_OP_RECT_COPY_2D = 1,
    MFH_OP_GATHER_ROWS = 2,
    MFH_OP_ADD = 3,
    MFH_OP_MULTIPLY = 4,
    MFH_OP_LINEAR = 5,
    MFH_OP_ROW_RMS_NORM = 6,
    MFH_OP_EMBEDDING = 7,
    MFH_OP_ROTARY = 8,
    MFH_OP_GROUPED_QUERY_ATTENTION = 9,
    MFH_OP_GATED_SHORT_CONVOLUTION = 10,
    MFH_OP_SWIGLU = 11,
    MFH_OP_LM_PROJECTION = 12,
    MFH_OP_PACKED_GATHER_ROWS = 13,
    MFH_OP_PACKED_LINEAR = 14,
    MFH_OP_ADD_ROW_RMS_NORM = 15,
    MFH_OP_PACKED_LINEAR_PAIR = 16,
    MFH_OP_PACKED_SWIGLU_LINEAR = 17,
    MFH_OP_PACKED_SWIGLU_PAIR = 18,
    MFH_OP_QK_NORM_ROPE = 19,
    MFH_OP_ARGMAX = 20,
    MFH_OP_GATHER_COLUMNS = 21
} mfh_operation;

/* ResourceLimits, engine-api/src/resources.rs:7-11. */
typedef struct mfh_limits {
    uint64_t max_allocation_bytes;
    uint64_t max_total_bytes;
    uint32_t max_pending_operations;
} mfh_limits;

/* BackendIdentity, engine-api/src/backend.rs:18-24.  `kind` is
 * BackendKind::Other(0x4850) ("HP"): the reference enum has no HIP variant. */
typedef struct mfh_backend_identity {
    uint32_t kind;
    uint32_t ordinal;
    uint64_t owner;
    uint64_t generation;
} mfh_backend_identity;

#define MFH_BACKEND_KIND_HIP 0x4850u

/* BackendCapabilities, engine-api/src/backend.rs:385-395. */
typedef struct mfh_backend_capabilities {
    uint32_t dtypes;          /* bit (1 << mfh_dtype) per supported dtype */
    uint64_t operations;      /* bit (1 << mfh_operation) per operation   */
    uint32_t max_rank;
    uint64_t max_elements;
    uint64_t max_allocation_bytes;
    uint32_t supports_nonblocking_completion;
} mfh_backend_capabilities;

/* ResourceReport, engine-api/src/resources.rs:47-54. */
typedef struct mfh_report {
    uint64_t resident_weight_bytes;
    uint64_t cache_bytes;
    uint64_t scratch_bytes;
    uint64_t staged_branch_bytes;
    uint64_t pending_operation_bytes;
    uint32_t pending_operations;
} mfh_report;

typedef struct mfh_ctx mfh_ctx;
typedef struct mfh_buf mfh_buf;
typedef struct mfh_fence mfh_fence;
typedef struct mfh_readback mfh_readback;

/* ---- context lifetime ------------------------------------------------- */

/* Create one backend instance on HIP device `ordinal`.  Replaces the
 * backend constructor, e.g. CpuBackend::new (backend-cpu/src/storage.rs:145). */
mfh_status mfh_create(uint32_t ordinal, uint64_t owner, const mfh_limits *limits,
                      mfh_ctx **out);
/* Drop the instance: waits for queued work, frees every device allocation.
 * Buffers of this context must not be used afterwards. */
void mfh_destroy(mfh_ctx *ctx);

/* Static message of the last failed call on `ctx` (never NULL). */
const char *mfh_last_error(const mfh_ctx *ctx);
/* Static message of a status code, ExecutorError's Display (error.rs:30-53). */
const char *mfh_status_message(mfh_status status);

/* InferenceOps::identity (inference.rs:39). */
mfh_status mfh_identity(const mfh_ctx *ctx, mfh_backend_identity *out);
/* InferenceOps::capabilities (inference.rs:47). */
mfh_status mfh_capabilities(const mfh_ctx *ctx, mfh_backend_capabilities *out);
/* InferenceOps::resource_report (inference.rs:48).  Counts physical bytes,
 * like the reference's wgpu backend (backend-wgpu/src/lib.rs:340-370): the
 * byte extent of each live buffer and of its backend-private derived copies
 * (the binary16 scale shadow, repacked code tiles, tiled scales) under the
 * buffer's class; the rest of the device memory the context holds (pool
 * bucket slack, context scratch, idle pooled blocks) under scratch; pinned
 * staging of unpolled readbacks as pending bytes.  The sum is the context's
 * device footprint plus that staging, and every allocation that would take
 * it past max_total_bytes fails with MFH_RESOURCE_LIMIT. */
mfh_status mfh_resource_report(const mfh_ctx *ctx, mfh_report *out);
/* InferenceOps::peak_accounted_bytes (inference.rs:52-56): the highest
 * such total since mfh_create. */
mfh_status mfh_peak_accounted_bytes(const mfh_ctx *ctx, uint64_t *out);
/* InferenceOps::advance_generation (inference.rs:57): older buffers then
 * fail with MFH_STALE_BUFFER (backend-cpu/src/storage.rs:258-267). */
mfh_status mfh_advance_generation(mfh_ctx *ctx);
/* CpuBackend::request_cancel / clear_cancel (backend-cpu/src/storage.rs:269-275). */
mfh_status mfh_request_cancel(mfh_ctx *ctx);
mfh_status mfh_clear_cancel(mfh_ctx *ctx);
/* InferenceOps::poll_retired_fences (inference.rs:46). */
mfh_status mfh_poll_retired_fences(mfh_ctx *ctx);

/* ---- buffers ---------------------------------------------------------- */

/* InferenceOps::allocate_f32_classified (inference.rs:60-64) when `zeroed`
 * is 1, allocate_f32_uninit (inference.rs:93-99) when 0. */
mfh_status mfh_alloc_f32(mfh_ctx *ctx, const uint64_t *dims, uint32_t rank,
                         mfh_alloc_class cls, int zeroed, mfh_buf **out);
/* InferenceOps::upload_f32_classified (inference.rs:67-72). `count` must
 * equal the element count of `dims`. */
mfh_status mfh_upload_f32(mfh_ctx *ctx, const uint64_t *dims, uint32_t rank,
                          const float *values, size_t count, mfh_alloc_class cls,
                          mfh_buf **out);
/* InferenceOps::upload_u8_classified (inference.rs:77-82). */
mfh_status mfh_upload_u8(mfh_ctx *ctx, const uint64_t *dims, uint32_t rank,
                         const uint8_t *bytes, size_t count, mfh_alloc_class cls,
                         mfh_buf **out);
/* Drop a buffer handle.  Device memory returns to the context's pool in
 * stream order, so work already queued against it completes first
 * (inference.rs:27-30). */
void mfh_release(mfh_buf *buf);
/* Descriptor queries: dtype, rank and dims (dims has room for 4). */
mfh_status mfh_buf_desc(const mfh_buf *buf, mfh_dtype *dtype, uint32_t *rank,
                        uint64_t *dims);

/* ---- completions (engine-api/src/resources.rs:84-99) ------------------- */

/* InferenceOps::fence (inference.rs:107). */
mfh_status mfh_fence_submit(mfh_ctx *ctx, mfh_fence **out);
/* InferenceCompletion::poll_step: *ready = 0 while pending; once ready the
 * return value is the completion's result. */
mfh_status mfh_fence_poll(mfh_fence *fence, int *ready);
/* InferenceCompletion::cancel. */
mfh_status mfh_fence_cancel(mfh_fence *fence);
void mfh_fence_free(mfh_fence *fence);

/* InferenceOps::read_f32_async (inference.rs:111). */
mfh_status mfh_read_f32_async(mfh_ctx *ctx, const mfh_buf *buf, mfh_readback **out);
/* Poll a readback. When ready, copies min(capacity, n) values into `dst`,
 * stores n in *count, and the completion is consumed: a second ready poll
 * returns MFH_COMPLETION_CONSUMED. */
mfh_status mfh_readback_poll(mfh_readback *rb, int *ready, float *dst, size_t capacity,
                             size_t *count);
mfh_status mfh_readback_cancel(mfh_readback *rb);
void mfh_readback_free(mfh_readback *rb);

/* Block until every queued operation of `ctx` finished (host convenience for
 * tests and benches; the executor path only polls fences). */
mfh_status mfh_synchronize(mfh_ctx *ctx);

/* ---- packed-weight operations (the hot path) --------------------------- */
/*
 * `codes` is a U8 [R, K/wpb] buffer and `scales` an F32 [R, K/128] buffer.
 * K comes from the scales width; the codes width selects the format:
 * K/4 = minifield.ternary.v1, K/2 = minifield.nf4.v1, K = signed INT8
 * (backend-cpu/src/packed.rs:177-220).  INT8 streams containing the
 * reserved byte 0x80 are rejected with MFH_INVALID_ARGUMENT; the scan runs
 * once at upload and is cached on the buffer.
 *
 * Token ids: pass `host_ids`/`host_count` for TokenIds::Host or
 * `device_ids` (an F32 rank-1 buffer) for TokenIds::Device, never both
 * (inference.rs:19-23).
 */

/* InferenceOps::packed_gather_rows (inference.rs:180-186). */
mfh_status mfh_packed_gather_rows(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *codes,
                                  const mfh_buf *scales, const uint32_t *host_ids,
                                  size_t host_count, const mfh_buf *device_ids);
/* InferenceOps::packed_linear (inference.rs:194-200). */
mfh_status mfh_packed_linear(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                             const mfh_buf *codes, const mfh_buf *scales);
/* InferenceOps::packed_linear_pair (inference.rs:209-218). */
mfh_status mfh_packed_linear_pair(mfh_ctx *ctx, mfh_buf *out_a, mfh_buf *out_b,
                                  const mfh_buf *input, const mfh_buf *codes_a,
                                  const mfh_buf *scales_a, const mfh_buf *codes_b,
                                  const mfh_buf *scales_b);
/* InferenceOps::packed_swiglu_linear (inference.rs:226-233). */
mfh_status mfh_packed_swiglu_linear(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *gate,
                                    const mfh_buf *up, const mfh_buf *codes,
                                    const mfh_buf *scales);
/* InferenceOps::packed_swiglu_pair (inference.rs:244-252). */
mfh_status mfh_packed_swiglu_pair(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                                  const mfh_buf *codes_a, const mfh_buf *scales_a,
                                  const mfh_buf *codes_b, const mfh_buf *scales_b);
/* Build the backend-private copies the matrix-core kernels read for this
 * (codes, scales) pair now: codes repacked into the tile layout of the format
 * the widths select and scales in tile order, charged to the buffers'
 * allocation classes.  Admission is packed_linear's (format, row count,
 * INT8 reserved code).  A loader calls it after uploading each packed weight
 * so that a ResourceLimit surfaces at load, the way the reference funds its
 * LUT2 repack at construction (executor-core/src/lfm2/executor/
 * construction.rs:404-424).  Without it the first packed operation on the
 * pair builds the copies, under the same accounting and limits, before
 * enqueueing anything else.  Idempotent. */
mfh_status mfh_prepare_packed(mfh_ctx *ctx, const mfh_buf *codes, const mfh_buf *scales);
/* 1 when the pair's copies exist for the format its widths select, else 0. */
int mfh_packed_prepared(const mfh_ctx *ctx, const mfh_buf *codes, const mfh_buf *scales);
/* InferenceOps::supports_ternary_lut2 (inference.rs:259-261).  Always 0:
 * the backend's private repack (mfh_prepare_packed) replaces LUT2, so the
 * *_lut2 hooks report MFH_UNSUPPORTED like the trait defaults
 * (inference.rs:268-309). */
int mfh_supports_ternary_lut2(const mfh_ctx *ctx);

/* No counterpart in the reference.  packed_linear for callers that cannot
 * allocate device memory (code under stream capture, serving loops,
 * harnesses that forbid hipMalloc): the same matrix-core decode GEMV as
 * mfh_packed_linear, with the same admission and result bits, but its
 * activation scratch is a fixed array of about 532 KiB that each GPU holds
 * for the life of the process, so the call performs no device allocation.
 * Serves input rows <= 8 and widths K <= 16384 (MFH_RESOURCE_LIMIT beyond
 * it), on weights already prepared with mfh_prepare_packed (MFH_UNSUPPORTED
 * otherwise, and on kernel path 1).  All calls on one GPU share the array:
 * calls whose work overlaps on one GPU (several contexts or threads) race. */
mfh_status mfh_packed_linear_noalloc(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                                     const mfh_buf *codes, const mfh_buf *scales);

/* ---- dense LFM2 operations (the rest of a forward pass) ---------------- */
/*
 * Same operand order as the trait.  Spec structs of the reference
 * (PackedHeadSpec, RotarySpec, GqaSpec, GatedShortConvSpec, RectCopy2d;
 * engine-api/src/backend.rs:120-380) are passed as their scalar fields and
 * validated with the same rules and messages.
 */

/* InferenceOps::copy (inference.rs:113). */
mfh_status mfh_copy(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input);
/* InferenceOps::copy_rect_2d (inference.rs:118-123), RectCopy2d fields. */
mfh_status mfh_copy_rect_2d(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                            uint64_t source_row, uint64_t source_column,
                            uint64_t destination_row, uint64_t destination_column,
                            uint64_t rows, uint64_t columns);
/* InferenceOps::argmax (inference.rs:131): first strict maximum per row as an
 * exact f32 index, NaN for a row holding any non-finite value. */
mfh_status mfh_argmax(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input);
/* InferenceOps::argmax_masked (inference.rs:140-149): `mask` holds
 * ceil(width / 64) u64 words, bit i % 64 of word i / 64 admits column i. */
mfh_status mfh_argmax_masked(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                             const uint64_t *mask, size_t mask_words);
/* InferenceOps::gather_rows (inference.rs:151-156); token ids as for
 * mfh_packed_gather_rows. */
mfh_status mfh_gather_rows(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *table,
                           const uint32_t *host_ids, size_t host_count,
                           const mfh_buf *device_ids);
/* InferenceOps::gather_columns (inference.rs:166-171). */
mfh_status mfh_gather_columns(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                              const uint32_t *columns, size_t count);
/* InferenceOps::add / multiply (inference.rs:346-357). */
mfh_status mfh_add(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *left, const mfh_buf *right);
mfh_status mfh_multiply(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *left,
                        const mfh_buf *right);
/* InferenceOps::linear (inference.rs:358-363): dense f32 X[M,K] * W[N,K]^T. */
mfh_status mfh_linear(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                      const mfh_buf *weight);
/* InferenceOps::row_rms_norm (inference.rs:364-370). */
mfh_status mfh_row_rms_norm(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                            const mfh_buf *weight, float epsilon);
/* InferenceOps::head_rms_norm (inference.rs:373-380), PackedHeadSpec fields. */
mfh_status mfh_head_rms_norm(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                             const mfh_buf *weight, uint32_t heads, uint32_t head_dim,
                             float epsilon);
/* InferenceOps::split_half_rotary (inference.rs:383-389), RotarySpec fields. */
mfh_status mfh_split_half_rotary(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                                 const uint64_t *positions, size_t position_count,
                                 uint32_t heads, uint32_t head_dim, float theta);
/* InferenceOps::add_row_rms_norm (inference.rs:316-324). */
mfh_status mfh_add_row_rms_norm(mfh_ctx *ctx, mfh_buf *sum, mfh_buf *normed,
                                const mfh_buf *left, const mfh_buf *right,
                                const mfh_buf *weight, float epsilon);
/* InferenceOps::qk_norm_rope (inference.rs:333-345): RotarySpec (query heads,
 * head_dim, theta) and the key/value PackedHeadSpec. */
mfh_status mfh_qk_norm_rope(mfh_ctx *ctx, mfh_buf *query_out, mfh_buf *key_out,
                            const mfh_buf *query, const mfh_buf *key,
                            const mfh_buf *query_weight, const mfh_buf *key_weight,
                            const uint64_t *positions, size_t position_count,
                            uint32_t query_heads, uint32_t head_dim, float theta,
                            uint32_t key_value_heads, uint32_t key_value_head_dim,
                            float epsilon);
/* InferenceOps::causal_gqa (inference.rs:394-404), GqaSpec fields.  The new
 * K/V rows are appended at [*cache_len, *cache_len + tokens) and *cache_len
 * advances only after every check passed. */
mfh_status mfh_causal_gqa(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *query,
                          const mfh_buf *key, const mfh_buf *value, mfh_buf *key_cache,
                          mfh_buf *value_cache, uint64_t *cache_len, uint32_t query_heads,
                          uint32_t key_value_heads, uint32_t head_dim);
/* InferenceOps::gated_short_convolution (inference.rs:409-416),
 * GatedShortConvSpec fields. */
mfh_status mfh_gated_short_convolution(mfh_ctx *ctx, mfh_buf *output,
                                       const mfh_buf *projection, const mfh_buf *kernel,
                                       mfh_buf *history, uint32_t hidden, uint32_t width);
/* InferenceOps::swiglu (inference.rs:419-424). */
mfh_status mfh_swiglu(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *gate, const mfh_buf *up);

/* ---- diagnostics (no counterpart in the reference) --------------------- */

/* The HIP stream (hipStream_t) all work of `ctx` is ordered on, so a caller
 * can bracket launches with its own HIP events. */
void *mfh_stream(const mfh_ctx *ctx);
/* Kernel path for packed GEMV/GEMM: 0 = automatic selection, 1 = FP32 FMA
 * kernels only, 2 = automatic but with the matrix-core GEMV's activation
 * prologue run as a kernel of its own, 3 = automatic kernels, with the LFM2
 * one-token pass issued op by op through these entry points instead of the
 * fused decode step.  Returns the previous setting. */
int mfh_set_kernel_path(mfh_ctx *ctx, int path);
/* Activation precision of the matrix-core prefill GEMM (m > 8): 0 (the
 * default) = each activation as binary16 hi + lo halves, two MFMAs per
 * product (three for NF4), 22 significant bits; 1 = one binary16 half, one
 * MFMA per product (two for NF4), each activation within 2^-12 of itself.
 * Weights, scales and the group epilogue are the same in both.  Any other
 * value selects 0.  Returns the previous setting (-1 for a null context). */
int mfh_set_gemm_activations(mfh_ctx *ctx, int mode);

#ifdef __cplusplus
}
#endif

#endif /* MINIFIELD_HIP_H */
