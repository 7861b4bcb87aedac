// Launch interface between the host admission code and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "internal.hpp"

namespace mfh {

// One packed weight stream as the kernels see it.
struct PackedStream {
    const uint8_t *codes = nullptr;      // canonical [n, k / wpb] row-major codes
    const float *scales = nullptr;       // f32 [n, k / 128]
    const uint16_t *scales16 = nullptr;  // binary16 copy of `scales`, or null
    const uint8_t *tiles = nullptr;      // backend-private repacked codes, or null
    const void *tiled_scales = nullptr;  // scales in tile order, or null
    bool tiled_half = false;             // tiled_scales holds binary16 values
};

enum class Epilogue : int {
    Single = 0,     // out_a = x . a
    Pair = 1,       // out_a = x . a, out_b = x . b
    SwigluPair = 2, // out_a = silu(x . a) * (x . b)
};

// How the matrix-core GEMV's activation prologue forms x as it reads it, so
// that the producing elementwise step needs no kernel of its own (decode).
enum class XKind : uint32_t {
    Plain = 0,   // x = a
    AddRms = 1,  // s = a + b (b may be null); x = (s * rsqrt(mean(s^2) + eps)) * w
    Swiglu = 2,  // x = silu(a) * b
    // x = one decode token's attention output merged from its key ranges:
    // a holds launch_gqa_decode's (m, l, acc[head_dim]) records, `ranges`
    // per head (gqa_combine_kernel's formula, summed in range order).
    GqaMerge = 3,
};
struct XForm {
    XKind kind = XKind::Plain;
    const float *a = nullptr;  // Plain x; AddRms left; Swiglu gate; GqaMerge records
    const float *b = nullptr;  // AddRms right; Swiglu up
    const float *w = nullptr;  // AddRms norm weight [k]
    float *side = nullptr;     // AddRms: s [m, k] (may be null)
    float epsilon = 0.0f;
    uint32_t ranges = 0, head_dim = 0;  // GqaMerge
};
// Most key ranges per head a GqaMerge prologue reads (each lane merges its
// head's records itself; more ranges keep the separate combine launch).
constexpr uint32_t kGqaMergeMaxRanges = 8;

constexpr uint32_t kMaxSegments = 3;

// Greedy selection's (value, index) candidate: index UINT32_MAX admits no
// value; `poisoned` marks a non-finite value seen.  Candidates merge keeping
// the largest value, the lowest index among equal values and any poison,
// so the order of the merges does not change the result.
struct Candidate {
    float value;
    uint32_t index;
    int poisoned;
};

// Whether candidate (ov, oi) replaces (best, index).
__device__ __forceinline__ bool takes(float ov, uint32_t oi, float best, uint32_t index)
{
    return oi != UINT32_MAX && (index == UINT32_MAX || ov > best || (ov == best && oi < index));
}

__device__ __forceinline__ void merge(Candidate &c, float ov, uint32_t oi, int op)
{
    c.poisoned |= op;
    if (takes(ov, oi, c.value, c.index)) {
        c.value = ov;
        c.index = oi;
    }
}

struct PackedCall {
    Format format = Format::Ternary;
    Epilogue epilogue = Epilogue::Single;
    uint32_t m = 0;  // activation rows
    uint32_t n = 0;  // weight rows (outputs per activation row)
    uint32_t k = 0;  // inner width, multiple of 128
    const float *x = nullptr;  // [m, k]
    PackedStream a, b;
    float *out_a = nullptr;  // [m, n]
    float *out_b = nullptr;  // [m, n] (Pair only)
    // Matrix-core GEMV: run the activation prologue as its own kernel even
    // where the in-kernel one fits (diagnostics).
    bool separate_prologue = false;
    // Matrix-core GEMM: activations as one binary16 half instead of hi + lo.
    bool single_half = false;
    // Matrix-core GEMV only: a transform other than Plain replaces `x`.
    XForm xform;
    // Matrix-core GEMV, Single epilogue only: when non-zero, the launch
    // runs `segments` weight streams of one format and width k over the
    // same activations, seg[i] (seg_n[i] rows) into seg_out[i]; a, n and
    // out_a are unused.  The scale halves of all segments must agree.
    uint32_t segments = 0;
    PackedStream seg[kMaxSegments];
    float *seg_out[kMaxSegments] = {};
    uint32_t seg_n[kMaxSegments] = {};
    // One-row products: where the launch's plan can (the one-row wide
    // kernel), each block also writes the greedy-selection candidate of its
    // outputs to argmax[block] and the launch stores the block count in
    // *argmax_count (left unchanged otherwise; the caller zeroes it).
    Candidate *argmax = nullptr;
    uint32_t *argmax_count = nullptr;
};

// One token of the gated short convolution (conv_step_kernel's arithmetic),
// finished by the convolution in-projection's vector GEMV from its own
// output rows: u = B * x (rows c and 2h + c), the causal taps over the
// history and u, times C (row h + c); the history rolls into `next`.
struct ConvStep {
    const float *kernel = nullptr;   // [hidden, width], oldest tap first
    const float *history = nullptr;  // [width - 1, hidden]
    float *next = nullptr;           // [width - 1, hidden]
    float *out = nullptr;            // [hidden]
    uint32_t hidden = 0, width = 0;
};

// packed_linear's admission (backend-cpu/src/packed.rs:96-140 order and
// messages): fills `call` for the plain product; enqueues nothing.
mfh_status admit_packed_linear(mfh_ctx *ctx, mfh_buf *output, const mfh_buf *input,
                               const mfh_buf *codes, const mfh_buf *scales, PackedCall *call);
// Whether the pair already holds its tile copies for `format`; fills the
// stream's tile fields when it does.
bool prepared_stream(const mfh_buf *codes, const mfh_buf *scales, Format format,
                     PackedStream *stream);

// A matrix-core GEMV (m <= 2) whose activation prologue
// applies `xform`, over admitted weights of n rows and width k (the LFM2
// decode step).  Fails with MFH_UNSUPPORTED where that kernel does not serve
// the call, before anything is enqueued.  `argmax` / `argmax_count`: see
// PackedCall.
mfh_status packed_xform(mfh_ctx *ctx, Epilogue epilogue, const XForm &xform, uint32_t m,
                        uint32_t n, uint32_t k, const mfh_buf *codes_a, const mfh_buf *scales_a,
                        const mfh_buf *codes_b, const mfh_buf *scales_b, float *out_a,
                        float *out_b, Candidate *argmax = nullptr,
                        uint32_t *argmax_count = nullptr);
// Whether the one-row wide kernel serves `call` with its GqaMerge prologue
// (the only kernel that reads that transform).
bool gqa_merge_supported(const PackedCall &call);
// Whether a one-row product of n x k weights in format f at the head size
// takes the add + RMS norm and the argmax candidates in its one launch
// (the one-row wide kernel).
bool head_fold_supported(Format f, uint32_t n, uint32_t k);

// The decode step's convolution block input: the in-projection of `codes`
// (3 * conv.hidden rows of width k) over add + RMS norm activations with
// the one-token convolution folded into its epilogue (try_wide_conv where
// it applies, else try_vgemv_conv).
// MFH_UNSUPPORTED, before anything is enqueued, where it does not apply.
mfh_status packed_xform_conv(mfh_ctx *ctx, const XForm &xform, uint32_t k,
                             const mfh_buf *codes, const mfh_buf *scales, const ConvStep &conv);

// Like packed_xform with the Single epilogue, over `count` weight streams of
// one format and width k in one launch (the LFM2 q/k/v projections).
mfh_status packed_xform_segments(mfh_ctx *ctx, const XForm &xform, uint32_t m, uint32_t k,
                                 uint32_t count, const mfh_buf *const *codes,
                                 const mfh_buf *const *scales, const uint32_t *n,
                                 float *const *out);

// Decode GEMV for m <= 8 on FP32 FMA units.
void launch_gemv_fma(hipStream_t stream, const PackedCall &call);
// f32 vector GEMV for wide contractions (one plain activation row, 4096 <=
// k <= 8192, n <= 8192, one stream, canonical codes): enqueues it and
// returns true, or returns false (nothing enqueued) where it does not serve
// the call.  The matrix-core GEMV tries it first.
bool try_vgemv(hipStream_t stream, const PackedCall &call);

// The in-projection (3 * hidden rows, add + RMS norm activations, one row)
// with the convolution folded in; false, with nothing enqueued, where the
// vector GEMV does not serve the call.
bool try_vgemv_conv(hipStream_t stream, const PackedCall &call, const ConvStep &conv);
// The same on the one-row wide matrix-core kernel (packed_mfma.hip), which
// reads the repacked tiles: whether it applies (checked before the tiles
// are prepared), and the launch (false where it does not apply or the
// tiles are missing).
bool wide_conv_supported(const PackedCall &call, const ConvStep &conv);
bool try_wide_conv(hipStream_t stream, const PackedCall &call, const ConvStep &conv);
// Matrix-core decode GEMV for m <= 8 (needs `tiles` and `tiled_scales` on
// every stream).  `scratch` holds gemv_mfma_scratch_bytes(call) bytes.
bool gemv_mfma_supported(Format format);
void launch_gemv_mfma(hipStream_t stream, const PackedCall &call, void *scratch);
size_t gemv_mfma_scratch_bytes(const PackedCall &call);
// Repack a canonical code stream into the private tile layout, and a scale
// stream into tile order (binary16 when `half`).
size_t repacked_bytes(Format format, uint32_t n, uint32_t k);
void launch_repack(hipStream_t stream, Format format, const uint8_t *codes, uint8_t *tiles,
                   uint32_t n, uint32_t k);
size_t tiled_scales_bytes(Format format, uint32_t n, uint32_t k, bool half);
void launch_tile_scales(hipStream_t stream, Format format, const float *scales, void *out,
                        uint32_t n, uint32_t k, bool half);

// Prefill GEMM for larger m: LDS-staged dequantized tiles with FP32 FMA.
void launch_gemm_fma(hipStream_t stream, const PackedCall &call);
// Prefill GEMM on matrix cores (binary16 hi/lo activations, exact weight
// levels, f32 group epilogue).  `scratch` holds gemm_mfma_scratch_bytes.
size_t gemm_mfma_scratch_bytes(const PackedCall &call);
void launch_gemm_mfma(hipStream_t stream, const PackedCall &call, void *scratch);

// out[i] = the binary16 value bits[i] as f32 (exact).
void launch_f16_to_f32(hipStream_t stream, float *out, const uint16_t *bits, size_t count);

// out[i] = silu(gate[i]) * up[i], the reference's SwiGLU staging
// (backend-cpu/src/packed.rs:431-441).
void launch_swiglu(hipStream_t stream, float *out, const float *gate, const float *up,
                   size_t count);

// Dequantize selected rows.  `ids` are f32 row selectors (device ids or
// staged host ids); invalid or out-of-range ids produce a NaN row.
void launch_packed_gather(hipStream_t stream, Format format, float *out, const uint8_t *codes,
                          const float *scales, const float *ids, uint32_t count, uint32_t rows,
                          uint32_t k);

// ---- dense f32 operations (dense.hip) ----------------------------------

struct RectCopy {
    uint64_t source_width, destination_width;
    uint64_t source_row, source_column, destination_row, destination_column;
    uint64_t rows, columns;
};

// Attention over caches of [capacity, key_value_heads * head_dim] rows; the
// `tokens` new rows land at row `initial_len`.
struct GqaShape {
    uint64_t tokens = 0;
    uint64_t initial_len = 0;
    uint32_t query_heads = 0;
    uint32_t key_value_heads = 0;
    uint32_t head_dim = 0;
    uint32_t group = 0;
    float scale = 0.0f;
};
// Widest head the attention kernel serves: a 256-thread block gives each
// thread at most this many output dimensions.
constexpr int kMaxDimsPerThread = 4;
constexpr uint32_t kMaxGqaHeadDim = 256 * kMaxDimsPerThread;

void launch_copy(hipStream_t stream, float *dst, const float *src, size_t count);
void launch_rect_copy(hipStream_t stream, float *dst, const float *src, const RectCopy &rect);
// `ids` are f32 row selectors; invalid or out-of-range ids give a NaN row.
void launch_gather_rows(hipStream_t stream, float *out, const float *table, const float *ids,
                        uint32_t count, uint32_t rows, uint64_t columns);
void launch_gather_columns(hipStream_t stream, float *out, const float *in, const uint32_t *cols,
                           uint64_t rows, uint64_t width, uint32_t count);
// `mask` is null for the unmasked selector.  Few wide rows are scanned by
// several blocks per row whose candidates take argmax_scratch_bytes bytes of
// `scratch` (0: none used).
size_t argmax_scratch_bytes(uint32_t rows, uint32_t width);
// `copy`, when non-null, receives the selectors too.
void launch_argmax(hipStream_t stream, float *out, const float *in, uint32_t rows, uint32_t width,
                   const uint64_t *mask, void *scratch, float *copy = nullptr);
// The selector of one row from `count` candidates a product's blocks wrote
// (PackedCall::argmax): the same result as launch_argmax over that row.
void launch_argmax_candidates(hipStream_t stream, float *out, float *copy,
                              const Candidate *candidates, uint32_t count);
// op 0: left + right, op 1: left * right.
void launch_binary(hipStream_t stream, int op, float *out, const float *left, const float *right,
                   size_t count);
void launch_linear(hipStream_t stream, float *out, const float *x, const float *w, uint32_t m,
                   uint32_t n, uint32_t k);
// With `sum` non-null: sum = left + right, out = rms(sum); else out = rms(left).
void launch_row_rms(hipStream_t stream, float *out, float *sum, const float *left,
                    const float *right, const float *weight, uint64_t rows, uint32_t width,
                    float epsilon);
void launch_head_rms(hipStream_t stream, float *out, const float *in, const float *weight,
                     uint64_t segments, uint32_t head_dim, float epsilon);
// Per-token rotary positions: `staged` (one f32 per token, device memory) or,
// when null, the consecutive positions base, base + 1, ...
struct Positions {
    const float *staged = nullptr;
    uint64_t base = 0;
};
void launch_rotary(hipStream_t stream, float *out, const float *in, const Positions &positions,
                   uint64_t tokens, uint32_t heads, uint32_t head_dim, float theta);
// The same for the consecutive positions first .. first + tokens - 1, with
// the coefficients from a launch_rotation_table table (bit-identical).
void launch_qk_norm_rope_table(hipStream_t stream, float *query_out, float *key_out,
                               const float *query, const float *key, const float *query_weight,
                               const float *key_weight, const float *table, uint64_t first,
                               uint64_t tokens, uint32_t query_heads, uint32_t key_heads,
                               uint32_t head_dim, float epsilon);
void launch_qk_norm_rope(hipStream_t stream, float *query_out, float *key_out, const float *query,
                         const float *key, const float *query_weight, const float *key_weight,
                         const Positions &positions, uint64_t tokens, uint32_t query_heads,
                         uint32_t key_heads, uint32_t head_dim, float theta, float epsilon);
// Appends the new rows (unless `key` is null: the caller has already written
// them at row `initial_len` of both caches), then attends.  Few (token,
// head) pairs over long caches take a split-key path whose partials need
// gqa_scratch_bytes(g) bytes of `scratch` (0: no scratch used).
size_t gqa_scratch_bytes(const GqaShape &g);
void launch_gqa(hipStream_t stream, float *out, const float *query, const float *key,
                const float *value, float *key_cache, float *value_cache, const GqaShape &g,
                float *scratch);
// One decode token's qk_norm_rope + causal_gqa (no cache append for the
// value: its row `position` must already hold the new value), as two
// launches.  Writes the rotated key into the key cache row `position` and
// the attention output.  `partial` holds gqa_decode_scratch_bytes.
// gqa_decode_splits gives the key ranges to put in `splits`, or 0 when the
// shape is outside the kernel.
struct DecodeAttention {
    const float *query = nullptr;         // [query_heads * head_dim], raw
    const float *key = nullptr;           // [key_value_heads * head_dim], raw
    const float *query_weight = nullptr;  // [head_dim]
    const float *key_weight = nullptr;    // [head_dim]
    float *key_cache = nullptr, *value_cache = nullptr;
    float *partial = nullptr;
    const float *rotation = nullptr;      // launch_rotation_table rows, >= position + 1
    float *out = nullptr;                 // [query_heads * head_dim]
    uint64_t position = 0;                // the new token's row (= cache length before it)
    uint32_t query_heads = 0, key_value_heads = 0, head_dim = 0, group = 0, splits = 0;
    float theta = 0.0f, epsilon = 0.0f, scale = 0.0f;
};
// table[t * head_dim + c] = cos, table[t * head_dim + head_dim / 2 + c] =
// sin of the rotation of position t, column c < head_dim / 2, for
// t < positions: bit for bit what the rotary kernels compute inline.
void launch_rotation_table(hipStream_t stream, float *table, uint64_t positions,
                           uint32_t head_dim, float theta);
uint32_t gqa_decode_splits(const DecodeAttention &p);
size_t gqa_decode_scratch_bytes(const DecodeAttention &p);
// `combine` false: the key ranges' records only, for a GqaMerge prologue
// (launch_gqa_combine merges them into p.out later if that prologue does
// not serve the projection).
void launch_gqa_decode(hipStream_t stream, const DecodeAttention &p, bool combine = true);
void launch_gqa_combine(hipStream_t stream, const DecodeAttention &p);
void launch_short_conv(hipStream_t stream, float *out, const float *projection,
                       const float *kernel, float *history, uint64_t tokens, uint32_t hidden,
                       uint32_t width);
// One decode token; the rolled history goes to `next` (width >= 1).
void launch_conv_step(hipStream_t stream, float *out, const float *projection,
                      const float *kernel, const float *history, float *next, uint32_t hidden,
                      uint32_t width);

}  // namespace mfh
