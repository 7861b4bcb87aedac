// Dense f32 kernels of the LFM2 forward pass: copies, gathers, element-wise
// arithmetic, row selectors, RMS normalisation, split-half rotary, causal
// grouped-query attention and the gated short convolution.
//
// Arithmetic follows the reference's scalar f32 code
// (crates/backend-cpu/src/{dense,normalization_rotary,attention_convolution}.rs):
// contraction is off, so every product and sum rounds where the reference's
// does.  Reductions the reference runs sequentially (sums of squares, softmax
// denominators, attention-weighted sums) run here as fixed-shape trees, so
// results are deterministic run to run and agree with the reference within
// f32 reassociation error.  The per-row attention kernels keep the
// reference's sequential dot order per key, so their scores are
// bit-identical to it; the prefill kernel on fp32 matrix cores sums each
// score in matrix-core order and takes the online softmax form, also
// within f32 reassociation error.
//
// Unlike the reference's CPU backend, a non-finite intermediate does not
// raise an error: device work is deferred, so NaN/Inf propagate to the
// outputs (argmax turns them into its NaN marker), as on the reference's
// device backends.
#pragma clang fp contract(off)

#include "kernels.hpp"

namespace mfh {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        v += __shfl_xor(v, offset, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        v = fmaxf(v, __shfl_xor(v, offset, 64));
    return v;
}

// Block-wide sum of a kBlock-thread block, the same value returned to every
// thread.  `scratch` holds kBlock / 64 floats.
__device__ __forceinline__ float block_sum(float v, float *scratch)
{
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0)
        scratch[wave] = v;
    __syncthreads();
    float total = scratch[0];
#pragma unroll
    for (int w = 1; w < kBlock / 64; ++w)
        total += scratch[w];
    return total;
}

__device__ __forceinline__ float block_max(float v, float *scratch)
{
    v = wave_max(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0)
        scratch[wave] = v;
    __syncthreads();
    float best = scratch[0];
#pragma unroll
    for (int w = 1; w < kBlock / 64; ++w)
        best = fmaxf(best, scratch[w]);
    return best;
}

unsigned grid_for(size_t count, size_t per_block = kBlock)
{
    size_t blocks = (count + per_block - 1) / per_block;
    return unsigned(blocks < 65536 * 4 ? (blocks ? blocks : 1) : 65536 * 4);
}

// ---- copies ------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void copy_kernel(float *__restrict__ dst,
                                                      const float *__restrict__ src, size_t count)
{
    // Buffers start on pool blocks (256-byte aligned): move float4s, then
    // the tail.
    const size_t quads = count / 4;
    const size_t stride = size_t(gridDim.x) * kBlock;
    for (size_t i = size_t(blockIdx.x) * kBlock + threadIdx.x; i < quads; i += stride)
        reinterpret_cast<float4 *>(dst)[i] = reinterpret_cast<const float4 *>(src)[i];
    for (size_t i = quads * 4 + size_t(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride)
        dst[i] = src[i];
}

__global__ __launch_bounds__(kBlock) void rect_copy_kernel(float *__restrict__ dst,
                                                           const float *__restrict__ src,
                                                           RectCopy rect)
{
    for (uint64_t row = blockIdx.x; row < rect.rows; row += gridDim.x) {
        const float *s = src + (rect.source_row + row) * rect.source_width + rect.source_column;
        float *d = dst + (rect.destination_row + row) * rect.destination_width +
                   rect.destination_column;
        for (uint64_t c = threadIdx.x; c < rect.columns; c += kBlock)
            d[c] = s[c];
    }
}

// ---- selectors ---------------------------------------------------------

// A device row selector is valid when finite, integral and in [0, 2^24)
// (backend-cpu/src/dense.rs:24-53) and, for a table, below its row count.
__device__ __forceinline__ bool valid_row(float id, uint32_t rows)
{
    return isfinite(id) && id >= 0.0f && truncf(id) == id && id < 16777216.0f &&
           uint32_t(id) < rows;
}

__global__ __launch_bounds__(kBlock) void gather_rows_kernel(float *__restrict__ out,
                                                             const float *__restrict__ table,
                                                             const float *__restrict__ ids,
                                                             uint32_t count, uint32_t rows,
                                                             uint64_t columns)
{
    for (uint32_t r = blockIdx.x; r < count; r += gridDim.x) {
        const float id = ids[r];
        float *dst = out + uint64_t(r) * columns;
        if (valid_row(id, rows)) {
            const float *src = table + uint64_t(uint32_t(id)) * columns;
            for (uint64_t c = threadIdx.x; c < columns; c += kBlock)
                dst[c] = src[c];
        } else {
            for (uint64_t c = threadIdx.x; c < columns; c += kBlock)
                dst[c] = __builtin_nanf("");
        }
    }
}

__global__ __launch_bounds__(kBlock) void gather_columns_kernel(float *__restrict__ out,
                                                                const float *__restrict__ in,
                                                                const uint32_t *__restrict__ cols,
                                                                uint64_t rows, uint64_t width,
                                                                uint32_t count)
{
    const uint64_t total = rows * count;
    const uint64_t stride = uint64_t(gridDim.x) * kBlock;
    for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride) {
        const uint64_t r = i / count;
        const uint32_t k = uint32_t(i - r * count);
        out[i] = in[r * width + cols[k]];
    }
}

// Row argmax: first strict maximum among admitted finite values; any
// admitted non-finite value, or no admitted value, gives NaN
// (backend-cpu/src/dense.rs:373-473).  A 1024-thread block scans a column
// range, each thread a strided slice in increasing order, then (value,
// index) candidates reduce with ties going to the lower index.  Wide rows
// are cut into ranges scanned by separate blocks whose candidates a second
// kernel reduces the same way.
constexpr int kArgmaxBlock = 1024;
constexpr uint32_t kArgmaxRange = 2048;

// Block-wide reduction; the result is valid in thread 0.
__device__ Candidate reduce_candidates(Candidate c)
{
    __shared__ float best_value[kArgmaxBlock / 64];
    __shared__ uint32_t best_index[kArgmaxBlock / 64];
    __shared__ int poison[kArgmaxBlock / 64];
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        merge(c, __shfl_xor(c.value, offset, 64), __shfl_xor(c.index, offset, 64),
              __shfl_xor(c.poisoned, offset, 64));
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        best_value[wave] = c.value;
        best_index[wave] = c.index;
        poison[wave] = c.poisoned;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < kArgmaxBlock / 64; ++w)
            merge(c, best_value[w], best_index[w], poison[w]);
    return c;
}

__device__ Candidate scan_range(const float *__restrict__ row, uint32_t begin, uint32_t end,
                                const uint64_t *__restrict__ mask)
{
    Candidate c{-__builtin_inff(), UINT32_MAX, 0};
    for (uint32_t j = begin + threadIdx.x; j < end; j += kArgmaxBlock) {
        if (mask && !((mask[j >> 6] >> (j & 63)) & 1))
            continue;
        const float v = row[j];
        if (!isfinite(v)) {
            c.poisoned = 1;
        } else if (c.index == UINT32_MAX || v > c.value) {
            // Strictly greater only: a thread's indices increase, so equal
            // values keep the earlier one.
            c.value = v;
            c.index = j;
        }
    }
    return reduce_candidates(c);
}

__device__ __forceinline__ float argmax_marker(const Candidate &c)
{
    return (c.poisoned || c.index == UINT32_MAX) ? __builtin_nanf("") : float(c.index);
}

// `copy` (may be null) receives the same selectors as `out`.
__global__ __launch_bounds__(kArgmaxBlock) void argmax_kernel(float *__restrict__ out,
                                                              float *__restrict__ copy,
                                                              const float *__restrict__ in,
                                                              uint32_t rows, uint32_t width,
                                                              const uint64_t *__restrict__ mask)
{
    for (uint32_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const Candidate c = scan_range(in + uint64_t(r) * width, 0, width, mask);
        if (threadIdx.x == 0) {
            out[r] = argmax_marker(c);
            if (copy)
                copy[r] = argmax_marker(c);
        }
    }
}

// Stage 1 of the wide-row path: block b scans range b % ranges of row
// b / ranges.
__global__ __launch_bounds__(kArgmaxBlock) void argmax_range_kernel(
    Candidate *__restrict__ partial, const float *__restrict__ in, uint32_t width,
    uint32_t ranges, const uint64_t *__restrict__ mask)
{
    const uint32_t r = blockIdx.x / ranges, range = blockIdx.x % ranges;
    const uint32_t begin = range * kArgmaxRange;
    const uint32_t end = width - begin < kArgmaxRange ? width : begin + kArgmaxRange;
    const Candidate c = scan_range(in + uint64_t(r) * width, begin, end, mask);
    if (threadIdx.x == 0)
        partial[blockIdx.x] = c;
}

__global__ __launch_bounds__(kArgmaxBlock) void argmax_final_kernel(
    float *__restrict__ out, float *__restrict__ copy, const Candidate *__restrict__ partial,
    uint32_t ranges)
{
    Candidate c{-__builtin_inff(), UINT32_MAX, 0};
    const Candidate *row = partial + uint64_t(blockIdx.x) * ranges;
    for (uint32_t i = threadIdx.x; i < ranges; i += kArgmaxBlock)
        merge(c, row[i].value, row[i].index, row[i].poisoned);
    c = reduce_candidates(c);
    if (threadIdx.x == 0) {
        out[blockIdx.x] = argmax_marker(c);
        if (copy)
            copy[blockIdx.x] = argmax_marker(c);
    }
}

// The same reduction by one wave (few ranges): shuffles only, no barrier.
// The merge keeps the largest value, the lowest index among equal values and
// any poison, so the order of the merges does not change the result.
__global__ __launch_bounds__(64) void argmax_final_wave_kernel(float *__restrict__ out,
                                                               float *__restrict__ copy,
                                                               const Candidate *__restrict__ partial,
                                                               uint32_t ranges)
{
    Candidate c{-__builtin_inff(), UINT32_MAX, 0};
    const Candidate *row = partial + uint64_t(blockIdx.x) * ranges;
    for (uint32_t i = threadIdx.x; i < ranges; i += 64)
        merge(c, row[i].value, row[i].index, row[i].poisoned);
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        merge(c, __shfl_xor(c.value, offset, 64), __shfl_xor(c.index, offset, 64),
              __shfl_xor(c.poisoned, offset, 64));
    if (threadIdx.x == 0) {
        out[blockIdx.x] = argmax_marker(c);
        if (copy)
            copy[blockIdx.x] = argmax_marker(c);
    }
}

// ---- element-wise ------------------------------------------------------

template <int OP>
__global__ __launch_bounds__(kBlock) void binary_kernel(float *__restrict__ out,
                                                        const float *__restrict__ left,
                                                        const float *__restrict__ right,
                                                        size_t count)
{
    const size_t stride = size_t(gridDim.x) * kBlock;
    for (size_t i = size_t(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride)
        out[i] = OP == 0 ? left[i] + right[i] : left[i] * right[i];
}

// ---- dense linear ------------------------------------------------------

// X[m, k] . W[n, k]^T: one wave per output element, lanes stride k.
__global__ __launch_bounds__(kBlock) void linear_kernel(float *__restrict__ out,
                                                        const float *__restrict__ x,
                                                        const float *__restrict__ w, uint32_t m,
                                                        uint32_t n, uint32_t k)
{
    const uint64_t total = uint64_t(m) * n;
    const uint64_t waves = uint64_t(gridDim.x) * (kBlock / 64);
    const int lane = threadIdx.x & 63;
    for (uint64_t o = uint64_t(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6); o < total;
         o += waves) {
        const uint32_t row = uint32_t(o / n);
        const uint32_t col = uint32_t(o - uint64_t(row) * n);
        const float *xr = x + uint64_t(row) * k;
        const float *wr = w + uint64_t(col) * k;
        float acc = 0.0f;
        for (uint32_t i = lane; i < k; i += 64)
            acc += xr[i] * wr[i];
        acc = wave_sum(acc);
        if (lane == 0)
            out[o] = acc;
    }
}

// ---- RMS normalisation -------------------------------------------------

// reciprocal = 1 / sqrt(sum(x * x) / width + epsilon); out = (x * r) * w
// (backend-cpu/src/normalization_rotary.rs:55-79).  With ADD the row is
// first formed as left + right and stored to `sum`
// (normalization_rotary.rs:223-235).  One block per row; each thread reads
// back only the elements it wrote.
template <bool ADD>
__global__ __launch_bounds__(kBlock) void row_rms_kernel(float *__restrict__ out,
                                                         float *__restrict__ sum,
                                                         const float *__restrict__ in,
                                                         const float *__restrict__ right,
                                                         const float *__restrict__ weight,
                                                         uint64_t rows, uint32_t width,
                                                         float epsilon)
{
    __shared__ float scratch[kBlock / 64];
    const float width_f = float(width);
    constexpr uint32_t kHeld = 8;
    if (width <= kHeld * kBlock) {
        // The row (and the weight) stay in registers: every load is issued
        // before the reduction, then one pass writes the outputs.
        for (uint64_t r = blockIdx.x; r < rows; r += gridDim.x) {
            const uint64_t base = r * width;
            float v[kHeld], w[kHeld];
#pragma unroll
            for (uint32_t i = 0; i < kHeld; ++i) {
                const uint32_t c = threadIdx.x + i * kBlock;
                v[i] = c < width ? in[base + c] : 0.0f;
                w[i] = c < width ? weight[c] : 0.0f;
                if (ADD)
                    v[i] = v[i] + (c < width ? right[base + c] : 0.0f);
            }
            float squares = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < kHeld; ++i) {
                const uint32_t c = threadIdx.x + i * kBlock;
                if (c < width) {
                    if (ADD)
                        sum[base + c] = v[i];
                    squares += v[i] * v[i];
                }
            }
            squares = block_sum(squares, scratch);
            const float reciprocal = 1.0f / sqrtf(squares / width_f + epsilon);
#pragma unroll
            for (uint32_t i = 0; i < kHeld; ++i) {
                const uint32_t c = threadIdx.x + i * kBlock;
                if (c < width)
                    out[base + c] = (v[i] * reciprocal) * w[i];
            }
        }
        return;
    }
    for (uint64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const uint64_t base = r * width;
        float squares = 0.0f;
        for (uint32_t c = threadIdx.x; c < width; c += kBlock) {
            float v = in[base + c];
            if (ADD) {
                v = v + right[base + c];
                sum[base + c] = v;
            }
            squares += v * v;
        }
        squares = block_sum(squares, scratch);
        const float reciprocal = 1.0f / sqrtf(squares / width_f + epsilon);
        const float *src = ADD ? sum : in;
        for (uint32_t c = threadIdx.x; c < width; c += kBlock) {
            const float normalized = src[base + c] * reciprocal;
            out[base + c] = normalized * weight[c];
        }
    }
}

// Head-local RMS norm over packed [tokens, heads * head_dim] rows
// (normalization_rotary.rs:124-151): one wave per (token, head).
__global__ __launch_bounds__(kBlock) void head_rms_kernel(float *__restrict__ out,
                                                          const float *__restrict__ in,
                                                          const float *__restrict__ weight,
                                                          uint64_t segments, uint32_t head_dim,
                                                          float epsilon)
{
    const int lane = threadIdx.x & 63;
    const uint64_t waves = uint64_t(gridDim.x) * (kBlock / 64);
    const float dim_f = float(head_dim);
    for (uint64_t s = uint64_t(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6); s < segments;
         s += waves) {
        const uint64_t base = s * head_dim;
        float squares = 0.0f;
        for (uint32_t c = lane; c < head_dim; c += 64) {
            const float v = in[base + c];
            squares += v * v;
        }
        squares = wave_sum(squares);
        const float reciprocal = 1.0f / sqrtf(squares / dim_f + epsilon);
        for (uint32_t c = lane; c < head_dim; c += 64) {
            const float normalized = in[base + c] * reciprocal;
            out[base + c] = normalized * weight[c];
        }
    }
}

// ---- split-half rotary -------------------------------------------------

// The reference's rotation coefficients: frequency = f32(theta^(-2c/d)) in
// f64, angle = position * frequency in f32, sine and cosine in f64 rounded
// to f32 (normalization_rotary.rs:196-207).
struct Rotation {
    float cosine, sine;
};

__device__ __forceinline__ Rotation rotation(float position, uint32_t column, uint32_t head_dim,
                                             float theta)
{
    const double exponent = -2.0 * double(column) / double(head_dim);
    const float frequency = float(pow(double(theta), exponent));
    const float angle = position * frequency;
    return {float(cos(double(angle))), float(sin(double(angle)))};
}

// Token t's position as the reference's `position as f32`: a staged f32
// array, or base + t converted here (u64 -> f32 rounds to nearest, as on the
// host).
__device__ __forceinline__ float position_of(const Positions &p, uint64_t token)
{
    return p.staged ? p.staged[token] : float(p.base + token);
}

// One thread per (token, head, column < half).
__global__ __launch_bounds__(kBlock) void rotary_kernel(float *__restrict__ out,
                                                        const float *__restrict__ in,
                                                        Positions positions, uint64_t tokens,
                                                        uint32_t heads, uint32_t head_dim,
                                                        float theta)
{
    const uint32_t half = head_dim / 2;
    const uint64_t total = tokens * heads * half;
    const uint64_t stride = uint64_t(gridDim.x) * kBlock;
    for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride) {
        const uint64_t segment = i / half;
        const uint32_t column = uint32_t(i - segment * half);
        const uint64_t token = segment / heads;
        const Rotation rot = rotation(position_of(positions, token), column, head_dim, theta);
        const uint64_t base = segment * head_dim;
        const float first = in[base + column];
        const float second = in[base + half + column];
        out[base + column] = first * rot.cosine - second * rot.sine;
        out[base + half + column] = second * rot.cosine + first * rot.sine;
    }
}

// One wave: head-local RMS norm of `in` (head_dim values) with `weight`,
// then the split-half rotation at `position`, into `out` and, when non-null,
// also `copy` (normalization_rotary.rs:246-369).
__device__ __forceinline__ void norm_rope_head(const float *__restrict__ in, float *out,
                                               float *copy, const float *__restrict__ weight,
                                               uint32_t head_dim, float position, float theta,
                                               float epsilon)
{
    const int lane = threadIdx.x & 63;
    const uint32_t half = head_dim / 2;
    float squares = 0.0f;
    for (uint32_t c = lane; c < head_dim; c += 64) {
        const float v = in[c];
        squares += v * v;
    }
    squares = wave_sum(squares);
    const float reciprocal = 1.0f / sqrtf(squares / float(head_dim) + epsilon);
    for (uint32_t c = lane; c < half; c += 64) {
        const float first = (in[c] * reciprocal) * weight[c];
        const float second = (in[half + c] * reciprocal) * weight[half + c];
        const Rotation rot = rotation(position, c, head_dim, theta);
        const float a = first * rot.cosine - second * rot.sine;
        const float b = second * rot.cosine + first * rot.sine;
        out[c] = a;
        out[half + c] = b;
        if (copy) {
            copy[c] = a;
            copy[half + c] = b;
        }
    }
}

// Per-head RMS norm then split-half rotary for query and key heads in one
// launch (normalization_rotary.rs:246-369): one wave per (token, head),
// query heads first.
__global__ __launch_bounds__(kBlock) void qk_norm_rope_kernel(
    float *__restrict__ query_out, float *__restrict__ key_out, const float *__restrict__ query,
    const float *__restrict__ key, const float *__restrict__ query_weight,
    const float *__restrict__ key_weight, Positions positions, uint64_t tokens,
    uint32_t query_heads, uint32_t key_heads, uint32_t head_dim, float theta, float epsilon)
{
    const uint32_t heads = query_heads + key_heads;
    const uint64_t segments = tokens * heads;
    const uint64_t waves = uint64_t(gridDim.x) * (kBlock / 64);
    for (uint64_t s = uint64_t(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6); s < segments;
         s += waves) {
        const uint64_t token = s / heads;
        const uint32_t head = uint32_t(s - token * heads);
        const bool is_query = head < query_heads;
        const uint32_t h = is_query ? head : head - query_heads;
        const uint64_t base =
            (token * (is_query ? query_heads : key_heads) + h) * uint64_t(head_dim);
        norm_rope_head((is_query ? query : key) + base, (is_query ? query_out : key_out) + base,
                       nullptr, is_query ? query_weight : key_weight, head_dim,
                       position_of(positions, token), theta, epsilon);
    }
}

// ---- causal grouped-query attention ------------------------------------

// Append the new key/value rows at row `start` of both caches.
__global__ __launch_bounds__(kBlock) void cache_append_kernel(float *__restrict__ key_cache,
                                                              float *__restrict__ value_cache,
                                                              const float *__restrict__ key,
                                                              const float *__restrict__ value,
                                                              uint64_t offset, uint64_t count)
{
    const uint64_t stride = uint64_t(gridDim.x) * kBlock;
    for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride) {
        key_cache[offset + i] = key[i];
        value_cache[offset + i] = value[i];
    }
}

constexpr int kKeyChunk = 1024;

// One block per (token, query head) over caches that already hold every
// visible key (the append runs first).  Three passes over the visible keys
// as in the reference (attention_convolution.rs:90-170): the maximum score,
// the softmax denominator, then probability-weighted values, with scores
// recomputed per pass.  Each score is a sequential dot in dimension order,
// the reference's exact arithmetic.
__global__ __launch_bounds__(kBlock) void gqa_kernel(float *__restrict__ out,
                                                     const float *__restrict__ query,
                                                     const float *__restrict__ key_cache,
                                                     const float *__restrict__ value_cache,
                                                     GqaShape g)
{
    extern __shared__ float lds[];
    float *q = lds;                        // head_dim
    float *prob = q + g.head_dim;          // kKeyChunk
    float *part = prob + kKeyChunk;        // kBlock
    __shared__ float scratch[kBlock / 64];

    const uint32_t query_heads = g.query_heads;
    const uint64_t token = blockIdx.x / query_heads;
    const uint32_t head = uint32_t(blockIdx.x - token * query_heads);
    const uint32_t kv_head = head / g.group;
    const uint32_t d = g.head_dim;
    const uint64_t kv_width = uint64_t(g.key_value_heads) * d;
    const uint64_t visible = g.initial_len + token + 1;
    const float *qrow = query + (token * query_heads + head) * uint64_t(d);
    const float *keys = key_cache + uint64_t(kv_head) * d;
    const float *values = value_cache + uint64_t(kv_head) * d;
    for (uint32_t c = threadIdx.x; c < d; c += kBlock)
        q[c] = qrow[c];
    __syncthreads();

    auto score = [&](uint64_t j) {
        const float *krow = keys + j * kv_width;
        float dot = 0.0f;
        for (uint32_t c = 0; c < d; ++c)
            dot += q[c] * krow[c];
        return dot * g.scale;
    };

    float maximum = -__builtin_inff();
    for (uint64_t j = threadIdx.x; j < visible; j += kBlock)
        maximum = fmaxf(maximum, score(j));
    maximum = block_max(maximum, scratch);

    float denominator = 0.0f;
    for (uint64_t j = threadIdx.x; j < visible; j += kBlock)
        denominator += expf(score(j) - maximum);
    denominator = block_sum(denominator, scratch);

    // Threads split as `groups` key groups of `span` dimensions; a head wider
    // than the block gives each thread up to kMaxDimsPerThread dimensions.
    const uint32_t span = d < kBlock ? d : kBlock;
    const uint32_t groups = kBlock / span;
    const uint32_t group = threadIdx.x / span;
    const uint32_t lane_dim = threadIdx.x - group * span;
    float acc[kMaxDimsPerThread];
#pragma unroll
    for (int i = 0; i < kMaxDimsPerThread; ++i)
        acc[i] = 0.0f;
    for (uint64_t base = 0; base < visible; base += kKeyChunk) {
        const uint32_t chunk = uint32_t(visible - base < kKeyChunk ? visible - base : kKeyChunk);
        __syncthreads();
        for (uint32_t j = threadIdx.x; j < chunk; j += kBlock)
            prob[j] = expf(score(base + j) - maximum) / denominator;
        __syncthreads();
        if (group < groups) {
#pragma unroll
            for (int i = 0; i < kMaxDimsPerThread; ++i) {
                const uint32_t dim = lane_dim + uint32_t(i) * kBlock;
                if (dim >= d)
                    break;
                float a = acc[i];
                for (uint32_t j = group; j < chunk; j += groups)
                    a += prob[j] * values[(base + j) * kv_width + dim];
                acc[i] = a;
            }
        }
    }
    float *orow = out + (token * query_heads + head) * uint64_t(d);
    if (groups == 1) {
        if (group != 0)
            return;
#pragma unroll
        for (int i = 0; i < kMaxDimsPerThread; ++i) {
            const uint32_t dim = lane_dim + uint32_t(i) * kBlock;
            if (dim < d)
                orow[dim] = acc[i];
        }
        return;
    }
    __syncthreads();
    if (group < groups)
        part[threadIdx.x] = acc[0];
    __syncthreads();
    if (threadIdx.x < d) {
        float total = part[threadIdx.x];
        for (uint32_t gi = 1; gi < groups; ++gi)
            total += part[gi * span + threadIdx.x];
        orow[threadIdx.x] = total;
    }
}

// ---- prefill attention on fp32 matrix cores ------------------------------
//
// Flash-style causal GQA for many (token, query head) pairs.  A block of
// kFlashWaves waves serves one key/value head and kFlashRows query rows:
// `tile_tokens` consecutive tokens times the group's query heads (row r is
// token t0 + r / group, query head r % group of the key/value head).  Key
// and value rows stream through LDS in kFlashKeys-key tiles that every row
// of the block shares; each wave owns 16 rows.
//
// Per tile, S^T = K Q^T on v_mfma_f32_16x16x4f32 leaves row j of a wave in
// lane column j: lane 16q + j holds the scores of keys 16c + 4q + r in
// register r of column block c.  The running maximum, the exponent sum and
// the output rescale therefore stay in the row's own four lanes (reduced
// over the lane blocks q).  The output accumulates as O^T = V^T P^T, whose B
// operand at step (c, r) is the lane's own probability register, and whose
// result lane 16q + j holds dimensions 16t + 4q + r of row j.
//
// Numerics: every score is the exact products summed in matrix-core order,
// and the softmax takes the online (running maximum) form of the
// reference's three passes (attention_convolution.rs:90-170); results agree
// within f32 reassociation error.  A key the causal mask hides gets
// probability zero, so a non-finite value row later in the same tile still
// reaches the earlier rows (0 * NaN), where the reference skips it.
constexpr int kFlashWaves = 4;
constexpr uint32_t kFlashRows = 16 * kFlashWaves;
constexpr uint32_t kFlashKeys = 64;
// Widest head of the fp32 matrix-core path: its key and transposed value
// tiles stay within 64 KB of LDS.
constexpr uint32_t kFlashMaxDim = 112;

typedef float v4f __attribute__((ext_vector_type(4)));

// K tile [keys][D + 4], then V^T tile [D][keys + 4] (pads keep 16-byte rows
// and spread the lane blocks over banks).
template <int D>
constexpr size_t flash_lds_bytes()
{
    return (size_t(kFlashKeys) * (D + 4) + size_t(D) * (kFlashKeys + 4)) * sizeof(float);
}

template <int D>
__global__ __launch_bounds__(64 * kFlashWaves) void gqa_flash_kernel(
    float *__restrict__ out, const float *__restrict__ query, const float *__restrict__ key_cache,
    const float *__restrict__ value_cache, GqaShape g, uint32_t tile_tokens, uint32_t token_tiles)
{
    static_assert(D % 16 == 0 && D <= int(kFlashMaxDim), "head width of the flash path");
    constexpr uint32_t KS = D + 4, VS = kFlashKeys + 4;
    constexpr int U = D / 16;                  // 16-wide dimension blocks
    constexpr int C = kFlashKeys / 16;         // 16-key column blocks
    constexpr uint32_t QUADS = kFlashKeys * D / 4;  // float4s per tile and matrix
    constexpr int PER = QUADS / (64 * kFlashWaves);
    static_assert(QUADS % (64 * kFlashWaves) == 0, "staging shape");
    extern __shared__ float lds[];
    float *kl = lds;
    float *vt = lds + kFlashKeys * KS;

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t q = lane >> 4, j = lane & 15;
    const uint32_t kv_heads = g.key_value_heads;
    const uint32_t kv_head = blockIdx.x % kv_heads;
    // Longest token tiles (most keys) first.
    const uint32_t tile = token_tiles - 1 - blockIdx.x / kv_heads;
    const uint64_t t0 = uint64_t(tile) * tile_tokens;
    const uint64_t t_end = t0 + tile_tokens < g.tokens ? t0 + tile_tokens : g.tokens;
    const uint64_t k_end = g.initial_len + t_end;  // keys [0, k_end) reach some row
    const uint64_t kv_width = uint64_t(kv_heads) * D;

    // The lane's row.  Rows past the tile (or past the last token) compute
    // over every staged key and store nothing.
    const uint32_t row = 16 * wave + j;
    const uint32_t group = g.group;
    const uint64_t token = t0 + row / group;
    const uint32_t head = kv_head * group + row % group;
    const bool valid = row < tile_tokens * group && token < g.tokens;
    const uint64_t last = valid ? g.initial_len + token : k_end - 1;  // last visible key

    // Q^T operand: dimensions 16u + 4q + e of the row at step 4u + e.
    v4f qv[U];
    const float *qrow = query + (token * g.query_heads + head) * uint64_t(D);
#pragma unroll
    for (int u = 0; u < U; ++u)
        qv[u] = valid ? *reinterpret_cast<const v4f *>(qrow + 16 * u + 4 * q) : v4f{0, 0, 0, 0};

    v4f kr[PER], vr[PER];
    auto stage_load = [&](uint32_t n) {
        const uint64_t k0 = uint64_t(n) * kFlashKeys;
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const uint32_t f = threadIdx.x + p * 64 * kFlashWaves;
            const uint32_t key = f / (D / 4), c4 = f % (D / 4);
            kr[p] = vr[p] = v4f{0, 0, 0, 0};
            if (k0 + key < k_end) {
                const size_t at = (k0 + key) * kv_width + uint64_t(kv_head) * D + 4 * c4;
                kr[p] = *reinterpret_cast<const v4f *>(key_cache + at);
                vr[p] = *reinterpret_cast<const v4f *>(value_cache + at);
            }
        }
    };
    auto stage_store = [&]() {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const uint32_t f = threadIdx.x + p * 64 * kFlashWaves;
            const uint32_t key = f / (D / 4), c4 = f % (D / 4);
            *reinterpret_cast<v4f *>(kl + key * KS + 4 * c4) = kr[p];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                vt[(4 * c4 + e) * VS + key] = vr[p][e];
        }
    };

    v4f o[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
        o[u] = v4f{0, 0, 0, 0};
    float m = -__builtin_inff(), l = 0.0f;
    const uint32_t tiles = uint32_t((k_end + kFlashKeys - 1) / kFlashKeys);
    stage_load(0);
    stage_store();
    __syncthreads();
    for (uint32_t n = 0; n < tiles; ++n) {
        if (n + 1 < tiles)
            stage_load(n + 1);  // in flight behind this tile's arithmetic
        // S^T = K Q^T.  A operand of lane (q, i): key 16c + i, dimensions
        // 16u + 4q + e.
        v4f s[C];
#pragma unroll
        for (int c = 0; c < C; ++c)
            s[c] = v4f{0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < U; ++u) {
            v4f kk[C];
#pragma unroll
            for (int c = 0; c < C; ++c)
                kk[c] = *reinterpret_cast<const v4f *>(kl + (16 * c + j) * KS + 16 * u + 4 * q);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int c = 0; c < C; ++c)
                    s[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[c][e], qv[u][e], s[c], 0, 0, 0);
        }
        // Scale, causal mask, online softmax over the row's four lanes.
        const uint64_t k0 = uint64_t(n) * kFlashKeys;
        float mx = -__builtin_inff();
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = s[c][r] * g.scale;
                if (k0 + 16 * c + 4 * q + r > last)
                    v = -__builtin_inff();
                s[c][r] = v;
                mx = fmaxf(mx, v);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m, mx);
        const float alpha = expf(m - m_new);
        float sum = 0.0f;
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = expf(s[c][r] - m_new);
                s[c][r] = p;
                sum += p;
            }
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        l = l * alpha + sum;
        m = m_new;
#pragma unroll
        for (int u = 0; u < U; ++u)
            o[u] *= alpha;
        // O^T += V^T P^T.  A operand of lane (q, i) at step (c, r): V^T row
        // 16t + i, key 16c + 4q + r.
#pragma unroll
        for (int c = 0; c < C; ++c) {
            v4f vv[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
                vv[u] = *reinterpret_cast<const v4f *>(vt + (16 * u + j) * VS + 16 * c + 4 * q);
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int u = 0; u < U; ++u)
                    o[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[u][r], s[c][r], o[u], 0, 0, 0);
        }
        if (n + 1 < tiles) {
            __syncthreads();
            stage_store();
            __syncthreads();
        }
    }
    if (!valid)
        return;
    float *orow = out + (token * g.query_heads + head) * uint64_t(D);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        v4f r;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            r[e] = o[u][e] / l;
        *reinterpret_cast<v4f *>(orow + 16 * u + 4 * q) = r;
    }
}

// Split-key attention for few (token, head) pairs (decode): the visible keys
// of one (token, key/value head) are cut into kSplitKeys-wide ranges, one
// block per range serving every query head of the group.  The block stages
// its range's key and value rows in LDS with coalesced loads, then stores,
// per query head, its range maximum m, its exponent sum l = sum exp(s - m)
// and the unnormalised sum acc = sum exp(s - m) * v; the combine kernel
// rescales the ranges to the global maximum.  Scores keep the reference's
// sequential dot; the softmax normalisation is regrouped (exp(s - m) *
// exp(m - M) / L for exp(s - M) / L), a reassociation within f32 rounding.
constexpr int kSplitKeys = 64;
// Limits of the split path: its dynamic LDS (below) and the combine
// kernel's per-range weights.
constexpr size_t kSplitMaxLds = 64 * 1024;
constexpr uint32_t kSplitMaxRanges = 8192;

// Dynamic LDS of gqa_split_kernel: q [group][d], keys [kSplitKeys][d + 1]
// (the pad puts consecutive keys on distinct banks), values
// [kSplitKeys][d], probabilities [group][kSplitKeys].
__host__ __device__ inline size_t gqa_split_lds(uint32_t group, uint32_t d)
{
    return (size_t(group) * d + size_t(kSplitKeys) * (d + 1) + size_t(kSplitKeys) * d +
            size_t(group) * kSplitKeys) *
           sizeof(float);
}

__global__ __launch_bounds__(kBlock) void gqa_split_kernel(float *__restrict__ partial,
                                                           const float *__restrict__ query,
                                                           const float *__restrict__ key_cache,
                                                           const float *__restrict__ value_cache,
                                                           GqaShape g, uint32_t splits)
{
    extern __shared__ float lds[];
    const uint32_t d = g.head_dim, group = g.group;
    float *q = lds;
    float *kl = q + group * d;
    float *vl = kl + kSplitKeys * (d + 1);
    float *p = vl + kSplitKeys * d;

    const uint32_t split = blockIdx.x % splits;
    const uint64_t pair = blockIdx.x / splits;
    const uint32_t kv_head = uint32_t(pair % g.key_value_heads);
    const uint64_t token = pair / g.key_value_heads;
    const uint64_t kv_width = uint64_t(g.key_value_heads) * d;
    const uint64_t visible = g.initial_len + token + 1;
    const uint64_t begin = uint64_t(split) * kSplitKeys;
    const uint32_t count =
        begin >= visible ? 0u : uint32_t(visible - begin < kSplitKeys ? visible - begin : kSplitKeys);
    // Record layout: [token][query head][split] of (m, l, acc[d]).
    const uint64_t record = uint64_t(d) + 2;
    const uint32_t head0 = kv_head * group;
    float *out = partial + ((token * g.query_heads + head0) * splits + split) * record;

    const float *qrow = query + (token * g.query_heads + head0) * uint64_t(d);
    for (uint32_t i = threadIdx.x; i < group * d; i += kBlock)
        q[i] = qrow[i];
    const float *keys = key_cache + begin * kv_width + kv_head * uint64_t(d);
    const float *values = value_cache + begin * kv_width + kv_head * uint64_t(d);
    if (d % 4 == 0) {
        // float4 loads, up to kStage per thread issued before any is stored.
        constexpr uint32_t kStage = 8;
        const uint32_t quads = count * d / 4;
        for (uint32_t base = 0; base < quads; base += kStage * kBlock) {
            float4 kq[kStage], vq[kStage];
#pragma unroll
            for (uint32_t u = 0; u < kStage; ++u)
                kq[u] = vq[u] = float4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t u = 0; u < kStage; ++u) {
                const uint32_t i = base + u * kBlock + threadIdx.x;
                if (i < quads) {
                    const uint32_t key = 4 * i / d, c = 4 * i - key * d;
                    kq[u] = *reinterpret_cast<const float4 *>(keys + key * kv_width + c);
                    vq[u] = *reinterpret_cast<const float4 *>(values + key * kv_width + c);
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < kStage; ++u) {
                const uint32_t i = base + u * kBlock + threadIdx.x;
                if (i < quads) {
                    const uint32_t key = 4 * i / d, c = 4 * i - key * d;
                    float *kr = kl + key * (d + 1) + c;
                    kr[0] = kq[u].x;
                    kr[1] = kq[u].y;
                    kr[2] = kq[u].z;
                    kr[3] = kq[u].w;
                    reinterpret_cast<float4 *>(vl)[i] = vq[u];
                }
            }
        }
    } else {
        for (uint32_t i = threadIdx.x; i < count * d; i += kBlock) {
            const uint32_t key = i / d, c = i - key * d;
            kl[key * (d + 1) + c] = keys[key * kv_width + c];
            vl[i] = values[key * kv_width + c];
        }
    }
    __syncthreads();

    // Scores of (head, key) items: the reference's sequential dot.
    for (uint32_t i = threadIdx.x; i < group * kSplitKeys; i += kBlock) {
        const uint32_t h = i / kSplitKeys, key = i % kSplitKeys;
        if (key < count) {
            const float *qh = q + h * d;
            const float *kr = kl + key * (d + 1);
            float dot = 0.0f;
            for (uint32_t c = 0; c < d; ++c)
                dot += qh[c] * kr[c];
            p[i] = dot * g.scale;
        }
    }
    __syncthreads();
    // One wave per head (kSplitKeys == 64 keys, one per lane).
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (uint32_t h = wave; h < group; h += kBlock / 64) {
        const float s = lane < count ? p[h * kSplitKeys + lane] : -__builtin_inff();
        const float m = wave_max(s);
        const float e = lane < count ? expf(s - m) : 0.0f;
        p[h * kSplitKeys + lane] = e;
        const float l = wave_sum(e);
        if (lane == 0) {
            out[uint64_t(h) * splits * record] = m;
            out[uint64_t(h) * splits * record + 1] = l;
        }
    }
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < group * d; t += kBlock) {
        const uint32_t h = t / d, dim = t - h * d;
        const float *ph = p + h * kSplitKeys;
        float acc = 0.0f;
        for (uint32_t j = 0; j < count; ++j)
            acc += ph[j] * vl[j * d + dim];
        out[uint64_t(h) * splits * record + 2 + dim] = acc;
    }
}

// One block per (token, query head): out = sum_s acc_s e^(m_s - M) / L with
// M = max m_s and L = sum l_s e^(m_s - M).  Empty ranges (l = 0) are
// skipped; a NaN anywhere reaches the output.  The block's threads split the
// ranges into kBlock / d interleaved parts, summed part by part at the end.
__global__ __launch_bounds__(kBlock) void gqa_combine_kernel(float *__restrict__ out,
                                                             const float *__restrict__ partial,
                                                             uint32_t head_dim, uint32_t splits)
{
    extern __shared__ float lds[];
    float *weight = lds;              // [splits] e^(m_s - M), 0 for empty ranges
    float *part = lds + splits;       // [parts][head_dim]
    __shared__ float scratch[kBlock / 64];
    const uint64_t record = uint64_t(head_dim) + 2;
    const float *rec = partial + uint64_t(blockIdx.x) * splits * record;
    const uint32_t parts = head_dim <= kBlock ? kBlock / head_dim : 1;
    const uint32_t part_id = threadIdx.x / head_dim, dim0 = threadIdx.x % head_dim;
    // Every load goes out before the reductions: this thread's range
    // record (m, l) when splits fit the block, and the acc values it sums
    // when head_dim fits the block and it sums at most kHeld of them.
    constexpr uint32_t kHeld = 16;
    const bool own = splits <= kBlock;
    const bool holds = part_id < parts && head_dim <= kBlock && splits <= parts * kHeld;
    float m_own = 0.0f, l_own = 0.0f;
    if (own && threadIdx.x < splits) {
        m_own = rec[threadIdx.x * record];
        l_own = rec[threadIdx.x * record + 1];
    }
    float held[kHeld];
#pragma unroll
    for (uint32_t i = 0; i < kHeld; ++i) {
        const uint32_t s = part_id + i * parts;
        held[i] = holds && s < splits ? rec[s * record + 2 + dim0] : 0.0f;
    }
    float maximum = -__builtin_inff();
    if (own) {
        if (threadIdx.x < splits && l_own != 0.0f)
            maximum = fmaxf(maximum, m_own);
    } else {
        for (uint32_t s = threadIdx.x; s < splits; s += kBlock)
            if (rec[s * record + 1] != 0.0f)
                maximum = fmaxf(maximum, rec[s * record]);
    }
    maximum = block_max(maximum, scratch);
    float denominator = 0.0f;
    for (uint32_t s = threadIdx.x; s < splits; s += kBlock) {
        // An empty range stores l = 0 and acc = 0: weight 0 drops it.
        const float l = own ? l_own : rec[s * record + 1];
        const float m = own ? m_own : rec[s * record];
        const float w = l != 0.0f ? expf(m - maximum) : 0.0f;
        weight[s] = w;
        if (l != 0.0f)
            denominator += l * w;
    }
    denominator = block_sum(denominator, scratch);  // also orders the weight stores
    if (holds) {
        float acc = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < kHeld; ++i) {
            const uint32_t s = part_id + i * parts;
            if (s < splits)
                acc += held[i] * weight[s];
        }
        part[part_id * head_dim + dim0] = acc;
    } else if (part_id < parts) {
        for (uint32_t dim = dim0; dim < head_dim; dim += kBlock) {
            float acc = 0.0f;
            for (uint32_t s = part_id; s < splits; s += parts)
                acc += rec[s * record + 2 + dim] * weight[s];
            part[part_id * head_dim + dim] = acc;
        }
    }
    __syncthreads();
    for (uint32_t dim = threadIdx.x; dim < head_dim; dim += kBlock) {
        float acc = part[dim];
        for (uint32_t pi = 1; pi < parts; ++pi)
            acc += part[pi * head_dim + dim];
        out[uint64_t(blockIdx.x) * head_dim + dim] = acc / denominator;
    }
}

// One decode token's qk_norm_rope, key append and split-key attention in
// one launch (gqa_combine_kernel then merges the ranges).  Block (kv head,
// range) stages its keys and values with float4 loads, normalises and
// rotates its group's queries into LDS (the coefficients come from a
// rotation table, see launch_rotation_table), and -- the block whose range
// ends at the new key -- that key's row, which it also writes to the cache
// (the value row is already there).  Each block then stores its (m, l, acc)
// records as gqa_split_kernel does.  Handing the records to the combine
// through a kernel boundary measured faster than a last-block combine,
// whose __threadfence() writes back the L2 of every XCD.
__device__ __forceinline__ void norm_rope_head_table(const float *__restrict__ in, float *out,
                                                     float *copy, const float *__restrict__ weight,
                                                     uint32_t head_dim, const float *cosine,
                                                     const float *sine, float epsilon)
{
    const int lane = threadIdx.x & 63;
    const uint32_t half = head_dim / 2;
    float squares = 0.0f;
    for (uint32_t c = lane; c < head_dim; c += 64) {
        const float v = in[c];
        squares += v * v;
    }
    squares = wave_sum(squares);
    const float reciprocal = 1.0f / sqrtf(squares / float(head_dim) + epsilon);
    for (uint32_t c = lane; c < half; c += 64) {
        const float first = (in[c] * reciprocal) * weight[c];
        const float second = (in[half + c] * reciprocal) * weight[half + c];
        const float a = first * cosine[c] - second * sine[c];
        const float b = second * cosine[c] + first * sine[c];
        out[c] = a;
        out[half + c] = b;
        if (copy) {
            copy[c] = a;
            copy[half + c] = b;
        }
    }
}


__global__ __launch_bounds__(kBlock) void gqa_decode_kernel(DecodeAttention p)
{
    extern __shared__ float lds[];
    const uint32_t d = p.head_dim, group = p.group, splits = p.splits;
    const uint32_t half = d / 2;
    float *q = lds;
    float *kl = q + group * d;
    float *vl = kl + kSplitKeys * (d + 1);
    float *pr = vl + kSplitKeys * d;
    const float *rot = p.rotation + p.position * d;  // cosines [half], sines [half]

    const uint32_t split = blockIdx.x % splits;
    const uint32_t kv_head = blockIdx.x / splits;
    const uint64_t kv_width = uint64_t(p.key_value_heads) * d;
    const uint64_t visible = p.position + 1;
    const uint64_t begin = uint64_t(split) * kSplitKeys;
    const uint32_t count =
        begin >= visible ? 0u : uint32_t(visible - begin < kSplitKeys ? visible - begin : kSplitKeys);
    const bool holds_new = count > 0 && begin + count == visible;
    const uint32_t cached = holds_new ? count - 1 : count;  // key rows read from the cache
    const uint64_t record = uint64_t(d) + 2;
    const uint32_t head0 = kv_head * group;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

    // Keys and values of the range (d % 4 == 0, checked by the launcher).
    const float *keys = p.key_cache + begin * kv_width + kv_head * uint64_t(d);
    const float *values = p.value_cache + begin * kv_width + kv_head * uint64_t(d);
    {
        constexpr uint32_t kStage = 8;
        const uint32_t quads = count * d / 4;
        for (uint32_t base = 0; base < quads; base += kStage * kBlock) {
            float4 kq[kStage], vq[kStage];
#pragma unroll
            for (uint32_t u = 0; u < kStage; ++u)
                kq[u] = vq[u] = float4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t u = 0; u < kStage; ++u) {
                const uint32_t i = base + u * kBlock + threadIdx.x;
                if (i < quads) {
                    const uint32_t key = 4 * i / d, c = 4 * i - key * d;
                    if (key < cached)
                        kq[u] = *reinterpret_cast<const float4 *>(keys + key * kv_width + c);
                    vq[u] = *reinterpret_cast<const float4 *>(values + key * kv_width + c);
                }
            }
            if (base == 0) {
                // The group's query heads (and the new key) are normalised
                // and rotated while the range's keys and values are in
                // flight; an empty range needs neither.
                for (uint32_t h = wave; h < group; h += kBlock / 64)
                    norm_rope_head_table(p.query + (head0 + h) * uint64_t(d), q + h * d, nullptr,
                                         p.query_weight, d, rot, rot + half, p.epsilon);
                if (holds_new && wave == kBlock / 64 - 1)
                    norm_rope_head_table(p.key + kv_head * uint64_t(d),
                                         kl + (count - 1) * (d + 1),
                                         p.key_cache + p.position * kv_width +
                                             kv_head * uint64_t(d),
                                         p.key_weight, d, rot, rot + half, p.epsilon);
            }
#pragma unroll
            for (uint32_t u = 0; u < kStage; ++u) {
                const uint32_t i = base + u * kBlock + threadIdx.x;
                if (i < quads) {
                    const uint32_t key = 4 * i / d, c = 4 * i - key * d;
                    if (key < cached) {
                        float *kr = kl + key * (d + 1) + c;
                        kr[0] = kq[u].x;
                        kr[1] = kq[u].y;
                        kr[2] = kq[u].z;
                        kr[3] = kq[u].w;
                    }
                    reinterpret_cast<float4 *>(vl)[i] = vq[u];
                }
            }
        }
    }
    __syncthreads();

    float *out_records = p.partial + (uint64_t(head0) * splits + split) * record;
    for (uint32_t i = threadIdx.x; i < group * kSplitKeys; i += kBlock) {
        const uint32_t h = i / kSplitKeys, key = i % kSplitKeys;
        if (key < count) {
            const float *qh = q + h * d;
            const float *kr = kl + key * (d + 1);
            float dot = 0.0f;
            for (uint32_t c = 0; c < d; ++c)
                dot += qh[c] * kr[c];
            pr[i] = dot * p.scale;
        }
    }
    __syncthreads();
    for (uint32_t h = wave; h < group; h += kBlock / 64) {
        const float s = lane < count ? pr[h * kSplitKeys + lane] : -__builtin_inff();
        const float m = wave_max(s);
        const float e = lane < count ? expf(s - m) : 0.0f;
        pr[h * kSplitKeys + lane] = e;
        const float l = wave_sum(e);
        if (lane == 0) {
            out_records[uint64_t(h) * splits * record] = m;
            out_records[uint64_t(h) * splits * record + 1] = l;
        }
    }
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < group * d; t += kBlock) {
        const uint32_t h = t / d, dim = t - h * d;
        const float *ph = pr + h * kSplitKeys;
        float acc = 0.0f;
        for (uint32_t j = 0; j < count; ++j)
            acc += ph[j] * vl[j * d + dim];
        out_records[uint64_t(h) * splits * record + 2 + dim] = acc;
    }

}

// Row t of the table: rotation(t, c) for c < head_dim / 2, cosines then
// sines (the coefficients the rotary kernels compute inline).
// qk_norm_rope_kernel for the consecutive positions first, first + 1, ...,
// with the coefficients read from a rotation table (launch_rotation_table)
// rather than computed per element: the same values bit for bit.
__global__ __launch_bounds__(kBlock) void qk_norm_rope_table_kernel(
    float *__restrict__ query_out, float *__restrict__ key_out, const float *__restrict__ query,
    const float *__restrict__ key, const float *__restrict__ query_weight,
    const float *__restrict__ key_weight, const float *__restrict__ table, uint64_t first,
    uint64_t tokens, uint32_t query_heads, uint32_t key_heads, uint32_t head_dim, float epsilon)
{
    const uint32_t heads = query_heads + key_heads;
    const uint64_t segments = tokens * heads;
    const uint64_t waves = uint64_t(gridDim.x) * (kBlock / 64);
    for (uint64_t s = uint64_t(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6); s < segments;
         s += waves) {
        const uint64_t token = s / heads;
        const uint32_t head = uint32_t(s - token * heads);
        const bool is_query = head < query_heads;
        const uint32_t h = is_query ? head : head - query_heads;
        const uint64_t base =
            (token * (is_query ? query_heads : key_heads) + h) * uint64_t(head_dim);
        const float *row = table + (first + token) * head_dim;
        norm_rope_head_table((is_query ? query : key) + base,
                             (is_query ? query_out : key_out) + base, nullptr,
                             is_query ? query_weight : key_weight, head_dim, row,
                             row + head_dim / 2, epsilon);
    }
}

__global__ __launch_bounds__(kBlock) void rotation_table_kernel(float *__restrict__ table,
                                                                uint64_t positions,
                                                                uint32_t head_dim, float theta)
{
    const uint32_t half = head_dim / 2;
    const uint64_t total = positions * half;
    const uint64_t stride = uint64_t(gridDim.x) * kBlock;
    for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride) {
        const uint64_t t = i / half;
        const uint32_t c = uint32_t(i - t * half);
        const Rotation r = rotation(float(t), c, head_dim, theta);
        table[t * head_dim + c] = r.cosine;
        table[t * head_dim + half + c] = r.sine;
    }
}

// ---- gated short convolution -------------------------------------------

// u = B * V per (token, channel); out = (sum over taps of kernel * u) * C,
// with taps oldest to current and the first width - 1 reaching into the
// rolling history; afterwards the history holds the last width - 1 u rows
// (attention_convolution.rs:220-340).  One thread per channel walks the
// tokens, so the in-place history update needs no cross-thread ordering.
__global__ __launch_bounds__(kBlock) void short_conv_kernel(float *__restrict__ out,
                                                            const float *__restrict__ projection,
                                                            const float *__restrict__ kernel,
                                                            float *__restrict__ history,
                                                            uint64_t tokens, uint32_t hidden,
                                                            uint32_t width)
{
    const uint32_t channel = blockIdx.x * kBlock + threadIdx.x;
    if (channel >= hidden)
        return;
    const uint64_t pw = uint64_t(hidden) * 3;
    const int64_t history_rows = int64_t(width) - 1;
    auto u_at = [&](int64_t relative) {
        if (relative < 0)
            return history[uint64_t(relative + history_rows) * hidden + channel];
        const float *p = projection + uint64_t(relative) * pw + channel;
        return p[0] * p[2 * uint64_t(hidden)];
    };
    const float *taps = kernel + uint64_t(channel) * width;
    for (uint64_t t = 0; t < tokens; ++t) {
        float total = 0.0f;
        for (uint32_t tap = 0; tap < width; ++tap)
            total += taps[tap] * u_at(int64_t(t) + int64_t(tap) - history_rows);
        out[t * hidden + channel] = total * projection[t * pw + hidden + channel];
    }
    if (history_rows <= 0)
        return;
    // Row r of the new history is logical position tokens - history_rows + r;
    // rows read from the old history sit strictly above the row written, so
    // an increasing walk reads each old value before overwriting it.
    for (int64_t r = 0; r < history_rows; ++r)
        history[uint64_t(r) * hidden + channel] = u_at(int64_t(tokens) - history_rows + r);
}

// The same convolution for many tokens, one thread per (token, channel)
// output, with the same per-output tap order (bit-identical results).  The
// history is only read here; conv_roll_kernel rolls it afterwards.
__global__ __launch_bounds__(kBlock) void conv_tokens_kernel(float *__restrict__ out,
                                                             const float *__restrict__ projection,
                                                             const float *__restrict__ kernel,
                                                             const float *__restrict__ history,
                                                             uint64_t tokens, uint32_t hidden,
                                                             uint32_t width)
{
    const uint64_t pw = uint64_t(hidden) * 3;
    const int64_t history_rows = int64_t(width) - 1;
    const uint64_t count = tokens * hidden, stride = uint64_t(gridDim.x) * kBlock;
    for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride) {
        const uint64_t t = i / hidden;
        const uint32_t channel = uint32_t(i - t * hidden);
        const float *taps = kernel + uint64_t(channel) * width;
        float total = 0.0f;
        for (uint32_t tap = 0; tap < width; ++tap) {
            const int64_t relative = int64_t(t) + int64_t(tap) - history_rows;
            float u;
            if (relative < 0) {
                u = history[uint64_t(relative + history_rows) * hidden + channel];
            } else {
                const float *p = projection + uint64_t(relative) * pw + channel;
                u = p[0] * p[2 * uint64_t(hidden)];
            }
            total += taps[tap] * u;
        }
        out[t * hidden + channel] = total * projection[t * pw + hidden + channel];
    }
}

// One decode token of the gated short convolution, reading the history
// from `history` and writing the rolled history to `next` (the two-buffer
// layout of the decode step), one thread per channel.  The arithmetic is
// short_conv_kernel's at one token, term for term.
__global__ __launch_bounds__(kBlock) void conv_step_kernel(float *__restrict__ out,
                                                           const float *__restrict__ projection,
                                                           const float *__restrict__ kernel,
                                                           const float *__restrict__ history,
                                                           float *__restrict__ next,
                                                           uint32_t hidden, uint32_t width)
{
    const uint32_t channel = blockIdx.x * kBlock + threadIdx.x;
    if (channel >= hidden)
        return;
    const uint32_t rows = width - 1;
    const float u = projection[channel] * projection[2 * uint64_t(hidden) + channel];
    const float *taps = kernel + uint64_t(channel) * width;
    float total = 0.0f;
    for (uint32_t tap = 0; tap < rows; ++tap)
        total += taps[tap] * history[uint64_t(tap) * hidden + channel];
    total += taps[rows] * u;
    for (uint32_t r = 0; r + 1 < rows; ++r)
        next[uint64_t(r) * hidden + channel] = history[uint64_t(r + 1) * hidden + channel];
    if (rows)
        next[uint64_t(rows - 1) * hidden + channel] = u;
    out[channel] = total * projection[uint64_t(hidden) + channel];
}

// The history roll of short_conv_kernel on its own, one thread per channel.
__global__ __launch_bounds__(kBlock) void conv_roll_kernel(const float *__restrict__ projection,
                                                           float *__restrict__ history,
                                                           uint64_t tokens, uint32_t hidden,
                                                           uint32_t width)
{
    const uint32_t channel = blockIdx.x * kBlock + threadIdx.x;
    if (channel >= hidden)
        return;
    const uint64_t pw = uint64_t(hidden) * 3;
    const int64_t history_rows = int64_t(width) - 1;
    for (int64_t r = 0; r < history_rows; ++r) {
        const int64_t relative = int64_t(tokens) - history_rows + r;
        float u;
        if (relative < 0) {
            // An old row strictly below the one written: read before it is
            // overwritten, as in short_conv_kernel.
            u = history[uint64_t(relative + history_rows) * hidden + channel];
        } else {
            const float *p = projection + uint64_t(relative) * pw + channel;
            u = p[0] * p[2 * uint64_t(hidden)];
        }
        history[uint64_t(r) * hidden + channel] = u;
    }
}

}  // namespace

// ---- launches ----------------------------------------------------------

void launch_copy(hipStream_t stream, float *dst, const float *src, size_t count)
{
    if (count)
        copy_kernel<<<grid_for((count + 3) / 4), kBlock, 0, stream>>>(dst, src, count);
}

void launch_rect_copy(hipStream_t stream, float *dst, const float *src, const RectCopy &rect)
{
    if (rect.rows && rect.columns)
        rect_copy_kernel<<<grid_for(rect.rows, 1), kBlock, 0, stream>>>(dst, src, rect);
}

void launch_gather_rows(hipStream_t stream, float *out, const float *table, const float *ids,
                        uint32_t count, uint32_t rows, uint64_t columns)
{
    if (count && columns)
        gather_rows_kernel<<<grid_for(count, 1), kBlock, 0, stream>>>(out, table, ids, count,
                                                                      rows, columns);
}

void launch_gather_columns(hipStream_t stream, float *out, const float *in, const uint32_t *cols,
                           uint64_t rows, uint64_t width, uint32_t count)
{
    if (rows && count)
        gather_columns_kernel<<<grid_for(rows * count), kBlock, 0, stream>>>(out, in, cols, rows,
                                                                             width, count);
}

namespace {

// Ranges per row of the wide-row path, or 0 when one block per row is used.
uint32_t argmax_ranges(uint32_t rows, uint32_t width)
{
    const uint32_t ranges = (width + kArgmaxRange - 1) / kArgmaxRange;
    return (ranges >= 2 && rows <= 64) ? ranges : 0;
}

}  // namespace

size_t argmax_scratch_bytes(uint32_t rows, uint32_t width)
{
    return size_t(argmax_ranges(rows, width)) * rows * sizeof(Candidate);
}

void launch_argmax(hipStream_t stream, float *out, const float *in, uint32_t rows, uint32_t width,
                   const uint64_t *mask, void *scratch, float *copy)
{
    if (!rows)
        return;
    if (const uint32_t ranges = argmax_ranges(rows, width)) {
        Candidate *partial = static_cast<Candidate *>(scratch);
        argmax_range_kernel<<<rows * ranges, kArgmaxBlock, 0, stream>>>(partial, in, width,
                                                                       ranges, mask);
        if (ranges <= 64)
            argmax_final_wave_kernel<<<rows, 64, 0, stream>>>(out, copy, partial, ranges);
        else
            argmax_final_kernel<<<rows, kArgmaxBlock, 0, stream>>>(out, copy, partial, ranges);
        return;
    }
    argmax_kernel<<<grid_for(rows, 1), kArgmaxBlock, 0, stream>>>(out, copy, in, rows, width,
                                                                  mask);
}

void launch_argmax_candidates(hipStream_t stream, float *out, float *copy,
                              const Candidate *candidates, uint32_t count)
{
    // One wave up to 64 candidates (512, the 1.2B-shape head's, measured the
    // same with either kernel).
    if (count <= 64)
        argmax_final_wave_kernel<<<1, 64, 0, stream>>>(out, copy, candidates, count);
    else
        argmax_final_kernel<<<1, kArgmaxBlock, 0, stream>>>(out, copy, candidates, count);
}

void launch_binary(hipStream_t stream, int op, float *out, const float *left, const float *right,
                   size_t count)
{
    if (!count)
        return;
    if (op == 0)
        binary_kernel<0><<<grid_for(count), kBlock, 0, stream>>>(out, left, right, count);
    else
        binary_kernel<1><<<grid_for(count), kBlock, 0, stream>>>(out, left, right, count);
}

void launch_linear(hipStream_t stream, float *out, const float *x, const float *w, uint32_t m,
                   uint32_t n, uint32_t k)
{
    if (uint64_t(m) * n)
        linear_kernel<<<grid_for(uint64_t(m) * n, kBlock / 64), kBlock, 0, stream>>>(out, x, w,
                                                                                   m, n, k);
}

void launch_row_rms(hipStream_t stream, float *out, float *sum, const float *left,
                    const float *right, const float *weight, uint64_t rows, uint32_t width,
                    float epsilon)
{
    if (!rows || !width)
        return;
    if (sum)
        row_rms_kernel<true><<<grid_for(rows, 1), kBlock, 0, stream>>>(out, sum, left, right,
                                                                       weight, rows, width,
                                                                       epsilon);
    else
        row_rms_kernel<false><<<grid_for(rows, 1), kBlock, 0, stream>>>(out, nullptr, left,
                                                                        nullptr, weight, rows,
                                                                        width, epsilon);
}

void launch_head_rms(hipStream_t stream, float *out, const float *in, const float *weight,
                     uint64_t segments, uint32_t head_dim, float epsilon)
{
    if (segments)
        head_rms_kernel<<<grid_for(segments, kBlock / 64), kBlock, 0, stream>>>(
            out, in, weight, segments, head_dim, epsilon);
}

void launch_rotary(hipStream_t stream, float *out, const float *in, const Positions &positions,
                   uint64_t tokens, uint32_t heads, uint32_t head_dim, float theta)
{
    const uint64_t total = tokens * heads * (head_dim / 2);
    if (total)
        rotary_kernel<<<grid_for(total), kBlock, 0, stream>>>(out, in, positions, tokens, heads,
                                                               head_dim, theta);
}

void launch_qk_norm_rope_table(hipStream_t stream, float *query_out, float *key_out,
                               const float *query, const float *key, const float *query_weight,
                               const float *key_weight, const float *table, uint64_t first,
                               uint64_t tokens, uint32_t query_heads, uint32_t key_heads,
                               uint32_t head_dim, float epsilon)
{
    const uint64_t segments = tokens * (query_heads + key_heads);
    if (segments)
        qk_norm_rope_table_kernel<<<grid_for(segments, kBlock / 64), kBlock, 0, stream>>>(
            query_out, key_out, query, key, query_weight, key_weight, table, first, tokens,
            query_heads, key_heads, head_dim, epsilon);
}

void launch_qk_norm_rope(hipStream_t stream, float *query_out, float *key_out, const float *query,
                         const float *key, const float *query_weight, const float *key_weight,
                         const Positions &positions, uint64_t tokens, uint32_t query_heads,
                         uint32_t key_heads, uint32_t head_dim, float theta, float epsilon)
{
    const uint64_t segments = tokens * (query_heads + key_heads);
    if (segments)
        qk_norm_rope_kernel<<<grid_for(segments, kBlock / 64), kBlock, 0, stream>>>(
            query_out, key_out, query, key, query_weight, key_weight, positions, tokens,
            query_heads, key_heads, head_dim, theta, epsilon);
}

namespace {

// Key ranges of the split path, or 0 when one block per (token, query head)
// already fills the device or the ranges would be too few to pay for the
// combine launch.
uint32_t gqa_splits(const GqaShape &g)
{
    const uint64_t pairs = g.tokens * g.query_heads;
    const uint64_t longest = g.initial_len + g.tokens;
    const uint64_t splits = (longest + kSplitKeys - 1) / kSplitKeys;
    if (pairs >= 1024 || splits < 2 || splits > kSplitMaxRanges ||
        gqa_split_lds(g.group, g.head_dim) > kSplitMaxLds ||
        splits * g.tokens * g.key_value_heads > (uint64_t(1) << 31))
        return 0;
    return uint32_t(splits);
}

// The fp32 matrix-core prefill kernel serves heads of 16..kFlashMaxDim
// dimensions in steps of 16, groups of at most kFlashRows query heads, and
// 16-byte aligned operands (its float4 loads and stores).
bool flash_served(const GqaShape &g, const float *out, const float *query, const float *key_cache,
                  const float *value_cache)
{
    auto aligned = [](const float *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    return g.head_dim && g.head_dim % 16 == 0 && g.head_dim <= kFlashMaxDim && g.group >= 1 &&
           g.group <= kFlashRows && aligned(out) && aligned(query) && aligned(key_cache) &&
           aligned(value_cache);
}

template <int D>
void launch_flash_d(hipStream_t stream, float *out, const float *query, const float *key_cache,
                    const float *value_cache, const GqaShape &g)
{
    const uint32_t tile_tokens = kFlashRows / g.group;
    const uint64_t token_tiles = (g.tokens + tile_tokens - 1) / tile_tokens;
    gqa_flash_kernel<D><<<unsigned(token_tiles * g.key_value_heads), 64 * kFlashWaves,
                          flash_lds_bytes<D>(), stream>>>(out, query, key_cache, value_cache, g,
                                                          tile_tokens, uint32_t(token_tiles));
}

void launch_flash(hipStream_t stream, float *out, const float *query, const float *key_cache,
                  const float *value_cache, const GqaShape &g)
{
    switch (g.head_dim) {
    case 16: return launch_flash_d<16>(stream, out, query, key_cache, value_cache, g);
    case 32: return launch_flash_d<32>(stream, out, query, key_cache, value_cache, g);
    case 48: return launch_flash_d<48>(stream, out, query, key_cache, value_cache, g);
    case 64: return launch_flash_d<64>(stream, out, query, key_cache, value_cache, g);
    case 80: return launch_flash_d<80>(stream, out, query, key_cache, value_cache, g);
    case 96: return launch_flash_d<96>(stream, out, query, key_cache, value_cache, g);
    default: return launch_flash_d<112>(stream, out, query, key_cache, value_cache, g);
    }
}

}  // namespace

size_t gqa_scratch_bytes(const GqaShape &g)
{
    const uint32_t splits = gqa_splits(g);
    return splits ? size_t(g.tokens) * g.query_heads * splits * (g.head_dim + 2) * sizeof(float)
                  : 0;
}

void launch_gqa(hipStream_t stream, float *out, const float *query, const float *key,
                const float *value, float *key_cache, float *value_cache, const GqaShape &g,
                float *scratch)
{
    const uint64_t kv_width = uint64_t(g.key_value_heads) * g.head_dim;
    const uint64_t appended = g.tokens * kv_width;
    if (appended && key)
        cache_append_kernel<<<grid_for(appended), kBlock, 0, stream>>>(
            key_cache, value_cache, key, value, g.initial_len * kv_width, appended);
    const uint64_t blocks = g.tokens * g.query_heads;
    if (!blocks)
        return;
    const uint32_t splits = gqa_splits(g);
    if (splits) {
        gqa_split_kernel<<<unsigned(g.tokens * g.key_value_heads * splits), kBlock,
                           gqa_split_lds(g.group, g.head_dim), stream>>>(
            scratch, query, key_cache, value_cache, g, splits);
        const size_t combine_lds = (size_t(splits) + kBlock) * sizeof(float);
        gqa_combine_kernel<<<unsigned(blocks), kBlock, combine_lds, stream>>>(
            out, scratch, g.head_dim, splits);
        return;
    }
    if (flash_served(g, out, query, key_cache, value_cache))
        return launch_flash(stream, out, query, key_cache, value_cache, g);
    const size_t lds = (size_t(g.head_dim) + kKeyChunk + kBlock) * sizeof(float);
    gqa_kernel<<<unsigned(blocks), kBlock, lds, stream>>>(out, query, key_cache, value_cache, g);
}

uint32_t gqa_decode_splits(const DecodeAttention &p)
{
    const uint64_t splits = (p.position + 1 + kSplitKeys - 1) / kSplitKeys;
    if (splits > kSplitMaxRanges || p.head_dim % 4 || p.group == 0 ||
        gqa_split_lds(p.group, p.head_dim) > kSplitMaxLds)
        return 0;
    return uint32_t(splits);
}

size_t gqa_decode_scratch_bytes(const DecodeAttention &p)
{
    return size_t(p.query_heads) * gqa_decode_splits(p) * (p.head_dim + 2) * sizeof(float);
}

void launch_rotation_table(hipStream_t stream, float *table, uint64_t positions,
                           uint32_t head_dim, float theta)
{
    if (positions && head_dim >= 2)
        rotation_table_kernel<<<grid_for(positions * (head_dim / 2)), kBlock, 0, stream>>>(
            table, positions, head_dim, theta);
}

void launch_gqa_combine(hipStream_t stream, const DecodeAttention &p)
{
    gqa_combine_kernel<<<p.query_heads, kBlock, (size_t(p.splits) + kBlock) * sizeof(float),
                         stream>>>(p.out, p.partial, p.head_dim, p.splits);
}

void launch_gqa_decode(hipStream_t stream, const DecodeAttention &p, bool combine)
{
    gqa_decode_kernel<<<p.key_value_heads * p.splits, kBlock,
                        gqa_split_lds(p.group, p.head_dim), stream>>>(p);
    if (combine)
        launch_gqa_combine(stream, p);
}

void launch_short_conv(hipStream_t stream, float *out, const float *projection,
                       const float *kernel, float *history, uint64_t tokens, uint32_t hidden,
                       uint32_t width)
{
    // A channel walk over few tokens is one launch; many tokens spread over
    // (token, channel) threads, then the history rolls in a second launch.
    constexpr uint64_t kWalkTokens = 16;
    if (tokens <= kWalkTokens) {
        short_conv_kernel<<<(hidden + kBlock - 1) / kBlock, kBlock, 0, stream>>>(
            out, projection, kernel, history, tokens, hidden, width);
        return;
    }
    conv_tokens_kernel<<<grid_for(tokens * hidden), kBlock, 0, stream>>>(
        out, projection, kernel, history, tokens, hidden, width);
    conv_roll_kernel<<<(hidden + kBlock - 1) / kBlock, kBlock, 0, stream>>>(projection, history,
                                                                           tokens, hidden, width);
}

void launch_conv_step(hipStream_t stream, float *out, const float *projection,
                      const float *kernel, const float *history, float *next, uint32_t hidden,
                      uint32_t width)
{
    conv_step_kernel<<<(hidden + kBlock - 1) / kBlock, kBlock, 0, stream>>>(
        out, projection, kernel, history, next, hidden, width);
}

}  // namespace mfh
