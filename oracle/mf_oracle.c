/*
 * mf_oracle.c - CPU oracle for the packed-weight matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the parity tests, the
 * smoke check and the CPU-baseline leg of the bench compare the HIP backend
 * against.  Nothing in the product library links or calls it.
 *
 * It restates, loop for loop, the reference's scalar CPU backend:
 *   - crates/kernels-simd/src/lib.rs:31-208   (row dots, x86 scalar path)
 *   - crates/backend-cpu/src/packed.rs:11-466 (packed ops and admission)
 *   - crates/backend-cpu/src/storage.rs:322-327 (per-call finite scans)
 *   - crates/backend-cpu/src/dense.rs:24-53   (device token-id resolution)
 *   - crates/executor-core/src/loader.rs:408-421 (F16 -> F32 scale decode)
 * It is compiled with -O2 -ffp-contract=off and without fast-math, so every
 * f32 operation rounds exactly as the Rust code's does (Rust never contracts
 * a*b+c into an FMA and never reassociates).
 *
 * Pinning (tests/test_oracle.py): the ternary-v1-001 fixture vectors, the
 * kernels-simd unit-test invariants (0x55 -> 0, 0x00 -> -scale*sum(x),
 * 0xD2 pattern), exact closed forms on integer-valued inputs where every
 * f32 partial sum is exact, f64 dense brute force, pair == two singles
 * bitwise and swiglu_pair == pair + swiglu bitwise
 * (backend-cpu/tests/packed_pair_validation.rs:169-208).
 * SiLU uses the platform expf exactly as Rust's f32::exp does on
 * linux-gnu; no reference test pins libm values, so the SiLU bits are
 * parity-unpinned beyond tolerance tests.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "mf_oracle.h"

/* NF4_LEVELS, crates/kernels-simd/src/lib.rs:113-130 (same f32 values as
 * tools/converters/src/minifield_converters/quantization.py:22-42). */
const float MFO_NF4_LEVELS[16] = {
    -1.0f,        -0.6961928f,  -0.52507305f, -0.3949175f,
    -0.28444138f, -0.18477343f, -0.091050036f, 0.0f,
    0.0795803f,   0.1609302f,   0.2461123f,   0.33791524f,
    0.44070983f,  0.562617f,    0.72295684f,  1.0f,
};

/* scalar_group_dot, kernels-simd/src/lib.rs:73-81. */
static float ternary_group_dot(const uint8_t *codes, const float *x)
{
    float acc = 0.0f;
    for (int index = 0; index < 128; ++index) {
        unsigned code = (codes[index / 4] >> (2 * (index % 4))) & 0x3u;
        acc += ((float)code - 1.0f) * x[index];
    }
    return acc;
}

/* ternary_row_dot, kernels-simd/src/lib.rs:31-57. */
float mfo_ternary_row_dot(const uint8_t *codes, const float *scales, const float *x,
                          size_t k)
{
    float row = 0.0f;
    for (size_t group = 0; group < k / 128; ++group)
        row += scales[group] * ternary_group_dot(codes + group * 32, x + group * 128);
    return row;
}

/* nf4_group_dot, kernels-simd/src/lib.rs:174-183: two accumulators over the
 * even and odd weights, summed at the end. */
static float nf4_group_dot(const uint8_t *codes, const float *x)
{
    float lo = 0.0f, hi = 0.0f;
    for (int index = 0; index < 64; ++index) {
        uint8_t byte = codes[index];
        lo += MFO_NF4_LEVELS[byte & 0x0F] * x[2 * index];
        hi += MFO_NF4_LEVELS[byte >> 4] * x[2 * index + 1];
    }
    return lo + hi;
}

/* nf4_row_dot, kernels-simd/src/lib.rs:145-171. */
float mfo_nf4_row_dot(const uint8_t *codes, const float *scales, const float *x, size_t k)
{
    float row = 0.0f;
    for (size_t group = 0; group < k / 128; ++group)
        row += scales[group] * nf4_group_dot(codes + group * 64, x + group * 128);
    return row;
}

/* int8_row_dot, kernels-simd/src/lib.rs:191-208: note `dot * scale`
 * (the ternary and NF4 paths compute `scale * dot`; f32 multiply commutes
 * exactly, so only the accumulation order matters). */
float mfo_int8_row_dot(const uint8_t *codes, const float *scales, const float *x, size_t k)
{
    float total = 0.0f;
    for (size_t group = 0; group < k / 128; ++group) {
        float dot = 0.0f;
        for (int j = 0; j < 128; ++j)
            dot += (float)(int8_t)codes[group * 128 + j] * x[group * 128 + j];
        total += dot * scales[group];
    }
    return total;
}

typedef float (*row_dot_fn)(const uint8_t *, const float *, const float *, size_t);

static row_dot_fn row_dot_for(int format)
{
    switch (format) {
    case MFO_TERNARY: return mfo_ternary_row_dot;
    case MFO_NF4: return mfo_nf4_row_dot;
    default: return mfo_int8_row_dot;
    }
}

/* check_packed_operands, backend-cpu/src/packed.rs:177-220: K is the scales
 * width times 128 and the codes width picks the format.  INT8 streams are
 * scanned for the reserved 0x80 byte on every call, as the reference does. */
int mfo_packed_format(size_t rows, size_t code_width, size_t groups, const uint8_t *codes,
                      int *format)
{
    size_t inner = groups * 128;
    if (code_width == inner / 4) {
        *format = MFO_TERNARY;
    } else if (code_width == inner / 2) {
        *format = MFO_NF4;
    } else if (code_width == inner) {
        if (codes && memchr(codes, 0x80, rows * code_width) != NULL)
            return MFO_ERR_INVALID_ARGUMENT;
        *format = MFO_INT8;
    } else {
        return MFO_ERR_INVALID_SHAPE;
    }
    return MFO_OK;
}

/* check_f32_buffer's finite scan, backend-cpu/src/storage.rs:322-327. */
static int all_finite(const float *values, size_t count)
{
    for (size_t i = 0; i < count; ++i)
        if (!isfinite(values[i]))
            return 0;
    return 1;
}

/* CpuBackend::packed_linear, backend-cpu/src/packed.rs:96-170. */
int mfo_packed_linear(float *out, const float *x, size_t m, const uint8_t *codes,
                      const float *scales, size_t n, size_t code_width, size_t groups)
{
    int format = 0;
    if (!all_finite(x, m * groups * 128))
        return MFO_ERR_BACKEND_FAILURE;
    int status = mfo_packed_format(n, code_width, groups, codes, &format);
    if (status)
        return status;
    if (!all_finite(scales, n * groups) || !all_finite(out, m * n))
        return MFO_ERR_BACKEND_FAILURE;
    size_t k = groups * 128;
    row_dot_fn dot = row_dot_for(format);
    for (size_t row = 0; row < m; ++row) {
        for (size_t column = 0; column < n; ++column) {
            float acc = dot(codes + column * code_width, scales + column * groups,
                            x + row * k, k);
            if (!isfinite(acc))
                return MFO_ERR_BACKEND_FAILURE;
            out[row * n + column] = acc;
        }
    }
    return MFO_OK;
}

/* Row-parallel variant over output columns for large parity references.
 * Each output element is computed by the same row dot, so the bits equal
 * mfo_packed_linear's; only the finite scans are skipped. */
int mfo_packed_linear_rows(float *out, const float *x, size_t m, const uint8_t *codes,
                           const float *scales, size_t n, size_t code_width, size_t groups,
                           size_t column_begin, size_t column_end)
{
    int format = 0;
    int status = mfo_packed_format(n, code_width, groups, NULL, &format);
    if (status)
        return status;
    size_t k = groups * 128;
    row_dot_fn dot = row_dot_for(format);
    for (size_t row = 0; row < m; ++row)
        for (size_t column = column_begin; column < column_end && column < n; ++column)
            out[row * n + column] = dot(codes + column * code_width, scales + column * groups,
                                        x + row * k, k);
    return MFO_OK;
}

/* CpuBackend::packed_linear_pair, backend-cpu/src/packed.rs:226-272: both
 * operand sets are admitted before either output is written. */
int mfo_packed_linear_pair(float *out_a, float *out_b, const float *x, size_t m,
                           const uint8_t *codes_a, const float *scales_a,
                           const uint8_t *codes_b, const float *scales_b, size_t n,
                           size_t code_width, size_t groups)
{
    int format = 0;
    int status = mfo_packed_format(n, code_width, groups, codes_a, &format);
    if (!status)
        status = mfo_packed_format(n, code_width, groups, codes_b, &format);
    if (status)
        return status;
    status = mfo_packed_linear(out_a, x, m, codes_a, scales_a, n, code_width, groups);
    if (status)
        return status;
    return mfo_packed_linear(out_b, x, m, codes_b, scales_b, n, code_width, groups);
}

/* SiLU gate as the reference writes it: `(g * (1 / (1 + exp(-g)))) * u`
 * (backend-cpu/src/packed.rs:361-362, 433-434). */
static float swiglu_value(float g, float u)
{
    float sigmoid = 1.0f / (1.0f + expf(-g));
    return (g * sigmoid) * u;
}

/* CpuBackend::packed_swiglu_pair, backend-cpu/src/packed.rs:278-372. */
int mfo_packed_swiglu_pair(float *out, const float *x, size_t m, const uint8_t *codes_a,
                           const float *scales_a, const uint8_t *codes_b,
                           const float *scales_b, size_t n, size_t code_width, size_t groups)
{
    int format = 0;
    if (!all_finite(x, m * groups * 128))
        return MFO_ERR_BACKEND_FAILURE;
    int status = mfo_packed_format(n, code_width, groups, codes_a, &format);
    if (!status)
        status = mfo_packed_format(n, code_width, groups, codes_b, &format);
    if (status)
        return status;
    size_t k = groups * 128;
    row_dot_fn dot = row_dot_for(format);
    for (size_t row = 0; row < m; ++row) {
        const float *xr = x + row * k;
        for (size_t column = 0; column < n; ++column) {
            float gate = dot(codes_a + column * code_width, scales_a + column * groups, xr, k);
            float up = dot(codes_b + column * code_width, scales_b + column * groups, xr, k);
            float value = swiglu_value(gate, up);
            if (!isfinite(value))
                return MFO_ERR_BACKEND_FAILURE;
            out[row * n + column] = value;
        }
    }
    return MFO_OK;
}

/* CpuBackend::packed_swiglu_linear, backend-cpu/src/packed.rs:377-466: the
 * activation row is staged first, then fed to the same row dot. */
int mfo_packed_swiglu_linear(float *out, const float *gate, const float *up, size_t m,
                             const uint8_t *codes, const float *scales, size_t n,
                             size_t code_width, size_t groups)
{
    int format = 0;
    if (!all_finite(gate, m * groups * 128) || !all_finite(up, m * groups * 128))
        return MFO_ERR_BACKEND_FAILURE;
    int status = mfo_packed_format(n, code_width, groups, codes, &format);
    if (status)
        return status;
    size_t k = groups * 128;
    row_dot_fn dot = row_dot_for(format);
    float *activated = (float *)malloc(k * sizeof(float));
    if (!activated)
        return MFO_ERR_RESOURCE_LIMIT;
    for (size_t row = 0; row < m; ++row) {
        for (size_t i = 0; i < k; ++i) {
            float value = swiglu_value(gate[row * k + i], up[row * k + i]);
            if (!isfinite(value)) {
                free(activated);
                return MFO_ERR_BACKEND_FAILURE;
            }
            activated[i] = value;
        }
        for (size_t column = 0; column < n; ++column) {
            float acc = dot(codes + column * code_width, scales + column * groups, activated, k);
            if (!isfinite(acc)) {
                free(activated);
                return MFO_ERR_BACKEND_FAILURE;
            }
            out[row * n + column] = acc;
        }
    }
    free(activated);
    return MFO_OK;
}

/* CpuBackend::swiglu's elementwise value, for composing pair + swiglu. */
void mfo_swiglu(float *out, const float *gate, const float *up, size_t count)
{
    for (size_t i = 0; i < count; ++i)
        out[i] = swiglu_value(gate[i], up[i]);
}

/* resolve_token_ids for TokenIds::Device, backend-cpu/src/dense.rs:24-53:
 * finite, non-negative, integral and < 2^24, else None (-1 here). */
void mfo_resolve_device_ids(const float *values, size_t count, int64_t *ids)
{
    for (size_t i = 0; i < count; ++i) {
        float v = values[i];
        if (isfinite(v) && v >= 0.0f && floorf(v) == v && v < 16777216.0f)
            ids[i] = (int64_t)v;
        else
            ids[i] = -1;
    }
}

/* CpuBackend::packed_gather_rows, backend-cpu/src/packed.rs:11-91.  An id of
 * -1 is a None row and fills NaN; an id >= rows fails OutOfBounds. */
int mfo_packed_gather_rows(float *out, const uint8_t *codes, const float *scales, size_t rows,
                           size_t code_width, size_t groups, const int64_t *ids, size_t count)
{
    int format = 0;
    int status = mfo_packed_format(rows, code_width, groups, codes, &format);
    if (status)
        return status;
    size_t inner = groups * 128;
    for (size_t destination = 0; destination < count; ++destination) {
        float *dst = out + destination * inner;
        if (ids[destination] < 0) {
            for (size_t i = 0; i < inner; ++i)
                dst[i] = NAN;
            continue;
        }
        size_t source = (size_t)ids[destination];
        if (source >= rows)
            return MFO_ERR_OUT_OF_BOUNDS;
        const uint8_t *row_codes = codes + source * code_width;
        const float *row_scales = scales + source * groups;
        for (size_t index = 0; index < inner; ++index) {
            size_t group = index / 128, within = index % 128;
            float weight;
            if (format == MFO_TERNARY) {
                unsigned code = (row_codes[group * 32 + within / 4] >> (2 * (within % 4))) & 3u;
                weight = (float)code - 1.0f;
            } else if (format == MFO_INT8) {
                weight = (float)(int8_t)row_codes[index];
            } else {
                uint8_t byte = row_codes[group * 64 + within / 2];
                weight = MFO_NF4_LEVELS[(within % 2 == 0) ? (byte & 0x0F) : (byte >> 4)];
            }
            dst[index] = weight * row_scales[group];
        }
    }
    return MFO_OK;
}

/* f16_to_f32, crates/executor-core/src/loader.rs:408-421: subnormals as
 * mantissa * 2^-24 (exact in f32), infinities/NaN keep their payload, normal
 * values re-bias the exponent; the sign bit is OR-ed in last. */
float mfo_f16_to_f32(uint16_t bits)
{
    uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    uint32_t exponent = (bits >> 10) & 0x1Fu;
    uint32_t mantissa = bits & 0x3FFu;
    float value;
    uint32_t out;
    if (exponent == 0) {
        value = (float)mantissa * 5.9604644775390625e-08f; /* 2^-24 */
        memcpy(&out, &value, sizeof out);
    } else if (exponent == 31) {
        out = 0x7F800000u | (mantissa << 13);
    } else {
        out = ((exponent + 112) << 23) | (mantissa << 13);
    }
    out |= sign;
    memcpy(&value, &out, sizeof value);
    return value;
}

/* Dense f64 brute force of the dequantized matvec, for tolerance checks that
 * do not share the oracle's loop structure. */
void mfo_dense_f64(double *out, const float *x, size_t m, const float *weights, size_t n,
                   size_t k)
{
    for (size_t row = 0; row < m; ++row)
        for (size_t column = 0; column < n; ++column) {
            double acc = 0.0;
            for (size_t i = 0; i < k; ++i)
                acc += (double)x[row * k + i] * (double)weights[column * k + i];
            out[row * n + column] = acc;
        }
}
