/*
 * mf_oracle.h - CPU oracle of the packed-weight path (test infrastructure).
 * Status codes equal mfh_status (include/minifield_hip.h) and ExecutorError
 * (crates/engine-api/src/error.rs:10-28).
 */
#ifndef MF_ORACLE_H
#define MF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#define MFO_OK 0
#define MFO_ERR_INVALID_ARGUMENT 1
#define MFO_ERR_INVALID_SHAPE 2
#define MFO_ERR_OUT_OF_BOUNDS 6
#define MFO_ERR_RESOURCE_LIMIT 8
#define MFO_ERR_BACKEND_FAILURE 17

#define MFO_TERNARY 0
#define MFO_NF4 1
#define MFO_INT8 2

extern const float MFO_NF4_LEVELS[16];

float mfo_ternary_row_dot(const uint8_t *codes, const float *scales, const float *x, size_t k);
float mfo_nf4_row_dot(const uint8_t *codes, const float *scales, const float *x, size_t k);
float mfo_int8_row_dot(const uint8_t *codes, const float *scales, const float *x, size_t k);
int mfo_packed_format(size_t rows, size_t code_width, size_t groups, const uint8_t *codes,
                      int *format);
int mfo_packed_linear(float *out, const float *x, size_t m, const uint8_t *codes,
                      const float *scales, size_t n, size_t code_width, size_t groups);
int mfo_packed_linear_rows(float *out, const float *x, size_t m, const uint8_t *codes,
                           const float *scales, size_t n, size_t code_width, size_t groups,
                           size_t column_begin, size_t column_end);
int mfo_packed_linear_pair(float *out_a, float *out_b, const float *x, size_t m,
                           const uint8_t *codes_a, const float *scales_a,
                           const uint8_t *codes_b, const float *scales_b, size_t n,
                           size_t code_width, size_t groups);
int mfo_packed_swiglu_pair(float *out, const float *x, size_t m, const uint8_t *codes_a,
                           const float *scales_a, const uint8_t *codes_b,
                           const float *scales_b, size_t n, size_t code_width, size_t groups);
int mfo_packed_swiglu_linear(float *out, const float *gate, const float *up, size_t m,
                             const uint8_t *codes, const float *scales, size_t n,
                             size_t code_width, size_t groups);
void mfo_swiglu(float *out, const float *gate, const float *up, size_t count);
void mfo_resolve_device_ids(const float *values, size_t count, int64_t *ids);
int mfo_packed_gather_rows(float *out, const uint8_t *codes, const float *scales, size_t rows,
                           size_t code_width, size_t groups, const int64_t *ids, size_t count);
float mfo_f16_to_f32(uint16_t bits);
void mfo_dense_f64(double *out, const float *x, size_t m, const float *weights, size_t n,
                   size_t k);

/* Dense LFM2 operations (mf_dense_oracle.c). */
int mfo_row_rms_norm(float *out, const float *in, const float *weight, size_t rows,
                     size_t width, float epsilon);
int mfo_head_rms_norm(float *out, const float *in, const float *weight, size_t tokens,
                      size_t heads, size_t head_dim, float epsilon);
int mfo_split_half_rotary(float *out, const float *in, const uint64_t *positions, size_t tokens,
                          size_t heads, size_t head_dim, float theta);
int mfo_qk_norm_rope(float *query_out, float *key_out, const float *query, const float *key,
                     const float *query_weight, const float *key_weight,
                     const uint64_t *positions, size_t tokens, size_t query_heads,
                     size_t key_heads, size_t head_dim, float theta, float epsilon);
int mfo_elementwise(float *out, const float *left, const float *right, size_t count, int op);
int mfo_linear(float *out, const float *x, const float *w, size_t m, size_t n, size_t k);
void mfo_argmax(float *out, const float *in, size_t rows, size_t width, const uint64_t *mask);
int mfo_gather_rows(float *out, const float *table, size_t rows, size_t columns,
                    const int64_t *ids, size_t count);
int mfo_causal_gqa(float *out, const float *query, const float *key, const float *value,
                   float *key_cache, float *value_cache, uint64_t *cache_len, size_t tokens,
                   size_t query_heads, size_t key_heads, size_t head_dim);
/* mfo_causal_gqa with the scores cached per (token, query head) and the
 * units spread over `threads` threads: the same bits and statuses. */
int mfo_causal_gqa_cached(float *out, const float *query, const float *key, const float *value,
                          float *key_cache, float *value_cache, uint64_t *cache_len,
                          size_t tokens, size_t query_heads, size_t key_heads, size_t head_dim,
                          size_t threads);
int mfo_gated_short_convolution(float *out, const float *projection, const float *kernel,
                                float *history, size_t tokens, size_t hidden, size_t width);

#endif
