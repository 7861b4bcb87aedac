/*
 * mf_dense_oracle.c - CPU oracle of the dense LFM2 operations.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the parity tests compare the HIP
 * backend's dense operations against.  Nothing in the product library links
 * or calls it.
 *
 * Each function restates, loop for loop, the reference's scalar CPU backend
 * for one operation (file:line on each function).  Built with
 * -ffp-contract=off and without fast-math, so every f32 operation rounds as
 * the Rust code's does; f64 pow/sin/cos and f32 expf come from the platform
 * libm exactly as Rust's f64::powf/sin/cos and f32::exp do on linux-gnu.
 * Admission (shapes, dtypes) is the caller's; the functions keep the
 * reference's value checks and return MFO_ERR_BACKEND_FAILURE where the
 * reference raises BackendFailure on a non-finite value.
 *
 * Pinning (tests/test_dense_oracle.py): the model-ops-001 and
 * inference-ops-001 fixture cases (NumPy f64 oracles of the reference),
 * the cr02a rounding sentinels (exact output bits for rotary and the
 * convolution), and closed forms: rotation at position 0 is the identity,
 * RMS of a constant row, attention over one visible key returns its value
 * row exactly, a one-hot convolution kernel selects one u value exactly,
 * and brute-force argmax.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "mf_oracle.h"

/* CpuBackend::row_rms_norm, crates/backend-cpu/src/normalization_rotary.rs:53-80. */
int mfo_row_rms_norm(float *out, const float *in, const float *weight, size_t rows,
                     size_t width, float epsilon)
{
    if (width == 0)
        return MFO_OK;
    const float width_f = (float)width;
    for (size_t row = 0; row < rows; ++row) {
        const size_t start = row * width;
        float squared_sum = 0.0f;
        for (size_t c = 0; c < width; ++c)
            squared_sum += in[start + c] * in[start + c];
        const float reciprocal = 1.0f / sqrtf(squared_sum / width_f + epsilon);
        if (!isfinite(reciprocal))
            return MFO_ERR_BACKEND_FAILURE;
        for (size_t c = 0; c < width; ++c) {
            const float normalized = in[start + c] * reciprocal;
            const float value = normalized * weight[c];
            if (!isfinite(value))
                return MFO_ERR_BACKEND_FAILURE;
            out[start + c] = value;
        }
    }
    return MFO_OK;
}

/* CpuBackend::head_rms_norm, normalization_rotary.rs:122-152. */
int mfo_head_rms_norm(float *out, const float *in, const float *weight, size_t tokens,
                      size_t heads, size_t head_dim, float epsilon)
{
    const float dim_f = (float)head_dim;
    const size_t packed_width = heads * head_dim;
    for (size_t token = 0; token < tokens; ++token) {
        for (size_t head = 0; head < heads; ++head) {
            const size_t start = token * packed_width + head * head_dim;
            float squared_sum = 0.0f;
            for (size_t c = 0; c < head_dim; ++c)
                squared_sum += in[start + c] * in[start + c];
            const float reciprocal = 1.0f / sqrtf(squared_sum / dim_f + epsilon);
            if (!isfinite(reciprocal))
                return MFO_ERR_BACKEND_FAILURE;
            for (size_t c = 0; c < head_dim; ++c) {
                const float normalized = in[start + c] * reciprocal;
                const float value = normalized * weight[c];
                if (!isfinite(value))
                    return MFO_ERR_BACKEND_FAILURE;
                out[start + c] = value;
            }
        }
    }
    return MFO_OK;
}

/* The per-column coefficients shared by split_half_rotary and qk_norm_rope
 * (normalization_rotary.rs:197-201, 346-350). */
static void rotation(float position, size_t column, size_t head_dim, float theta, float *cosine,
                     float *sine)
{
    const double exponent = -2.0 * (double)column / (double)head_dim;
    const float frequency = (float)pow((double)theta, exponent);
    const float angle = position * frequency;
    *sine = (float)sin((double)angle);
    *cosine = (float)cos((double)angle);
}

/* CpuBackend::split_half_rotary, normalization_rotary.rs:180-218. */
int mfo_split_half_rotary(float *out, const float *in, const uint64_t *positions, size_t tokens,
                          size_t heads, size_t head_dim, float theta)
{
    const size_t half = head_dim / 2;
    const size_t packed_width = heads * head_dim;
    for (size_t token = 0; token < tokens; ++token) {
        const float position = (float)positions[token];
        for (size_t head = 0; head < heads; ++head) {
            const size_t start = token * packed_width + head * head_dim;
            for (size_t c = 0; c < half; ++c) {
                float cosine, sine;
                rotation(position, c, head_dim, theta, &cosine, &sine);
                const float first = in[start + c];
                const float second = in[start + half + c];
                const float rotated_first = first * cosine - second * sine;
                const float rotated_second = second * cosine + first * sine;
                if (!isfinite(rotated_first) || !isfinite(rotated_second))
                    return MFO_ERR_BACKEND_FAILURE;
                out[start + c] = rotated_first;
                out[start + half + c] = rotated_second;
            }
        }
    }
    return MFO_OK;
}

/* One side of CpuBackend::qk_norm_rope, normalization_rotary.rs:310-366. */
static int norm_rope_side(float *out, const float *in, const float *weight,
                          const uint64_t *positions, size_t tokens, size_t heads,
                          size_t head_dim, float theta, float epsilon, float *normed)
{
    const size_t half = head_dim / 2;
    const size_t packed_width = heads * head_dim;
    const float dim_f = (float)head_dim;
    for (size_t token = 0; token < tokens; ++token) {
        const float position = (float)positions[token];
        for (size_t head = 0; head < heads; ++head) {
            const size_t start = token * packed_width + head * head_dim;
            float squared_sum = 0.0f;
            for (size_t c = 0; c < head_dim; ++c)
                squared_sum += in[start + c] * in[start + c];
            const float reciprocal = 1.0f / sqrtf(squared_sum / dim_f + epsilon);
            if (!isfinite(reciprocal))
                return MFO_ERR_BACKEND_FAILURE;
            for (size_t c = 0; c < head_dim; ++c)
                normed[c] = in[start + c] * reciprocal * weight[c];
            for (size_t c = 0; c < half; ++c) {
                float cosine, sine;
                rotation(position, c, head_dim, theta, &cosine, &sine);
                const float first = normed[c];
                const float second = normed[half + c];
                const float rotated_first = first * cosine - second * sine;
                const float rotated_second = second * cosine + first * sine;
                if (!isfinite(rotated_first) || !isfinite(rotated_second))
                    return MFO_ERR_BACKEND_FAILURE;
                out[start + c] = rotated_first;
                out[start + half + c] = rotated_second;
            }
        }
    }
    return MFO_OK;
}

/* CpuBackend::qk_norm_rope, normalization_rotary.rs:246-369. */
int mfo_qk_norm_rope(float *query_out, float *key_out, const float *query, const float *key,
                     const float *query_weight, const float *key_weight,
                     const uint64_t *positions, size_t tokens, size_t query_heads,
                     size_t key_heads, size_t head_dim, float theta, float epsilon)
{
    float *normed = (float *)malloc((head_dim ? head_dim : 1) * sizeof(float));
    if (!normed)
        return MFO_ERR_RESOURCE_LIMIT;
    int status = norm_rope_side(query_out, query, query_weight, positions, tokens, query_heads,
                                head_dim, theta, epsilon, normed);
    if (status == MFO_OK)
        status = norm_rope_side(key_out, key, key_weight, positions, tokens, key_heads, head_dim,
                                theta, epsilon, normed);
    free(normed);
    return status;
}

/* CpuBackend::elementwise for add (op 0) and multiply (op 1),
 * crates/backend-cpu/src/dense.rs:153-198. */
int mfo_elementwise(float *out, const float *left, const float *right, size_t count, int op)
{
    for (size_t i = 0; i < count; ++i) {
        const float value = op == 0 ? left[i] + right[i] : left[i] * right[i];
        if (!isfinite(value))
            return MFO_ERR_BACKEND_FAILURE;
        out[i] = value;
    }
    return MFO_OK;
}

/* CpuBackend::linear, dense.rs:237-269: sequential f32 accumulation in
 * increasing k. */
int mfo_linear(float *out, const float *x, const float *w, size_t m, size_t n, size_t k)
{
    for (size_t row = 0; row < m; ++row) {
        for (size_t col = 0; col < n; ++col) {
            float acc = 0.0f;
            for (size_t i = 0; i < k; ++i)
                acc += x[row * k + i] * w[col * k + i];
            if (!isfinite(acc))
                return MFO_ERR_BACKEND_FAILURE;
            out[row * n + col] = acc;
        }
    }
    return MFO_OK;
}

/* CpuBackend::argmax and argmax_masked, dense.rs:390-472; `mask` null for
 * the unmasked form. */
void mfo_argmax(float *out, const float *in, size_t rows, size_t width, const uint64_t *mask)
{
    for (size_t row = 0; row < rows; ++row) {
        const float *values = in + row * width;
        float best = -INFINITY;
        size_t best_index = mask ? SIZE_MAX : 0;
        int poisoned = 0;
        for (size_t i = 0; i < width; ++i) {
            if (mask && !((mask[i / 64] >> (i % 64)) & 1))
                continue;
            const float v = values[i];
            if (!isfinite(v))
                poisoned = 1;
            else if (v > best || (mask && v == best && i < best_index)) {
                best = v;
                best_index = i;
            }
        }
        out[row] = (poisoned || best_index == SIZE_MAX) ? NAN : (float)best_index;
    }
}

/* CpuBackend::gather_rows, dense.rs:81-107, over resolved ids (-1 = None,
 * as produced by mfo_resolve_device_ids). */
int mfo_gather_rows(float *out, const float *table, size_t rows, size_t columns,
                    const int64_t *ids, size_t count)
{
    for (size_t r = 0; r < count; ++r) {
        float *dst = out + r * columns;
        if (ids[r] < 0) {
            for (size_t c = 0; c < columns; ++c)
                dst[c] = NAN;
            continue;
        }
        if ((uint64_t)ids[r] >= rows)
            return MFO_ERR_OUT_OF_BOUNDS;
        memcpy(dst, table + (size_t)ids[r] * columns, columns * sizeof(float));
    }
    return MFO_OK;
}

/* CpuBackend::gqa_score, attention_convolution.rs:190-216. */
static float gqa_score(const float *query, const float *key, const float *key_cache,
                       size_t initial_len, size_t key_index, size_t query_start, size_t kv_head,
                       size_t kv_width, size_t head_dim, float scale)
{
    float dot = 0.0f;
    for (size_t d = 0; d < head_dim; ++d) {
        const float key_value =
            key_index < initial_len
                ? key_cache[key_index * kv_width + kv_head * head_dim + d]
                : key[(key_index - initial_len) * kv_width + kv_head * head_dim + d];
        dot += query[query_start + d] * key_value;
    }
    return dot * scale;
}

/* CpuBackend::causal_gqa, attention_convolution.rs:85-186.  Reads the new
 * rows from key/value, appends them to the caches at row *cache_len and
 * advances *cache_len. */
int mfo_causal_gqa(float *out, const float *query, const float *key, const float *value,
                   float *key_cache, float *value_cache, uint64_t *cache_len, size_t tokens,
                   size_t query_heads, size_t key_heads, size_t head_dim)
{
    const size_t group = query_heads / key_heads;
    const size_t query_width = query_heads * head_dim;
    const size_t kv_width = key_heads * head_dim;
    const size_t initial_len = (size_t)*cache_len;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const size_t staged_count = tokens * query_width;
    float *staged = (float *)malloc((staged_count ? staged_count : 1) * sizeof(float));
    if (!staged)
        return MFO_ERR_RESOURCE_LIMIT;
    for (size_t token = 0; token < tokens; ++token) {
        const size_t visible = initial_len + token + 1;
        for (size_t qh = 0; qh < query_heads; ++qh) {
            const size_t kv_head = qh / group;
            const size_t query_start = token * query_width + qh * head_dim;
            float maximum = -INFINITY;
            for (size_t j = 0; j < visible; ++j) {
                const float s = gqa_score(query, key, key_cache, initial_len, j, query_start,
                                          kv_head, kv_width, head_dim, scale);
                if (!isfinite(s)) {
                    free(staged);
                    return MFO_ERR_BACKEND_FAILURE;
                }
                maximum = fmaxf(maximum, s);
            }
            float denominator = 0.0f;
            for (size_t j = 0; j < visible; ++j)
                denominator += expf(gqa_score(query, key, key_cache, initial_len, j, query_start,
                                              kv_head, kv_width, head_dim, scale) -
                                    maximum);
            if (!isfinite(denominator) || denominator <= 0.0f) {
                free(staged);
                return MFO_ERR_BACKEND_FAILURE;
            }
            for (size_t d = 0; d < head_dim; ++d) {
                float weighted = 0.0f;
                for (size_t j = 0; j < visible; ++j) {
                    const float s = gqa_score(query, key, key_cache, initial_len, j, query_start,
                                              kv_head, kv_width, head_dim, scale);
                    const float probability = expf(s - maximum) / denominator;
                    const float v =
                        j < initial_len
                            ? value_cache[j * kv_width + kv_head * head_dim + d]
                            : value[(j - initial_len) * kv_width + kv_head * head_dim + d];
                    weighted += probability * v;
                }
                if (!isfinite(weighted)) {
                    free(staged);
                    return MFO_ERR_BACKEND_FAILURE;
                }
                staged[token * query_width + qh * head_dim + d] = weighted;
            }
        }
    }
    memcpy(key_cache + initial_len * kv_width, key, tokens * kv_width * sizeof(float));
    memcpy(value_cache + initial_len * kv_width, value, tokens * kv_width * sizeof(float));
    memcpy(out, staged, tokens * query_width * sizeof(float));
    free(staged);
    *cache_len = initial_len + tokens;
    return MFO_OK;
}

/* mfo_causal_gqa with each (token, query head)'s scores computed once and
 * the units spread over `threads` threads.  The reference recomputes
 * gqa_score in each of its three passes (attention_convolution.rs:139-176),
 * but gqa_score is a pure function of its inputs (:190-216) and exp() of the
 * same argument is the same value, so caching the scores and their
 * exponentials changes no bit: every sum is taken in the reference's order
 * over the same values.  A non-finite score, denominator or output fails
 * the call with the same status, and then nothing is written. */
struct gqa_job {
    float *staged;
    const float *query, *key, *value, *key_cache, *value_cache;
    size_t tokens, query_heads, group, head_dim, query_width, kv_width, initial_len;
    float scale;
    size_t next;  /* next unit, taken under `lock` */
    int status;
    pthread_mutex_t lock;
};

static void *gqa_worker(void *arg)
{
    struct gqa_job *job = (struct gqa_job *)arg;
    const size_t most = job->initial_len + job->tokens;
    float *scores = (float *)malloc((most ? most : 1) * sizeof(float));
    float *weights = (float *)malloc((most ? most : 1) * sizeof(float));
    if (!scores || !weights) {
        pthread_mutex_lock(&job->lock);
        job->status = MFO_ERR_RESOURCE_LIMIT;
        pthread_mutex_unlock(&job->lock);
        free(scores);
        free(weights);
        return NULL;
    }
    const size_t units = job->tokens * job->query_heads;
    for (;;) {
        pthread_mutex_lock(&job->lock);
        const size_t unit = job->next++;
        const int stop = job->status != MFO_OK;
        pthread_mutex_unlock(&job->lock);
        if (stop || unit >= units)
            break;
        const size_t token = unit / job->query_heads, qh = unit % job->query_heads;
        const size_t kv_head = qh / job->group;
        const size_t visible = job->initial_len + token + 1;
        const size_t query_start = token * job->query_width + qh * job->head_dim;
        int status = MFO_OK;
        float maximum = -INFINITY;
        for (size_t j = 0; j < visible && !status; ++j) {
            scores[j] = gqa_score(job->query, job->key, job->key_cache, job->initial_len, j,
                                  query_start, kv_head, job->kv_width, job->head_dim, job->scale);
            if (!isfinite(scores[j]))
                status = MFO_ERR_BACKEND_FAILURE;
            maximum = fmaxf(maximum, scores[j]);
        }
        float denominator = 0.0f;
        for (size_t j = 0; j < visible && !status; ++j) {
            weights[j] = expf(scores[j] - maximum);
            denominator += weights[j];
        }
        if (!status && (!isfinite(denominator) || denominator <= 0.0f))
            status = MFO_ERR_BACKEND_FAILURE;
        for (size_t d = 0; d < job->head_dim && !status; ++d) {
            float weighted = 0.0f;
            for (size_t j = 0; j < visible; ++j) {
                const float probability = weights[j] / denominator;
                const float v =
                    j < job->initial_len
                        ? job->value_cache[j * job->kv_width + kv_head * job->head_dim + d]
                        : job->value[(j - job->initial_len) * job->kv_width +
                                     kv_head * job->head_dim + d];
                weighted += probability * v;
            }
            if (!isfinite(weighted))
                status = MFO_ERR_BACKEND_FAILURE;
            job->staged[query_start + d] = weighted;
        }
        if (status) {
            pthread_mutex_lock(&job->lock);
            job->status = status;
            pthread_mutex_unlock(&job->lock);
        }
    }
    free(scores);
    free(weights);
    return NULL;
}

int mfo_causal_gqa_cached(float *out, const float *query, const float *key, const float *value,
                          float *key_cache, float *value_cache, uint64_t *cache_len,
                          size_t tokens, size_t query_heads, size_t key_heads, size_t head_dim,
                          size_t threads)
{
    struct gqa_job job;
    memset(&job, 0, sizeof job);
    job.group = query_heads / key_heads;
    job.query_width = query_heads * head_dim;
    job.kv_width = key_heads * head_dim;
    job.initial_len = (size_t)*cache_len;
    job.scale = 1.0f / sqrtf((float)head_dim);
    job.query = query;
    job.key = key;
    job.value = value;
    job.key_cache = key_cache;
    job.value_cache = value_cache;
    job.tokens = tokens;
    job.query_heads = query_heads;
    job.head_dim = head_dim;
    job.status = MFO_OK;
    const size_t staged_count = tokens * job.query_width;
    job.staged = (float *)malloc((staged_count ? staged_count : 1) * sizeof(float));
    if (!job.staged)
        return MFO_ERR_RESOURCE_LIMIT;
    pthread_mutex_init(&job.lock, NULL);
    if (threads < 1)
        threads = 1;
    if (threads > 64)
        threads = 64;
    pthread_t pool[64];
    size_t started = 0;
    for (; started < threads; ++started)
        if (pthread_create(&pool[started], NULL, gqa_worker, &job) != 0)
            break;
    if (started == 0)
        gqa_worker(&job);
    for (size_t i = 0; i < started; ++i)
        pthread_join(pool[i], NULL);
    pthread_mutex_destroy(&job.lock);
    const int status = job.status;
    if (status == MFO_OK) {
        memcpy(key_cache + job.initial_len * job.kv_width, key,
               tokens * job.kv_width * sizeof(float));
        memcpy(value_cache + job.initial_len * job.kv_width, value,
               tokens * job.kv_width * sizeof(float));
        memcpy(out, job.staged, staged_count * sizeof(float));
        *cache_len = job.initial_len + tokens;
    }
    free(job.staged);
    return status;
}

/* CpuBackend::gated_short_convolution, attention_convolution.rs:269-339. */
int mfo_gated_short_convolution(float *out, const float *projection, const float *kernel,
                                float *history, size_t tokens, size_t hidden, size_t width)
{
    const size_t history_rows = width - 1;
    const size_t pw = 3 * hidden;
    const size_t count = tokens * hidden;
    float *u = (float *)malloc((count ? count : 1) * sizeof(float));
    float *produced = (float *)malloc((count ? count : 1) * sizeof(float));
    if (!u || !produced) {
        free(u);
        free(produced);
        return MFO_ERR_RESOURCE_LIMIT;
    }
    int status = MFO_OK;
    for (size_t i = 0; i < tokens * hidden && status == MFO_OK; ++i) {
        const size_t token = i / hidden, channel = i % hidden;
        const size_t base = token * pw + channel;
        const float gate = projection[base] * projection[base + 2 * hidden];
        if (!isfinite(gate))
            status = MFO_ERR_BACKEND_FAILURE;
        u[i] = gate;
    }
    for (size_t token = 0; token < tokens && status == MFO_OK; ++token) {
        for (size_t channel = 0; channel < hidden; ++channel) {
            float total = 0.0f;
            for (size_t tap = 0; tap < width; ++tap) {
                const long long relative = (long long)token + (long long)tap -
                                           (long long)history_rows;
                const float u_value =
                    relative < 0
                        ? history[(size_t)(relative + (long long)history_rows) * hidden + channel]
                        : u[(size_t)relative * hidden + channel];
                total += kernel[channel * width + tap] * u_value;
            }
            const float result = total * projection[token * pw + hidden + channel];
            if (!isfinite(result)) {
                status = MFO_ERR_BACKEND_FAILURE;
                break;
            }
            produced[token * hidden + channel] = result;
        }
    }
    if (status == MFO_OK) {
        if (history_rows > 0) {
            if (tokens >= history_rows) {
                memcpy(history, u + (tokens - history_rows) * hidden,
                       history_rows * hidden * sizeof(float));
            } else {
                const size_t keep = history_rows - tokens;
                memmove(history, history + (history_rows - keep) * hidden,
                        keep * hidden * sizeof(float));
                memcpy(history + keep * hidden, u, tokens * hidden * sizeof(float));
            }
        }
        memcpy(out, produced, tokens * hidden * sizeof(float));
    }
    free(u);
    free(produced);
    return status;
}
