/*
 * minifield_lfm2.h - LFM2 token pass over the HIP backend's C ABI.
 *
 * A C++ restatement of the reference executor's model pass
 * (crates/executor-core/src/lfm2/executor/execution.rs:35-585,
 * `append_tokens`, `sample_epilogue`, `append_token`): the same operations in
 * the same order, each issued through the `mfh_*` entry points of
 * minifield_hip.h, with the same role routing (dense `linear` or the packed
 * entry points by how each role is stored, the K/V and FFN pair and fused
 * variants on the same conditions).  It exists so that whole-model decode can
 * be driven and timed without a host round trip per token; weights are
 * buffers the caller uploads and attaches by role.
 *
 * Threading and errors follow minifield_hip.h: a model belongs to one
 * context, and every call returns an mfh_status.
 */
#ifndef MINIFIELD_LFM2_H
#define MINIFIELD_LFM2_H

#include <stddef.h>
#include <stdint.h>

#include "minifield_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Lfm2Config (crates/executor-core/src/lfm2/config.rs:33-51), the fields the
 * token pass reads.  `layer_kinds[i]` is 0 for a gated short-convolution
 * block and 1 for a full-attention block.  `max_tokens` bounds the prefix
 * (the executor's max_logical_tokens) and sizes the KV caches. */
typedef struct mfl_config {
    uint32_t hidden;
    uint32_t intermediate;
    uint32_t attention_heads;
    uint32_t key_value_heads;
    uint32_t head_dim;
    uint32_t conv_width;
    uint32_t vocab;
    uint32_t layer_count;
    const uint8_t *layer_kinds;
    float rope_theta;
    float norm_epsilon;       /* final (embedding) norm */
    float block_norm_epsilon; /* per-block norms */
    uint64_t max_tokens;
} mfl_config;

/* Weight roles (crates/executor-core/src/lfm2/weights.rs:210-237).  The tied
 * LM head reads the token embedding. */
typedef enum mfl_role {
    MFL_TOKEN_EMBEDDING = 0,  /* [vocab, hidden]                   */
    MFL_EMBEDDING_NORM = 1,   /* [hidden]                          */
    MFL_OPERATOR_NORM = 2,    /* per layer [hidden]                */
    MFL_FFN_NORM = 3,         /* per layer [hidden]                */
    MFL_CONV_KERNEL = 4,      /* conv layer [hidden, conv_width]   */
    MFL_CONV_IN = 5,          /* conv layer [3 * hidden, hidden]   */
    MFL_CONV_OUT = 6,         /* conv layer [hidden, hidden]       */
    MFL_QUERY_NORM = 7,       /* attention layer [head_dim]        */
    MFL_KEY_NORM = 8,         /* attention layer [head_dim]        */
    MFL_QUERY = 9,            /* attention layer [hidden, hidden]  */
    MFL_KEY = 10,             /* attention layer [kv_width, hidden]*/
    MFL_VALUE = 11,           /* attention layer [kv_width, hidden]*/
    MFL_OUTPUT = 12,          /* attention layer [hidden, hidden]  */
    MFL_FFN_W1 = 13,          /* per layer [intermediate, hidden]  */
    MFL_FFN_W2 = 14,          /* per layer [hidden, intermediate]  */
    MFL_FFN_W3 = 15           /* per layer [intermediate, hidden]  */
} mfl_role;

typedef struct mfl_model mfl_model;
typedef struct mfl_prefix mfl_prefix;

/* Validate the configuration and allocate the prefix state (zeroed
 * convolution histories and KV caches of `max_tokens` rows). */
mfh_status mfl_create(mfh_ctx *ctx, const mfl_config *config, mfl_model **out);
void mfl_destroy(mfl_model *model);

/* Attach one role's weight.  A dense role passes its f32 tensor and a null
 * `scales`; a packed matmul role passes its U8 codes and f32 scales
 * (Lfm2ResolvedWeight, weights.rs:1154-1185).  `layer` is ignored for
 * model-level roles.  The buffers stay owned by the caller and must outlive
 * the model's use of them. */
mfh_status mfl_set_weight(mfl_model *model, uint32_t role, uint32_t layer, const mfh_buf *tensor,
                          const mfh_buf *scales);

/* Empty the prefix: length 0, zeroed histories (cache contents past the
 * length are never read). */
mfh_status mfl_reset(mfl_model *model);
uint64_t mfl_length(const mfl_model *model);

/* append_tokens (execution.rs:35-540): `count` host ids, or a rank-1 f32
 * device id buffer (TokenIds::Device) when `device_ids` is non-null.  With
 * `produce_logits` the last row's logits land in the model's [1, vocab]
 * logits buffer. */
mfh_status mfl_append(mfl_model *model, const uint32_t *tokens, size_t count,
                      const mfh_buf *device_ids, int produce_logits);

/* sample_epilogue (execution.rs:546-571) without a mask: argmax of the
 * current logits into the model's [1] sampled-id buffer. */
mfh_status mfl_sample(mfl_model *model);

/* Greedy decode: `steps` times { sample; record the id in
 * `ids_out[i]`; append it as a device id with logits }.  `ids_out` is an f32
 * buffer of `steps` elements; nothing is read back to the host. */
mfh_status mfl_generate(mfl_model *model, uint32_t steps, mfh_buf *ids_out);

/* The model-owned logits [1, vocab] and sampled-id [1] buffers (valid until
 * mfl_destroy; readable with mfh_read_f32_async). */
const mfh_buf *mfl_logits(const mfl_model *model);
const mfh_buf *mfl_sampled(const mfl_model *model);

/* Lfm2Prefix (crates/executor-core/src/lfm2/executor.rs:249-281): an
 * immutable copy of the model's current prefix state -- per layer the
 * convolution history or the live key/value rows, the last pass's logits and
 * sampled id, and the lengths -- in Cache-class buffers of the model's
 * context.  The model keeps running from its own state. */
mfh_status mfl_snapshot(mfl_model *model, mfl_prefix **out);
/* Continue from a stored prefix: the model's prefix state becomes a copy of
 * `prefix`, which stays unchanged and can be restored again (the reference's
 * fork of a shared prefix, prefix_task.rs:158 and executor/storage.rs:104-155).
 * The prefix must come from this model (MFH_INVALID_ARGUMENT otherwise). */
mfh_status mfl_restore(mfl_model *model, const mfl_prefix *prefix);
uint64_t mfl_prefix_length(const mfl_prefix *prefix);
/* Release a prefix's buffers (before its context is destroyed). */
void mfl_prefix_destroy(mfl_prefix *prefix);

#ifdef __cplusplus
}
#endif

#endif
