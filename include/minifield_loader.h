/*
 * minifield_loader.h - safetensors bundles straight into HIP device buffers.
 *
 * The on-disk path of the reference's weight loader for the packed formats
 * (crates/executor-core/src/loader.rs:1130-1200 and loader/header.rs, the
 * LFM2 tensor plan in crates/executor-core/src/lfm2/weights.rs:268-500,
 * 756-835): a bounded header parse with the reference's rules and messages,
 * then per tensor one host-to-device copy of the file bytes.
 *
 * Split streams: a packed matmul role `<name>` is stored as `<name>.codes`
 * (U8 [rows, k / weights_per_byte], uploaded byte-exact) and `<name>.scales`
 * (F16 [rows, k / 128]).  The scales travel as their 2-byte file values and
 * stay on the device as binary16 (the kernels' scale shadow); the F32 scale
 * buffer the operation contract expects is decoded from them on the device,
 * with the loader's f16 -> f32 rule (loader.rs:408-421).  INT8 streams
 * holding the reserved code 0x80 are rejected before anything is uploaded
 * (loader.rs:1154-1162), and so are scales that decode to a non-finite value.
 *
 * Errors: every call returns an mfh_status (the ExecutorError variant);
 * mfs_error() gives the static message of this thread's last failure.
 */
#ifndef MINIFIELD_LOADER_H
#define MINIFIELD_LOADER_H

#include <stddef.h>
#include <stdint.h>

#include "minifield_hip.h"
#include "minifield_lfm2.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Storage dtypes (crates/executor-core/src/loader.rs:52-73). */
typedef enum mfs_dtype {
    MFS_F32 = 0,
    MFS_BF16 = 1,
    MFS_F16 = 2,
    MFS_U8 = 3
} mfs_dtype;

typedef struct mfs_file mfs_file;

/* Open and validate a safetensors file (memory-mapped, read only), with the
 * checks of parse_safetensors_header (loader/header.rs:18-133): header length
 * within `max_header_bytes` and the file, a JSON object with string metadata
 * values, tensor objects of exactly dtype/shape/data_offsets, no duplicate
 * names (MFH_DUPLICATE_NAME), ranges matching shape x dtype width, and
 * payload ranges covering the payload without holes or overlap. */
mfh_status mfs_open(const char *path, uint64_t max_header_bytes, mfs_file **out);
void mfs_close(mfs_file *file);
/* The static message of this thread's last failed mfs_* / mfl_load call. */
const char *mfs_error(void);

size_t mfs_tensor_count(const mfs_file *file);
/* Name of tensor `index` in header order (NULL past the end). */
const char *mfs_tensor_name(const mfs_file *file, size_t index);
/* Dtype, rank and dims (room for 4) of a tensor; MFH_MISSING_REQUIRED_TENSOR
 * when the file has no tensor of that name. */
mfh_status mfs_tensor_info(const mfs_file *file, const char *name, mfs_dtype *dtype,
                           uint32_t *rank, uint64_t *dims);
/* A `__metadata__` string value, or NULL. */
const char *mfs_metadata(const mfs_file *file, const char *key);

/* Stored scheme of a matmul tensor (Lfm2WeightFormat resolved per role). */
typedef enum mfs_scheme {
    MFS_SCHEME_DENSE = 0,
    MFS_SCHEME_TERNARY = 1,
    MFS_SCHEME_NF4 = 2,
    MFS_SCHEME_INT8 = 3
} mfs_scheme;

/* The scheme the bundle declares for matmul tensor `name`, as the
 * reference's plan resolves it (weights.rs:64-130, 756-790): the
 * `tensor_quantization` override for the name when present, else the bundle
 * format -- absent or "pt": dense; minifield.{ternary,nf4,int8}.v1: that
 * scheme; minifield.mixed.v1: dense.  An unknown format marker is
 * MFH_UNSUPPORTED; a malformed override map or level MFH_INVALID_ARGUMENT. */
mfh_status mfs_matmul_scheme(const mfs_file *file, const char *name, mfs_scheme *out);

/* Upload packed role `base` (base.codes + base.scales) as U8 codes and F32
 * scales whose binary16 values stay on the device, then build the private
 * tile copies (mfh_prepare_packed). */
mfh_status mfs_upload_packed(mfh_ctx *ctx, const mfs_file *file, const char *base,
                             mfh_alloc_class cls, mfh_buf **codes, mfh_buf **scales);
/* Upload a dense F32 / BF16 / F16 tensor as F32 (loader.rs decode_tensor);
 * non-finite values fail with MFH_BACKEND_FAILURE. */
mfh_status mfs_upload_dense(mfh_ctx *ctx, const mfs_file *file, const char *name,
                            mfh_alloc_class cls, mfh_buf **out);

/* Attach every weight role of `model` from an LFM2 bundle, by the
 * reference's tensor names (weights.rs:268-500): model.embed_tokens.weight
 * (also the tied head), model.embedding_norm.weight, and per layer
 * model.layers.{i}.{operator_norm, ffn_norm, feed_forward.w1/w2/w3,
 * conv.conv / conv.in_proj / conv.out_proj | self_attn.q_layernorm /
 * k_layernorm / q_proj / k_proj / v_proj / out_proj}.weight.  Each matmul
 * role takes the scheme mfs_matmul_scheme resolves: a dense tensor, or the
 * split streams `<name>.codes` / `<name>.scales` whose code width must be
 * the scheme's.  Shapes must equal the model configuration's
 * (MFH_INVALID_SHAPE), a missing tensor is MFH_MISSING_REQUIRED_TENSOR, a
 * tensor of the file that no role consumes MFH_UNEXPECTED_TENSOR, and the
 * conv kernel [hidden, 1, width] becomes [hidden, width].  Nothing is
 * uploaded unless the whole inventory checks out.  The model owns the
 * uploaded buffers (Weight class). */
mfh_status mfl_load_safetensors(mfl_model *model, const mfs_file *file);

#ifdef __cplusplus
}
#endif

#endif
