// LFM2 token pass over the backend's own C ABI: a restatement of the
// reference executor's `append_tokens` / `sample_epilogue`
// (crates/executor-core/src/lfm2/executor/execution.rs:35-585).
//
// Every operation is issued through the same mfh_* entry points an external
// caller uses, in the reference's order and with its role routing.  What this
// file adds is buffer management suited to a device: every intermediate of a
// pass lives in a per-row-count workspace allocated once, so steady-state
// decode allocates nothing and never waits on the host.
#include <cmath>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "../../include/minifield_lfm2.h"
#include "../../include/minifield_loader.h"
#include "internal.hpp"
#include "kernels.hpp"

namespace mfh {
namespace {

struct Weight {
    const mfh_buf *tensor = nullptr;
    const mfh_buf *scales = nullptr;  // null: dense f32
    bool packed() const { return scales != nullptr; }
};

struct LayerWeights {
    Weight operator_norm, ffn_norm;
    Weight conv_kernel, conv_in, conv_out;
    Weight query_norm, key_norm, query, key, value, output;
    Weight w1, w2, w3;
};

// Owned buffer handle.
struct Owned {
    mfh_buf *buf = nullptr;
    Owned() = default;
    Owned(const Owned &) = delete;
    Owned &operator=(const Owned &) = delete;
    ~Owned()
    {
        if (buf)
            mfh_release(buf);
    }
};

mfh_status alloc(mfh_ctx *ctx, Owned &o, uint64_t rows, uint64_t cols, mfh_alloc_class cls,
                 bool zeroed)
{
    const uint64_t dims[2] = {rows, cols};
    return mfh_alloc_f32(ctx, dims, 2, cls, zeroed ? 1 : 0, &o.buf);
}

// Every intermediate of one pass over `rows` tokens (execution.rs allocates
// these per call as Scratch).  x/u ping-pong between layers.
struct Workspace {
    uint64_t rows = 0;
    Owned x[2], u[2], op, projection, convolved;
    Owned q, k, v, q_rope, k_rope, attention;
    Owned residual, ffn_input, gate, up, hidden, down;
};

struct LayerState {
    // conv: [conv_width - 1, hidden], two copies: the fused decode step reads
    // one and writes the rolled history into the other.
    Owned history[2];
    int current = 0;         // the copy that holds the history
    Owned key, value;        // attention: [max_tokens, kv_width]
    uint64_t length = 0;
};

}  // namespace
}  // namespace mfh

using namespace mfh;

struct mfl_model {
    mfh_ctx *ctx = nullptr;
    uint64_t id = 0;  // distinguishes models for prefix ownership checks
    mfl_config config{};
    std::vector<uint8_t> kinds;
    uint64_t kv_width = 0;
    Weight embedding, embedding_norm;
    std::vector<LayerWeights> layers;
    std::vector<LayerState> state;
    uint64_t length = 0;
    std::map<uint64_t, std::unique_ptr<Workspace>> workspaces;
    Owned logits, sampled;
    // Greedy-selection candidates the fused step's LM head wrote beside the
    // logits (one per head block, Candidate layout), valid while
    // candidate_count != 0 and the prefix is still candidate_length long.
    Owned candidates;
    uint32_t candidate_count = 0;
    uint64_t candidate_length = 0;
    Owned rotation;  // [max_tokens, head_dim] rotation coefficients by position
    // Weights uploaded by mfl_load_safetensors (the model owns them).
    std::vector<std::unique_ptr<Owned>> loaded;
};

// An immutable copy of a model's prefix state (Lfm2Prefix,
// executor-core/src/lfm2/executor.rs:249-281): per layer the convolution
// history, or the live key/value cache rows; the logits and sampled id of
// the last pass; the lengths.  Its buffers are Cache class, like the
// reference's fork storage (executor/storage.rs:104-155).
struct mfl_prefix {
    mfh_ctx *ctx = nullptr;
    uint64_t model_id = 0;
    uint64_t length = 0;
    struct Layer {
        Owned history;      // conv: [conv_width - 1, hidden]
        Owned key, value;   // attention: [length, kv_width] (none when empty)
        uint64_t length = 0;
    };
    std::vector<Layer> layers;
    Owned logits, sampled;
};

namespace mfh {
namespace {

mfh_status workspace(mfl_model *m, uint64_t rows, Workspace **out)
{
    auto it = m->workspaces.find(rows);
    if (it != m->workspaces.end()) {
        *out = it->second.get();
        return MFH_OK;
    }
    auto ws = std::make_unique<Workspace>();
    ws->rows = rows;
    mfh_ctx *c = m->ctx;
    const uint64_t h = m->config.hidden, inter = m->config.intermediate, kv = m->kv_width;
    const mfh_alloc_class S = MFH_CLASS_SCRATCH;
    mfh_status s = MFH_OK;
    for (int i = 0; i < 2 && !s; ++i) {
        s = alloc(c, ws->x[i], rows, h, S, false);
        if (!s)
            s = alloc(c, ws->u[i], rows, h, S, false);
    }
    const struct {
        Owned *o;
        uint64_t cols;
    } plan[] = {{&ws->op, h},          {&ws->projection, 3 * h}, {&ws->convolved, h},
                {&ws->q, h},           {&ws->k, kv},             {&ws->v, kv},
                {&ws->q_rope, h},      {&ws->k_rope, kv},        {&ws->attention, h},
                {&ws->residual, h},    {&ws->ffn_input, h},      {&ws->gate, inter},
                {&ws->up, inter},      {&ws->hidden, inter},     {&ws->down, h}};
    for (const auto &p : plan)
        if (!s)
            s = alloc(c, *p.o, rows, p.cols, S, false);
    if (s)
        return s;
    *out = ws.get();
    m->workspaces.emplace(rows, std::move(ws));
    return MFH_OK;
}

// weight_linear (execution.rs:12-25).
mfh_status weight_linear(mfh_ctx *c, mfh_buf *out, const mfh_buf *in, const Weight &w)
{
    if (!w.tensor)
        return fail(c, MFH_MISSING_REQUIRED_TENSOR, "LFM2 weight role is not attached");
    if (w.packed())
        return mfh_packed_linear(c, out, in, w.tensor, w.scales);
    return mfh_linear(c, out, in, w.tensor);
}

// The pair/fused conditions compare the stored quantization of two roles
// (role_quant, weights.rs:588): packed streams of one shape share a format
// exactly when their code widths agree.
// The format of a packed weight of inner width k, from its code width.
Format packed_format_of(const Weight &w, uint32_t k)
{
    const uint64_t cols = w.tensor->dims[1];
    return cols == k ? Format::Int8 : 2 * cols == k ? Format::Nf4 : Format::Ternary;
}

bool same_packed_format(const Weight &a, const Weight &b)
{
    return a.packed() && b.packed() && a.tensor->dims[1] == b.tensor->dims[1] &&
           a.scales->dims[1] == b.scales->dims[1];
}

mfh_status need(mfh_ctx *c, const Weight &w)
{
    return w.tensor ? MFH_OK
                    : fail(c, MFH_MISSING_REQUIRED_TENSOR, "LFM2 weight role is not attached");
}

// The FFN of one layer on `ffn_rows` rows (execution.rs:289-497).
mfh_status ffn(mfl_model *m, const LayerWeights &lw, Workspace &ws, mfh_buf *ffn_input,
               mfh_buf *down)
{
    mfh_ctx *c = m->ctx;
    mfh_status s;
    const uint64_t ffn_rows = ws.rows;
    const bool pair = same_packed_format(lw.w1, lw.w3);
    if (ffn_rows >= 96 && pair && lw.w2.packed()) {
        // Fused prefill: SwiGLU in the gate/up epilogue, then the down GEMM.
        if ((s = mfh_packed_swiglu_pair(c, ws.hidden.buf, ffn_input, lw.w1.tensor, lw.w1.scales,
                                        lw.w3.tensor, lw.w3.scales)))
            return s;
        return mfh_packed_linear(c, down, ws.hidden.buf, lw.w2.tensor, lw.w2.scales);
    }
    if (pair) {
        s = mfh_packed_linear_pair(c, ws.gate.buf, ws.up.buf, ffn_input, lw.w1.tensor,
                                   lw.w1.scales, lw.w3.tensor, lw.w3.scales);
    } else {
        s = weight_linear(c, ws.gate.buf, ffn_input, lw.w1);
        if (!s)
            s = weight_linear(c, ws.up.buf, ffn_input, lw.w3);
    }
    if (s)
        return s;
    if ((s = need(c, lw.w2)))
        return s;
    if (lw.w2.packed())
        return mfh_packed_swiglu_linear(c, down, ws.gate.buf, ws.up.buf, lw.w2.tensor,
                                        lw.w2.scales);
    if ((s = mfh_swiglu(c, ws.hidden.buf, ws.gate.buf, ws.up.buf)))
        return s;
    return weight_linear(c, down, ws.hidden.buf, lw.w2);
}

float *dev(const Owned &o)
{
    return static_cast<float *>(o.buf->dev);
}

const float *dev(const Weight &w)
{
    return static_cast<const float *>(w.tensor->dev);
}

// Whether the one-token step can run fused: every matmul role packed (the
// K/V and FFN gate/up pairs in one format each), every norm and kernel
// attached, and the matrix-core GEMV in use (kernel path 0 or 2; with 2 the
// transforms run in the separate prologue kernels; path 3 keeps the
// automatic kernels but runs the step op by op).
bool fused_decode_ready(const mfl_model *m)
{
    if (m->ctx->kernel_path == 1 || m->ctx->kernel_path == 3 || !m->embedding.packed() ||
        !m->embedding_norm.tensor)
        return false;
    for (uint32_t i = 0; i < m->config.layer_count; ++i) {
        const LayerWeights &lw = m->layers[i];
        if (!lw.operator_norm.tensor || !lw.ffn_norm.tensor || !same_packed_format(lw.w1, lw.w3) ||
            !lw.w2.packed())
            return false;
        if (m->kinds[i] == 0) {
            if (!lw.conv_in.packed() || !lw.conv_out.packed() || !lw.conv_kernel.tensor)
                return false;
        } else if (!lw.query.packed() || !same_packed_format(lw.key, lw.value) ||
                   !lw.output.packed() || !lw.query_norm.tensor || !lw.key_norm.tensor) {
            return false;
        }
    }
    return true;
}

// One decode token with the elementwise steps folded into the products
// (see XForm) where that measured faster: per convolution block the in
// projection forms the residual add + operator norm and finishes the
// one-token convolution in its epilogue, and the gate/up pair forms the
// residual add + FFN norm with SwiGLU in its epilogue; the LM head forms the
// final add + norm and writes the greedy-selection candidates of its blocks
// beside the logits.  Attention blocks run q/k/v as one launch (v lands in
// its cache row) and qk_norm_rope + the key append + attention as two.  Same
// operations and order as append() on one row; only the f32 reduction trees
// of the norms and the softmax differ.
mfh_status decode_step(mfl_model *m, const mfh_buf *device_ids, bool produce_logits)
{
    mfh_ctx *c = m->ctx;
    const mfl_config &cfg = m->config;
    const uint32_t h = cfg.hidden, inter = cfg.intermediate;
    const uint32_t kv = uint32_t(m->kv_width);
    Workspace *ws = nullptr;
    mfh_status s = workspace(m, 1, &ws);
    if (s)
        return s;
    if ((s = mfh_packed_gather_rows(c, ws->x[0].buf, m->embedding.tensor, m->embedding.scales,
                                    nullptr, 0, device_ids)))
        return s;
    DeviceGuard guard(c->device);
    float *x = dev(ws->x[0]);
    float *residual = dev(ws->residual), *down = dev(ws->down), *op = dev(ws->op);
    // The block input is left + right (layer 0: the embedding row alone).
    const float *left = x, *right = nullptr;
    const auto norm_of = [&](const Weight &w, float *side) {
        XForm t;
        t.kind = XKind::AddRms;
        t.a = left;
        t.b = right;
        t.w = dev(w);
        t.side = side;
        t.epsilon = cfg.block_norm_epsilon;
        return t;
    };
    const uint64_t position = m->length;
    for (uint32_t index = 0; index < cfg.layer_count; ++index) {
        const LayerWeights &lw = m->layers[index];
        LayerState &st = m->state[index];
        float *block_input_side = right ? x : nullptr;
        if (m->kinds[index] == 0) {
            // The in-projection finishes the one-token convolution in its
            // epilogue where the vector GEMV serves it (one launch), else
            // the projection and conv_step_kernel (two).
            ConvStep conv;
            conv.kernel = dev(lw.conv_kernel);
            conv.history = dev(st.history[st.current]);
            conv.next = dev(st.history[1 - st.current]);
            conv.out = dev(ws->convolved);
            conv.hidden = h;
            conv.width = cfg.conv_width;
            s = packed_xform_conv(c, norm_of(lw.operator_norm, block_input_side), h,
                                  lw.conv_in.tensor, lw.conv_in.scales, conv);
            if (s == MFH_UNSUPPORTED) {
                if ((s = packed_xform(c, Epilogue::Single,
                                      norm_of(lw.operator_norm, block_input_side), 1, 3 * h, h,
                                      lw.conv_in.tensor, lw.conv_in.scales, nullptr, nullptr,
                                      dev(ws->projection), nullptr)))
                    return s;
                launch_conv_step(c->stream, dev(ws->convolved), dev(ws->projection),
                                 dev(lw.conv_kernel), dev(st.history[st.current]),
                                 dev(st.history[1 - st.current]), h, cfg.conv_width);
            } else if (s) {
                return s;
            }
            XForm convolved;
            convolved.a = dev(ws->convolved);
            if ((s = packed_xform(c, Epilogue::Single, convolved, 1, h, h, lw.conv_out.tensor,
                                  lw.conv_out.scales, nullptr, nullptr, op, nullptr)))
                return s;
            st.current = 1 - st.current;
        } else {
            float *key_row = dev(st.key) + position * kv;
            float *value_row = dev(st.value) + position * kv;
            // q, k and v in one launch when they share a format, else q and
            // the k/v pair; v lands in its cache row.
            s = MFH_UNSUPPORTED;
            if (same_packed_format(lw.query, lw.key) && same_packed_format(lw.key, lw.value)) {
                const mfh_buf *codes[3] = {lw.query.tensor, lw.key.tensor, lw.value.tensor};
                const mfh_buf *scales[3] = {lw.query.scales, lw.key.scales, lw.value.scales};
                const uint32_t rows[3] = {h, kv, kv};
                float *outs[3] = {dev(ws->q), dev(ws->k), value_row};
                s = packed_xform_segments(c, norm_of(lw.operator_norm, block_input_side), 1, h, 3,
                                          codes, scales, rows, outs);
            }
            if (s == MFH_UNSUPPORTED &&
                !(s = packed_xform(c, Epilogue::Single,
                                   norm_of(lw.operator_norm, block_input_side), 1, h, h,
                                   lw.query.tensor, lw.query.scales, nullptr, nullptr, dev(ws->q),
                                   nullptr)))
                s = packed_xform(c, Epilogue::Pair, norm_of(lw.operator_norm, nullptr), 1, kv, h,
                                 lw.key.tensor, lw.key.scales, lw.value.tensor, lw.value.scales,
                                 dev(ws->k), value_row);
            if (s)
                return s;
            // qk_norm_rope, the key append and split-key attention in one
            // launch plus the range combine where the shape allows, else
            // qk_norm_rope (writing the key row) and causal_gqa without an
            // append.
            DecodeAttention da;
            da.query = dev(ws->q);
            da.key = dev(ws->k);
            da.query_weight = dev(lw.query_norm);
            da.key_weight = dev(lw.key_norm);
            da.key_cache = dev(st.key);
            da.value_cache = dev(st.value);
            da.rotation = dev(m->rotation);
            da.out = dev(ws->attention);
            da.position = st.length;
            da.query_heads = cfg.attention_heads;
            da.key_value_heads = cfg.key_value_heads;
            da.head_dim = cfg.head_dim;
            da.group = cfg.attention_heads / cfg.key_value_heads;
            da.theta = cfg.rope_theta;
            da.epsilon = cfg.block_norm_epsilon;
            da.scale = 1.0f / std::sqrt(float(cfg.head_dim));
            da.splits = gqa_decode_splits(da);
            // With few key ranges the output projection merges them in its
            // prologue (no combine launch); else the combine kernel does.
            XForm merged;
            merged.kind = XKind::GqaMerge;
            merged.ranges = da.splits;
            merged.head_dim = cfg.head_dim;
            bool merge = false;
            if (da.splits) {
                da.partial = static_cast<float *>(work_scratch(c, gqa_decode_scratch_bytes(da)));
                if (!da.partial)
                    return allocation_failed(c);
                merged.a = da.partial;
                merge = da.splits <= kGqaMergeMaxRanges;
                launch_gqa_decode(c->stream, da, !merge);
            } else {
                Positions positions;
                positions.base = position;
                launch_qk_norm_rope(c->stream, dev(ws->q_rope), key_row, dev(ws->q), dev(ws->k),
                                    dev(lw.query_norm), dev(lw.key_norm), positions, 1,
                                    cfg.attention_heads, cfg.key_value_heads, cfg.head_dim,
                                    cfg.rope_theta, cfg.block_norm_epsilon);
                GqaShape g;
                g.tokens = 1;
                g.initial_len = st.length;
                g.query_heads = cfg.attention_heads;
                g.key_value_heads = cfg.key_value_heads;
                g.head_dim = cfg.head_dim;
                g.group = da.group;
                g.scale = da.scale;
                float *partials = nullptr;
                if (const size_t bytes = gqa_scratch_bytes(g)) {
                    partials = static_cast<float *>(work_scratch(c, bytes));
                    if (!partials)
                        return allocation_failed(c);
                }
                launch_gqa(c->stream, dev(ws->attention), dev(ws->q_rope), nullptr, nullptr,
                           dev(st.key), dev(st.value), g, partials);
            }
            st.length += 1;
            if (merge) {
                s = packed_xform(c, Epilogue::Single, merged, 1, h, h, lw.output.tensor,
                                 lw.output.scales, nullptr, nullptr, op, nullptr);
                if (s == MFH_UNSUPPORTED) {
                    // Not the one-row wide kernel's shape: combine, then the
                    // plain projection below.
                    launch_gqa_combine(c->stream, da);
                    merge = false;
                } else if (s) {
                    return s;
                }
            }
            if (!merge) {
                XForm plain;
                plain.a = dev(ws->attention);
                if ((s = packed_xform(c, Epilogue::Single, plain, 1, h, h, lw.output.tensor,
                                      lw.output.scales, nullptr, nullptr, op, nullptr)))
                    return s;
            }
        }
        // FFN: residual = block input + op, normed into the gate/up pair,
        // whose epilogue forms silu(gate) * up (the value packed_swiglu_linear
        // stages) for the down projection.
        left = right ? x : left;
        right = op;
        if ((s = packed_xform(c, Epilogue::SwigluPair, norm_of(lw.ffn_norm, residual), 1, inter,
                              h, lw.w1.tensor, lw.w1.scales, lw.w3.tensor, lw.w3.scales,
                              dev(ws->hidden), nullptr)))
            return s;
        XForm hidden;
        hidden.a = dev(ws->hidden);
        if ((s = packed_xform(c, Epilogue::Single, hidden, 1, h, inter, lw.w2.tensor,
                              lw.w2.scales, nullptr, nullptr, down, nullptr)))
            return s;
        left = residual;
        right = down;
    }
    if (produce_logits && head_fold_supported(packed_format_of(m->embedding, h), cfg.vocab, h)) {
        // The final add + norm formed in the LM head's slices, and each head
        // block's greedy-selection candidate beside the logits (one launch
        // for what was a row-norm kernel, the head and argmax's range pass).
        XForm head;
        head.kind = XKind::AddRms;
        head.a = left;
        head.b = right;
        head.w = dev(m->embedding_norm);
        head.epsilon = cfg.norm_epsilon;
        uint32_t count = 0;
        if ((s = packed_xform(c, Epilogue::Single, head, 1, cfg.vocab, h, m->embedding.tensor,
                              m->embedding.scales, nullptr, nullptr, dev(m->logits), nullptr,
                              reinterpret_cast<Candidate *>(dev(m->candidates)), &count)))
            return s;
        m->candidate_count = count;
        m->candidate_length = m->length + 1;
    } else if (produce_logits) {
        // The final add + norm as a row kernel of its own (the sum goes to a
        // scratch row), then a plain product.
        launch_row_rms(c->stream, dev(ws->u[0]), right ? dev(ws->u[1]) : nullptr, left, right,
                       dev(m->embedding_norm), 1, h, cfg.norm_epsilon);
        XForm head;
        head.a = dev(ws->u[0]);
        if ((s = packed_xform(c, Epilogue::Single, head, 1, cfg.vocab, h, m->embedding.tensor,
                              m->embedding.scales, nullptr, nullptr, dev(m->logits), nullptr)))
            return s;
    }
    if (hipGetLastError() != hipSuccess)
        return fail(c, MFH_BACKEND_FAILURE, "decode step launch failed");
    m->length += 1;
    return MFH_OK;
}

// append_tokens (execution.rs:35-540).
mfh_status append(mfl_model *m, const uint32_t *tokens, size_t count, const mfh_buf *device_ids,
                  bool produce_logits)
{
    mfh_ctx *c = m->ctx;
    const mfl_config &cfg = m->config;
    m->candidate_count = 0;
    uint64_t rows = count;
    if (device_ids) {
        mfh_status s = check_f32(c, device_ids);
        if (s)
            return s;
        if (device_ids->rank != 1)
            return fail(c, MFH_INVALID_SHAPE, "device token-id buffer must be rank one");
        rows = device_ids->dims[0];
    }
    if (rows == 0)
        return fail(c, MFH_INVALID_ARGUMENT, "token pass requires at least one token");
    for (size_t i = 0; !device_ids && i < count; ++i)
        if (tokens[i] >= cfg.vocab)
            return fail(c, MFH_OUT_OF_BOUNDS, "valid token ID exceeds loaded model vocabulary");
    if (m->length > UINT64_MAX - rows)
        return fail(c, MFH_OVERFLOW, "prefix logical length overflows u64");
    if (m->length + rows > cfg.max_tokens)
        return fail(c, MFH_OUT_OF_BOUNDS, "append exceeds configured logical prefix capacity");
    if (!m->embedding.tensor || !m->embedding_norm.tensor)
        return fail(c, MFH_MISSING_REQUIRED_TENSOR, "LFM2 weight role is not attached");
    if (rows == 1 && device_ids && fused_decode_ready(m))
        return decode_step(m, device_ids, produce_logits);

    Workspace *ws = nullptr, *ws1 = nullptr;
    mfh_status s = workspace(m, rows, &ws);
    if (!s)
        s = workspace(m, 1, &ws1);
    if (s)
        return s;
    std::vector<uint64_t> positions(rows);
    for (uint64_t i = 0; i < rows; ++i)
        positions[i] = m->length + i;

    // Embedding gather, then the first layer's operator norm.
    int p = 0;
    mfh_buf *x = ws->x[p].buf, *u = ws->u[p].buf;
    if (m->embedding.packed())
        s = mfh_packed_gather_rows(c, x, m->embedding.tensor, m->embedding.scales, tokens,
                                   device_ids ? 0 : count, device_ids);
    else
        s = mfh_gather_rows(c, x, m->embedding.tensor, tokens, device_ids ? 0 : count,
                            device_ids);
    if (s)
        return s;
    if ((s = need(c, m->layers[0].operator_norm)) ||
        (s = mfh_row_rms_norm(c, u, x, m->layers[0].operator_norm.tensor, cfg.block_norm_epsilon)))
        return s;

    const uint32_t L = cfg.layer_count;
    for (uint32_t index = 0; index < L; ++index) {
        const LayerWeights &lw = m->layers[index];
        LayerState &st = m->state[index];
        if (m->kinds[index] == 0) {
            if ((s = weight_linear(c, ws->projection.buf, u, lw.conv_in)) || (s = need(c, lw.conv_kernel)) ||
                (s = mfh_gated_short_convolution(c, ws->convolved.buf, ws->projection.buf,
                                                 lw.conv_kernel.tensor,
                                                 st.history[st.current].buf, cfg.hidden,
                                                 cfg.conv_width)) ||
                (s = weight_linear(c, ws->op.buf, ws->convolved.buf, lw.conv_out)))
                return s;
        } else {
            if ((s = weight_linear(c, ws->q.buf, u, lw.query)))
                return s;
            if (same_packed_format(lw.key, lw.value))
                s = mfh_packed_linear_pair(c, ws->k.buf, ws->v.buf, u, lw.key.tensor,
                                           lw.key.scales, lw.value.tensor, lw.value.scales);
            else if (!(s = weight_linear(c, ws->k.buf, u, lw.key)))
                s = weight_linear(c, ws->v.buf, u, lw.value);
            if (s)
                return s;
            if ((s = need(c, lw.query_norm)) || (s = need(c, lw.key_norm)))
                return s;
            if (cfg.head_dim >= 2 && cfg.head_dim % 2 == 0) {
                // Positions length .. length + rows - 1 are rows of the
                // model's rotation table (the coefficients qk_norm_rope
                // would compute, bit for bit).
                launch_qk_norm_rope_table(c->stream, dev(ws->q_rope), dev(ws->k_rope), dev(ws->q),
                                          dev(ws->k), dev(lw.query_norm), dev(lw.key_norm),
                                          dev(m->rotation), m->length, rows, cfg.attention_heads,
                                          cfg.key_value_heads, cfg.head_dim,
                                          cfg.block_norm_epsilon);
            } else if ((s = mfh_qk_norm_rope(c, ws->q_rope.buf, ws->k_rope.buf, ws->q.buf,
                                             ws->k.buf, lw.query_norm.tensor, lw.key_norm.tensor,
                                             positions.data(), rows, cfg.attention_heads,
                                             cfg.head_dim, cfg.rope_theta, cfg.key_value_heads,
                                             cfg.head_dim, cfg.block_norm_epsilon))) {
                return s;
            }
            if ((s = mfh_causal_gqa(c, ws->attention.buf, ws->q_rope.buf, ws->k_rope.buf,
                                    ws->v.buf, st.key.buf, st.value.buf, &st.length,
                                    cfg.attention_heads, cfg.key_value_heads, cfg.head_dim)) ||
                (s = weight_linear(c, ws->op.buf, ws->attention.buf, lw.output)))
                return s;
        }
        if ((s = need(c, lw.ffn_norm)) ||
            (s = mfh_add_row_rms_norm(c, ws->residual.buf, ws->ffn_input.buf, x, ws->op.buf,
                                      lw.ffn_norm.tensor, cfg.block_norm_epsilon)))
            return s;
        // The last layer's FFN runs on the last row only (execution.rs:282-306).
        const bool last = index + 1 == L;
        Workspace *fw = ws;
        mfh_buf *ffn_input = ws->ffn_input.buf, *residual = ws->residual.buf;
        if (last && rows > 1) {
            fw = ws1;
            if ((s = mfh_copy_rect_2d(c, ws1->ffn_input.buf, ws->ffn_input.buf, rows - 1, 0, 0, 0,
                                      1, cfg.hidden)) ||
                (s = mfh_copy_rect_2d(c, ws1->residual.buf, ws->residual.buf, rows - 1, 0, 0, 0,
                                      1, cfg.hidden)))
                return s;
            ffn_input = ws1->ffn_input.buf;
            residual = ws1->residual.buf;
        }
        if ((s = ffn(m, lw, *fw, ffn_input, fw->down.buf)))
            return s;
        // Next layer's operator norm (or the final embedding norm) fused with
        // the residual add.
        mfh_buf *next_x = fw->x[1 - p].buf, *next_u = fw->u[1 - p].buf;
        const Weight &next_norm = last ? m->embedding_norm : m->layers[index + 1].operator_norm;
        const float eps = last ? cfg.norm_epsilon : cfg.block_norm_epsilon;
        if ((s = need(c, next_norm)) ||
            (s = mfh_add_row_rms_norm(c, next_x, next_u, residual, fw->down.buf, next_norm.tensor,
                                      eps)))
            return s;
        p = 1 - p;
        x = next_x;
        u = next_u;
    }
    if (produce_logits && (s = weight_linear(c, m->logits.buf, u, m->embedding)))
        return s;
    m->length += rows;
    return MFH_OK;
}

}  // namespace
}  // namespace mfh

extern "C" {

mfh_status mfl_create(mfh_ctx *ctx, const mfl_config *config, mfl_model **out)
{
    if (!ctx)
        return MFH_INVALID_ARGUMENT;
    if (!config || !out)
        return fail(ctx, MFH_INVALID_ARGUMENT, "LFM2 configuration or output pointer is null");
    const mfl_config &c = *config;
    // Lfm2Config::validate (config.rs:54-100).
    if (c.hidden == 0 || c.intermediate == 0 || c.attention_heads == 0 ||
        c.key_value_heads == 0 || c.conv_width == 0 || c.vocab == 0 || c.layer_count == 0 ||
        !c.layer_kinds || c.head_dim == 0 || c.max_tokens == 0)
        return fail(ctx, MFH_INVALID_ARGUMENT, "LFM2 configuration has a zero dimension");
    if (uint64_t(c.attention_heads) * c.head_dim != c.hidden)
        return fail(ctx, MFH_INVALID_SHAPE, "LFM2 hidden size must equal heads * head_dim");
    if (c.attention_heads % c.key_value_heads != 0)
        return fail(ctx, MFH_INVALID_SHAPE,
                    "query heads must be a nonzero multiple of key/value heads");
    for (uint32_t i = 0; i < c.layer_count; ++i)
        if (c.layer_kinds[i] > 1)
            return fail(ctx, MFH_INVALID_ARGUMENT, "unknown LFM2 layer kind");
    static uint64_t next_id = 0;
    auto m = std::make_unique<mfl_model>();
    m->ctx = ctx;
    m->id = ++next_id;
    m->config = c;
    m->kinds.assign(c.layer_kinds, c.layer_kinds + c.layer_count);
    m->config.layer_kinds = m->kinds.data();
    m->kv_width = uint64_t(c.key_value_heads) * c.head_dim;
    m->layers.resize(c.layer_count);
    m->state = std::vector<LayerState>(c.layer_count);
    mfh_status s = MFH_OK;
    for (uint32_t i = 0; i < c.layer_count && !s; ++i) {
        LayerState &st = m->state[i];
        if (m->kinds[i] == 0) {
            for (int h = 0; h < 2 && !s; ++h)
                s = alloc(ctx, st.history[h], c.conv_width - 1, c.hidden, MFH_CLASS_CACHE, true);
        } else {
            s = alloc(ctx, st.key, c.max_tokens, m->kv_width, MFH_CLASS_CACHE, true);
            if (!s)
                s = alloc(ctx, st.value, c.max_tokens, m->kv_width, MFH_CLASS_CACHE, true);
        }
    }
    if (!s)
        s = alloc(ctx, m->logits, 1, c.vocab, MFH_CLASS_CACHE, true);
    if (!s) {
        // At most one candidate per 16 logits (sizeof(Candidate) = 3 floats).
        static_assert(sizeof(Candidate) == 3 * sizeof(float), "Candidate layout");
        s = alloc(ctx, m->candidates, (uint64_t(c.vocab) + 63) / 64 * 4, 3, MFH_CLASS_SCRATCH,
                  false);
    }
    if (!s && (s = alloc(ctx, m->rotation, c.max_tokens, c.head_dim, MFH_CLASS_CACHE, false)) ==
                  MFH_OK) {
        DeviceGuard guard(ctx->device);
        launch_rotation_table(ctx->stream, static_cast<float *>(m->rotation.buf->dev),
                              c.max_tokens, c.head_dim, c.rope_theta);
    }
    if (!s) {
        const uint64_t dims[1] = {1};
        s = mfh_alloc_f32(ctx, dims, 1, MFH_CLASS_CACHE, 1, &m->sampled.buf);
    }
    if (s)
        return s;
    *out = m.release();
    return MFH_OK;
}

void mfl_destroy(mfl_model *model)
{
    delete model;
}

mfh_status mfl_set_weight(mfl_model *m, uint32_t role, uint32_t layer, const mfh_buf *tensor,
                          const mfh_buf *scales)
{
    if (!m)
        return MFH_INVALID_ARGUMENT;
    mfh_ctx *c = m->ctx;
    mfh_status s = scales ? check_u8(c, tensor) : check_f32(c, tensor);
    if (!s && scales)
        s = check_f32(c, scales);
    if (s)
        return s;
    // Packed matmul roles get their private tile copies now, so a resource
    // limit fails the attach rather than a later token pass.
    if (scales && (s = prepare_packed(c, tensor, scales)))
        return s;
    Weight w{tensor, scales};
    if (role == MFL_TOKEN_EMBEDDING) {
        m->embedding = w;
        return MFH_OK;
    }
    if (role == MFL_EMBEDDING_NORM) {
        m->embedding_norm = w;
        return MFH_OK;
    }
    if (role > MFL_FFN_W3)
        return fail(c, MFH_INVALID_ARGUMENT, "unknown LFM2 weight role");
    if (layer >= m->config.layer_count)
        return fail(c, MFH_OUT_OF_BOUNDS, "LFM2 layer index exceeds the layer count");
    const bool conv = m->kinds[layer] == 0;
    const bool conv_role = role == MFL_CONV_KERNEL || role == MFL_CONV_IN || role == MFL_CONV_OUT;
    const bool attention_role = role >= MFL_QUERY_NORM && role <= MFL_OUTPUT;
    if ((conv && attention_role) || (!conv && conv_role))
        return fail(c, MFH_UNEXPECTED_TENSOR, "LFM2 weight role does not match the layer kind");
    LayerWeights &lw = m->layers[layer];
    Weight *slot[] = {nullptr,          nullptr,         &lw.operator_norm, &lw.ffn_norm,
                      &lw.conv_kernel,  &lw.conv_in,     &lw.conv_out,      &lw.query_norm,
                      &lw.key_norm,     &lw.query,       &lw.key,           &lw.value,
                      &lw.output,       &lw.w1,          &lw.w2,            &lw.w3};
    *slot[role] = w;
    return MFH_OK;
}

mfh_status mfl_reset(mfl_model *m)
{
    if (!m)
        return MFH_INVALID_ARGUMENT;
    DeviceGuard guard(m->ctx->device);
    for (uint32_t i = 0; i < m->config.layer_count; ++i) {
        LayerState &st = m->state[i];
        st.length = 0;
        st.current = 0;
        for (Owned &h : st.history)
            if (h.buf && h.buf->elements)
                launch_fill_f32(m->ctx->stream, static_cast<float *>(h.buf->dev),
                                h.buf->elements, 0.0f);
    }
    m->length = 0;
    return MFH_OK;
}

uint64_t mfl_length(const mfl_model *m)
{
    return m ? m->length : 0;
}

mfh_status mfl_append(mfl_model *m, const uint32_t *tokens, size_t count,
                      const mfh_buf *device_ids, int produce_logits)
{
    if (!m)
        return MFH_INVALID_ARGUMENT;
    if (device_ids && tokens)
        return fail(m->ctx, MFH_INVALID_ARGUMENT, "token ids must be either host or device ids");
    if (!device_ids && count && !tokens)
        return fail(m->ctx, MFH_INVALID_ARGUMENT, "host id pointer is null");
    return append(m, tokens, count, device_ids, produce_logits != 0);
}

mfh_status mfl_sample(mfl_model *m)
{
    if (!m)
        return MFH_INVALID_ARGUMENT;
    return mfh_argmax(m->ctx, m->sampled.buf, m->logits.buf);
}

mfh_status mfl_generate(mfl_model *m, uint32_t steps, mfh_buf *ids_out)
{
    if (!m)
        return MFH_INVALID_ARGUMENT;
    mfh_ctx *c = m->ctx;
    const uint64_t dims[1] = {steps};
    mfh_status s = check_output(c, ids_out, dims, 1);
    if (s)
        return s;
    if (m->length + steps > m->config.max_tokens)
        return fail(c, MFH_OUT_OF_BOUNDS, "append exceeds configured logical prefix capacity");
    mark_written(ids_out);
    const uint32_t vocab = m->config.vocab;
    for (uint32_t i = 0; i < steps; ++i) {
        {
            // mfl_sample, with the selector also written to ids_out[i]: from
            // the LM head's candidates where the fused step left them for
            // these logits, else over the logits.
            DeviceGuard guard(c->device);
            float *ids = static_cast<float *>(ids_out->dev) + i;
            if (m->candidate_count && m->candidate_length == m->length) {
                launch_argmax_candidates(c->stream, static_cast<float *>(m->sampled.buf->dev), ids,
                                         reinterpret_cast<const Candidate *>(dev(m->candidates)),
                                         m->candidate_count);
            } else {
                void *partials = nullptr;
                if (const size_t bytes = argmax_scratch_bytes(1, vocab)) {
                    partials = work_scratch(c, bytes);
                    if (!partials)
                        return allocation_failed(c);
                }
                launch_argmax(c->stream, static_cast<float *>(m->sampled.buf->dev),
                              static_cast<const float *>(m->logits.buf->dev), 1, vocab, nullptr,
                              partials, ids);
            }
        }
        if ((s = append(m, nullptr, 0, m->sampled.buf, true)))
            return s;
    }
    return MFH_OK;
}

const mfh_buf *mfl_logits(const mfl_model *m)
{
    return m ? m->logits.buf : nullptr;
}

const mfh_buf *mfl_sampled(const mfl_model *m)
{
    return m ? m->sampled.buf : nullptr;
}

namespace {

void copy_rows(mfh_ctx *c, mfh_buf *dst, const mfh_buf *src, uint64_t elements)
{
    launch_copy(c->stream, static_cast<float *>(dst->dev), static_cast<const float *>(src->dev),
                elements);
}

}  // namespace

mfh_status mfl_snapshot(mfl_model *m, mfl_prefix **out)
{
    if (!m)
        return MFH_INVALID_ARGUMENT;
    mfh_ctx *c = m->ctx;
    if (!out)
        return fail(c, MFH_INVALID_ARGUMENT, "prefix output pointer is null");
    *out = nullptr;
    auto p = std::make_unique<mfl_prefix>();
    p->ctx = c;
    p->model_id = m->id;
    p->length = m->length;
    p->layers = std::vector<mfl_prefix::Layer>(m->config.layer_count);
    const uint64_t h = m->config.hidden;
    // Allocate everything first, so a ResourceLimit records no copy.
    mfh_status s = MFH_OK;
    for (uint32_t i = 0; i < m->config.layer_count && !s; ++i) {
        mfl_prefix::Layer &pl = p->layers[i];
        const LayerState &st = m->state[i];
        pl.length = st.length;
        if (m->kinds[i] == 0) {
            s = alloc(c, pl.history, m->config.conv_width - 1, h, MFH_CLASS_CACHE, false);
        } else if (st.length) {
            s = alloc(c, pl.key, st.length, m->kv_width, MFH_CLASS_CACHE, false);
            if (!s)
                s = alloc(c, pl.value, st.length, m->kv_width, MFH_CLASS_CACHE, false);
        }
    }
    if (!s)
        s = alloc(c, p->logits, 1, m->config.vocab, MFH_CLASS_CACHE, false);
    if (!s) {
        const uint64_t dims[1] = {1};
        s = mfh_alloc_f32(c, dims, 1, MFH_CLASS_CACHE, 0, &p->sampled.buf);
    }
    if (s)
        return s;
    DeviceGuard guard(c->device);
    for (uint32_t i = 0; i < m->config.layer_count; ++i) {
        mfl_prefix::Layer &pl = p->layers[i];
        const LayerState &st = m->state[i];
        if (m->kinds[i] == 0) {
            copy_rows(c, pl.history.buf, st.history[st.current].buf, pl.history.buf->elements);
        } else if (st.length) {
            copy_rows(c, pl.key.buf, st.key.buf, st.length * m->kv_width);
            copy_rows(c, pl.value.buf, st.value.buf, st.length * m->kv_width);
        }
    }
    copy_rows(c, p->logits.buf, m->logits.buf, m->config.vocab);
    copy_rows(c, p->sampled.buf, m->sampled.buf, 1);
    if (hipGetLastError() != hipSuccess)
        return fail(c, MFH_BACKEND_FAILURE, "prefix copy launch failed");
    *out = p.release();
    return MFH_OK;
}

mfh_status mfl_restore(mfl_model *m, const mfl_prefix *p)
{
    if (!m)
        return MFH_INVALID_ARGUMENT;
    mfh_ctx *c = m->ctx;
    if (!p || p->ctx != c || p->model_id != m->id)
        return fail(c, MFH_INVALID_ARGUMENT, "prefix belongs to another model");
    mfh_status s = check_f32(c, p->logits.buf);
    for (uint32_t i = 0; i < m->config.layer_count && !s; ++i)
        if (m->kinds[i] == 0)
            s = check_f32(c, p->layers[i].history.buf);
        else if (p->layers[i].length && !(s = check_f32(c, p->layers[i].key.buf)))
            s = check_f32(c, p->layers[i].value.buf);
    if (s)
        return s;
    DeviceGuard guard(c->device);
    for (uint32_t i = 0; i < m->config.layer_count; ++i) {
        const mfl_prefix::Layer &pl = p->layers[i];
        LayerState &st = m->state[i];
        st.length = pl.length;
        if (m->kinds[i] == 0) {
            st.current = 0;
            copy_rows(c, st.history[0].buf, pl.history.buf, pl.history.buf->elements);
        } else if (pl.length) {
            copy_rows(c, st.key.buf, pl.key.buf, pl.length * m->kv_width);
            copy_rows(c, st.value.buf, pl.value.buf, pl.length * m->kv_width);
        }
    }
    copy_rows(c, m->logits.buf, p->logits.buf, m->config.vocab);
    copy_rows(c, m->sampled.buf, p->sampled.buf, 1);
    m->length = p->length;
    m->candidate_count = 0;
    if (hipGetLastError() != hipSuccess)
        return fail(c, MFH_BACKEND_FAILURE, "prefix copy launch failed");
    return MFH_OK;
}

uint64_t mfl_prefix_length(const mfl_prefix *p)
{
    return p ? p->length : 0;
}

void mfl_prefix_destroy(mfl_prefix *p)
{
    delete p;
}

}  // extern "C"

namespace {

struct RolePlan {
    uint32_t role, layer;
    std::string name;
    uint64_t dims[3];
    uint32_t rank;
    bool matmul;
};

// weights.rs:268-500: the tensor of every role of the configuration.
std::vector<RolePlan> role_plan(const mfl_model *m)
{
    const mfl_config &c = m->config;
    const uint64_t h = c.hidden, inter = c.intermediate, kv = m->kv_width;
    std::vector<RolePlan> plan;
    plan.push_back({MFL_TOKEN_EMBEDDING, 0, "model.embed_tokens.weight", {c.vocab, h, 0}, 2, true});
    plan.push_back({MFL_EMBEDDING_NORM, 0, "model.embedding_norm.weight", {h, 0, 0}, 1, false});
    for (uint32_t i = 0; i < c.layer_count; ++i) {
        const std::string p = "model.layers." + std::to_string(i);
        if (m->kinds[i] == 0) {
            plan.push_back({MFL_CONV_KERNEL, i, p + ".conv.conv.weight", {h, 1, c.conv_width}, 3,
                            false});
            plan.push_back({MFL_CONV_IN, i, p + ".conv.in_proj.weight", {3 * h, h, 0}, 2, true});
            plan.push_back({MFL_CONV_OUT, i, p + ".conv.out_proj.weight", {h, h, 0}, 2, true});
        } else {
            plan.push_back({MFL_QUERY_NORM, i, p + ".self_attn.q_layernorm.weight",
                            {c.head_dim, 0, 0}, 1, false});
            plan.push_back({MFL_KEY_NORM, i, p + ".self_attn.k_layernorm.weight",
                            {c.head_dim, 0, 0}, 1, false});
            plan.push_back({MFL_QUERY, i, p + ".self_attn.q_proj.weight", {h, h, 0}, 2, true});
            plan.push_back({MFL_KEY, i, p + ".self_attn.k_proj.weight", {kv, h, 0}, 2, true});
            plan.push_back({MFL_VALUE, i, p + ".self_attn.v_proj.weight", {kv, h, 0}, 2, true});
            plan.push_back({MFL_OUTPUT, i, p + ".self_attn.out_proj.weight", {h, h, 0}, 2, true});
        }
        plan.push_back({MFL_FFN_W1, i, p + ".feed_forward.w1.weight", {inter, h, 0}, 2, true});
        plan.push_back({MFL_FFN_W2, i, p + ".feed_forward.w2.weight", {h, inter, 0}, 2, true});
        plan.push_back({MFL_FFN_W3, i, p + ".feed_forward.w3.weight", {inter, h, 0}, 2, true});
        plan.push_back({MFL_FFN_NORM, i, p + ".ffn_norm.weight", {h, 0, 0}, 1, false});
        plan.push_back({MFL_OPERATOR_NORM, i, p + ".operator_norm.weight", {h, 0, 0}, 1, false});
    }
    return plan;
}

mfh_status load_error(mfh_ctx *c, mfh_status s)
{
    // Keep the loader's message on the context too.
    return fail(c, s, mfs_error());
}

bool dims_equal(const uint64_t *a, uint32_t ra, const uint64_t *b, uint32_t rb)
{
    if (ra != rb)
        return false;
    for (uint32_t i = 0; i < ra; ++i)
        if (a[i] != b[i])
            return false;
    return true;
}

}  // namespace

extern "C" {

mfh_status mfl_load_safetensors(mfl_model *m, const mfs_file *file)
{
    if (!m)
        return MFH_INVALID_ARGUMENT;
    mfh_ctx *c = m->ctx;
    if (!file)
        return fail(c, MFH_INVALID_ARGUMENT, "safetensors file is null");
    const std::vector<RolePlan> plan = role_plan(m);
    // 1. Check the whole inventory before uploading anything.
    std::vector<mfs_scheme> schemes(plan.size(), MFS_SCHEME_DENSE);
    std::set<std::string> consumed;
    for (size_t r = 0; r < plan.size(); ++r) {
        const RolePlan &rp = plan[r];
        mfs_dtype dtype;
        uint32_t rank = 0;
        uint64_t dims[4] = {0, 0, 0, 0};
        if (rp.matmul) {
            mfh_status s = mfs_matmul_scheme(file, rp.name.c_str(), &schemes[r]);
            if (s)
                return load_error(c, s);
        }
        if (schemes[r] == MFS_SCHEME_DENSE) {
            mfh_status s = mfs_tensor_info(file, rp.name.c_str(), &dtype, &rank, dims);
            if (s)
                return load_error(c, s);
            if (!dims_equal(dims, rank, rp.dims, rp.rank))
                return fail(c, MFH_INVALID_SHAPE, "tensor shape differs from the model plan");
            if (dtype == MFS_U8)
                return fail(c, MFH_INVALID_DTYPE, "dense LFM2 weights are F32, F16 or BF16");
            consumed.insert(rp.name);
            continue;
        }
        const uint64_t wpb = schemes[r] == MFS_SCHEME_TERNARY ? 4
                             : schemes[r] == MFS_SCHEME_NF4   ? 2
                                                              : 1;
        if (rp.dims[1] % 128)
            return fail(c, MFH_INVALID_SHAPE, "packed weight input width must be a multiple of 128");
        const uint64_t codes_dims[2] = {rp.dims[0], rp.dims[1] / wpb};
        const uint64_t scale_dims[2] = {rp.dims[0], rp.dims[1] / 128};
        const std::string cn = rp.name + ".codes", sn = rp.name + ".scales";
        mfh_status s = mfs_tensor_info(file, cn.c_str(), &dtype, &rank, dims);
        if (s)
            return load_error(c, s);
        if (dtype != MFS_U8 || !dims_equal(dims, rank, codes_dims, 2))
            return fail(c, MFH_INVALID_SHAPE, "packed codes differ from the role's stored scheme");
        if ((s = mfs_tensor_info(file, sn.c_str(), &dtype, &rank, dims)))
            return load_error(c, s);
        if (dtype != MFS_F16 || !dims_equal(dims, rank, scale_dims, 2))
            return fail(c, MFH_INVALID_SHAPE, "packed scales differ from the role's stored scheme");
        consumed.insert(cn);
        consumed.insert(sn);
    }
    for (size_t i = 0; i < mfs_tensor_count(file); ++i)
        if (!consumed.count(mfs_tensor_name(file, i)))
            return fail(c, MFH_UNEXPECTED_TENSOR, "undeclared tensor is present");
    // 2. Upload every role, with its private tile copies, before attaching
    // any: a failure here releases what this load uploaded and leaves the
    // model's weights as they were.
    std::vector<std::unique_ptr<Owned>> staged;  // [tensor, scales or null] per role
    for (size_t r = 0; r < plan.size(); ++r) {
        const RolePlan &rp = plan[r];
        mfh_status s;
        if (schemes[r] == MFS_SCHEME_DENSE) {
            auto t = std::make_unique<Owned>();
            if ((s = mfs_upload_dense(c, file, rp.name.c_str(), MFH_CLASS_WEIGHT, &t->buf)))
                return load_error(c, s);
            if (rp.role == MFL_CONV_KERNEL) {
                // [hidden, 1, width] -> [hidden, width]: the same elements.
                t->buf->rank = 2;
                t->buf->dims[1] = rp.dims[2];
                t->buf->dims[2] = 0;
            }
            staged.push_back(std::move(t));
            staged.push_back(nullptr);
        } else {
            auto codes = std::make_unique<Owned>(), scales = std::make_unique<Owned>();
            if ((s = mfs_upload_packed(c, file, rp.name.c_str(), MFH_CLASS_WEIGHT, &codes->buf,
                                       &scales->buf)))
                return load_error(c, s);
            if ((s = prepare_packed(c, codes->buf, scales->buf)))
                return s;
            staged.push_back(std::move(codes));
            staged.push_back(std::move(scales));
        }
    }
    // 3. Attach.  Step 1 checked every role against the layer kinds and the
    // copies are prepared, so this cannot fail short of a broken plan; if it
    // does, the previous weights are put back.
    const Weight embedding = m->embedding, embedding_norm = m->embedding_norm;
    const std::vector<LayerWeights> layers = m->layers;
    for (size_t r = 0; r < plan.size(); ++r) {
        const Owned *t = staged[2 * r].get(), *sc = staged[2 * r + 1].get();
        const mfh_status s =
            mfl_set_weight(m, plan[r].role, plan[r].layer, t->buf, sc ? sc->buf : nullptr);
        if (s) {
            m->embedding = embedding;
            m->embedding_norm = embedding_norm;
            m->layers = layers;
            return s;
        }
    }
    // Every role of the plan now holds this load's buffers, so an earlier
    // load's are released (into the stream-ordered pool: passes already
    // queued still read them safely).
    m->loaded.clear();
    for (auto &o : staged)
        if (o)
            m->loaded.push_back(std::move(o));
    return MFH_OK;
}

}  // extern "C"
