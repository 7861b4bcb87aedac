// f32 vector-ALU decode GEMV for wide contractions: one activation row,
// 4096 <= K <= 8192 (the FFN down projections, 2048 x 8192 and 1024 x 4608),
// NF4 from K = 2048 (the LFM2-1.2B attention and convolution projections),
// ternary below 2048 rows from K = 1024 (the LFM2-350M ones).
//
// out[b, n] = sum_g scale[n, g] * sum_{k in g} x[b, k] * level(code[n, k])
// in f32, the reference's group-then-scale order
// (crates/kernels-simd/src/lib.rs:54,168,205); only the order of the
// additions inside a group and across groups differs from the CPU.
//
// Why a vector kernel here.  At these widths the integer-MFMA GEMV cannot
// form its activation digits inside the kernel (each wave's K share is too
// long for the register prologue), so it runs behind a separate prologue
// kernel: two dependent launches per product.  This kernel reads the f32
// activations as they are, in one launch; at one row its arithmetic (about
// 2.5 vector instructions per weight) stays below the launch and memory
// latency it replaces.  Measured against the two launches, one row (with
// 32-wide slices):
// 1024 x 4608 ternary 6.9 -> 4.2 us, 2048 x 8192 7.2 -> 7.05 us (INT8 8.0 ->
// 7.6, NF4 8.1 -> 7.6); LFM2 decode 350M shape 2172 -> 2376 tok/s, 1.2B
// 1567 -> 1596.  Two rows measured slower (2048 x 8192 ternary 9.1 us), and
// so did forming SwiGLU activations here, which every block would recompute
// for all of K (1.2B-shape op-by-op decode, whose down projections take
// packed_swiglu_linear, 1254 -> 1170 tok/s).
//
// Layout.  Lane L of wave w owns the SL-wide k slice s = 64 w + L for every
// row of the block: it holds its SL activations in registers and reads the
// slice's codes of each row from the canonical row-major stream (SL / 4,
// SL / 2 or SL bytes: ternary, NF4, INT8), so a wave reads 64 SL / 4 to 64 SL
// bytes of one row contiguously.  128 / SL lanes make a 128-group: their
// partial sums add over the lane quad (DPP) and shuffles, the sum is scaled,
// and the groups add across the wave (shuffles) and across the block's waves
// (LDS, in wave order).  A block holds R rows (R = 4 from 2048 rows, else
// 2, at least 512 blocks; ternary rows below 2048 at K < 4096 take one and
// the norm variant four for NF4, two for ternary, as measured in the decode
// chain; 2048 x 8192 with R = 1, 2, 8 took 10.2, 7.2, 8.8
// us against 7.05, 1024 x 4608 with R = 4 5.3 against 4.2) and
// ceil(K / (64 SL)) waves.  SL = 16 from 2048 rows, else 8: shorter slices
// halve each lane's dependent arithmetic and spread it over more waves.
// Inside the LFM2 decode chain SL = 32 / 16 / 8 measured 1593 / 1635 / 1629
// tok/s for the 1.2B shape (2048 x 8192 down projections) and 2370 / 2424 /
// 2440 for the 350M shape (1024 x 4608); back to back at 2048 x 8192, one
// row, ternary 7.0 / 6.2 / 6.4 us, INT8 7.5 / 6.6 / 6.9, NF4 7.6 / 7.3 / 7.8.
//
// Norm variant (NF4 at 2048 <= K <= 8192, ternary from K = 1024; one row,
// optionally segmented into up to three weight streams): each lane adds the right-hand row to its
// slice, the block sums the squares (its waves cover all of K), and the
// activations become (s * reciprocal) * weight as in the reference's
// add_row_rms_norm (backend-cpu/src/normalization_rotary.rs:223); block 0 also
// writes the sum row.  It serves the LFM2 decode step's norm-fed NF4 and
// ternary products (conv in-projections, grouped q/k/v).
//
// Convolution variant of the norm variant (the conv in-projection of the
// decode step): block c computes rows c, h + c and 2h + c (the B, C and x
// chunks of channel c), so its epilogue holds everything one token of the
// gated short convolution of channel c needs and finishes it (ConvStep;
// conv_step_kernel's arithmetic, so the outputs equal the two-launch form bit
// for bit), rolling the history into the second buffer.  One launch per
// convolution block instead of two.
//
// Decode (crates/kernels-simd/src/lib.rs:31-57,113-130,145-183):
//   ternary  level = c - 1, c = 2-bit field (code 3 gives +2, as on the CPU):
//            sum (c - 1) x = sum c x - sum x, with c converted by byte;
//   INT8     level = signed byte b: the byte of code ^ 0x80 is b + 128, so
//            sum b x = sum (b + 128) x - 128 sum x;
//   NF4      a 256-entry LDS table of (low nibble, high nibble) level pairs.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <type_traits>

#include "kernels.hpp"

namespace mfh {
namespace {

constexpr uint32_t kMinK = 4096;
constexpr uint32_t kMaxK = 8192;
constexpr int kMaxWaves = 16;  // K = 8192 at SL = 8
// Widest weight matrix served; wider ones (LM heads) stream better on the
// matrix cores.
constexpr uint32_t kMaxRows = 8192;

__constant__ float kLevelsV[16] = {
    -1.0f,        -0.6961928f,  -0.52507305f, -0.3949175f,
    -0.28444138f, -0.18477343f, -0.091050036f, 0.0f,
    0.0795803f,   0.1609302f,   0.2461123f,   0.33791524f,
    0.44070983f,  0.562617f,    0.72295684f,  1.0f,
};

struct VArgs {
    const float *x;  // [k]
    const uint8_t *codes;
    const float *scales;
    const uint16_t *scales16;  // binary16 copy of scales, or null
    float *out;  // [n]
    uint32_t n, k;
    // Norm variant: x = ((x + right) * reciprocal) * weight (right may be
    // null), the sum row written to `side` (if set) by block 0.
    const float *right, *weight;
    float *side;
    float epsilon;
    // Norm variant: blocks [seg_first[i], seg_first[i + 1]) run stream i
    // (0 segments: the single stream above).
    uint32_t segments;
    uint32_t seg_first[kMaxSegments];
    const uint8_t *seg_codes[kMaxSegments];
    const float *seg_scales[kMaxSegments];
    const uint16_t *seg_scales16[kMaxSegments];
    float *seg_out[kMaxSegments];
    uint32_t seg_n[kMaxSegments];
    // Convolution variant: the block's rows are c, hidden + c and
    // 2 hidden + c of its R channels c, and its epilogue finishes their
    // one-token convolution (ConvStep).
    ConvStep conv;
};

// Code words of one row's SL-wide slice: N words of EB bytes each (a slice
// of two bytes, ternary at SL = 8, is one half-filled word).
template <Format F, int SL>
struct Slice {
    static constexpr int bytes = SL / weights_per_byte(F);
    static constexpr int N = bytes >= 4 ? bytes / 4 : 1;
    static constexpr int EB = bytes >= 4 ? 4 : bytes;
};

template <int N, int EB>
__device__ __forceinline__ void load_slice(const uint8_t *p, unsigned (&w)[N])
{
    if constexpr (EB == 2) {
        w[0] = *reinterpret_cast<const unsigned short *>(p);
    } else if constexpr (N == 1) {
        w[0] = *reinterpret_cast<const unsigned *>(p);
    } else if constexpr (N == 2) {
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        w[0] = v.x;
        w[1] = v.y;
    } else {
#pragma unroll
        for (int h = 0; h < N / 4; ++h) {
            const uint4 v = reinterpret_cast<const uint4 *>(p)[h];
            w[4 * h] = v.x;
            w[4 * h + 1] = v.y;
            w[4 * h + 2] = v.z;
            w[4 * h + 3] = v.w;
        }
    }
}

// Byte e of a word as f32 (one v_cvt_f32_ubyte).
__device__ __forceinline__ float byte_f(unsigned w, int e)
{
    return float((w >> (8 * e)) & 0xFFu);
}

// The lane's partial dot over its slice: sum level(code) * x, before the
// ternary / INT8 offset correction (applied by the caller from sum x).
template <Format F, int SL, int N, int EB>
__device__ __forceinline__ float slice_dot(const unsigned (&c)[N], const float (&x)[SL],
                                           const float2 *pairs)
{
    float dot = 0.0f;
#pragma unroll
    for (int q = 0; q < N; ++q) {
        if constexpr (F == Format::Ternary) {
            // Word q holds k = 16q + 4e + f at byte e, field f.
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                const unsigned t = (c[q] >> (2 * f)) & 0x03030303u;
#pragma unroll
                for (int e = 0; e < EB; ++e)
                    dot = fmaf(byte_f(t, e), x[16 * q + 4 * e + f], dot);
            }
        } else if constexpr (F == Format::Nf4) {
            // Byte e of word q holds k = 8q + 2e (low nibble) and 8q + 2e + 1.
#pragma unroll
            for (int e = 0; e < EB; ++e) {
                const float2 lv = pairs[(c[q] >> (8 * e)) & 0xFFu];
                dot = fmaf(lv.x, x[8 * q + 2 * e], dot);
                dot = fmaf(lv.y, x[8 * q + 2 * e + 1], dot);
            }
        } else {
            // Word q holds k = 4q + e at byte e.
            const unsigned d = c[q] ^ 0x80808080u;
#pragma unroll
            for (int e = 0; e < EB; ++e)
                dot = fmaf(byte_f(d, e), x[4 * q + e], dot);
        }
    }
    return dot;
}

template <int CTRL>
__device__ __forceinline__ float quad_add(float v)
{
    return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <Format F, int R, int SL, int NORM, bool CONV = false>
__global__ __launch_bounds__(64 * kMaxWaves) void vgemv_kernel(VArgs a)
{
    using SC = Slice<F, SL>;
    constexpr int LPG = 128 / SL;  // lanes per 128-group
    // Rows per block: R, or the three chunks of R channels (CONV).
    constexpr int RR = CONV ? 3 * R : R;
    __shared__ float2 pairs[F == Format::Nf4 ? 256 : 1];
    __shared__ float red[kMaxWaves][RR];
    __shared__ float squares_of[NORM ? kMaxWaves : 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // The block's weight stream (compile-time segment indices only: a
    // dynamic index into the argument arrays would copy them to scratch).
    uint32_t block = blockIdx.x;
    const uint8_t *codes_of = a.codes;
    const float *scales_of = a.scales;
    const uint16_t *scales16_of = a.scales16;
    float *out = a.out;
    uint32_t n = a.n;
    if constexpr (NORM) {
        uint32_t first = 0;
#pragma unroll
        for (uint32_t sg = 0; sg < kMaxSegments; ++sg) {
            if (sg < a.segments && block >= a.seg_first[sg]) {
                codes_of = a.seg_codes[sg];
                scales_of = a.seg_scales[sg];
                scales16_of = a.seg_scales16[sg];
                out = a.seg_out[sg];
                n = a.seg_n[sg];
                first = a.seg_first[sg];
            }
        }
        block -= first;
    }
    if constexpr (F == Format::Nf4) {
        for (int e = tid; e < 256; e += blockDim.x)
            pairs[e] = float2{kLevelsV[e & 15], kLevelsV[e >> 4]};
    }
    const uint32_t slices = a.k / SL;
    const uint32_t slice = uint32_t(wave) * 64 + lane;
    const bool live = slice < slices;
    const uint32_t sl = live ? slice : 0;  // dead lanes read slice 0, contribute 0
    const uint32_t row0 = block * R;
    constexpr int wpb = weights_per_byte(F);
    const size_t row_bytes = a.k / wpb;
    const uint32_t groups = a.k / 128;

    // Loads in the order they are needed: activations (from L2), then every
    // row's codes and group scale.
    float x[SL];
    const float4 *xp = reinterpret_cast<const float4 *>(a.x + sl * SL);
#pragma unroll
    for (int q = 0; q < SL / 4; ++q) {
        const float4 v = xp[q];
        x[4 * q] = v.x;
        x[4 * q + 1] = v.y;
        x[4 * q + 2] = v.z;
        x[4 * q + 3] = v.w;
    }
    if constexpr (NORM) {
        // s = x + right over the slice, the row's squares summed over the
        // block (its waves cover all of K), then the reference's
        // (s * reciprocal) * weight.
        // NORM == 2: no right-hand row (the first layer's block input); a
        // separate instantiation, so that no load waits behind a branch.
        const float4 *rp = reinterpret_cast<const float4 *>(a.right + sl * SL);
        const float4 *wp = reinterpret_cast<const float4 *>(a.weight + sl * SL);
        float w[SL];
#pragma unroll
        for (int q = 0; q < SL / 4; ++q) {
            const float4 u = wp[q];
            if constexpr (NORM == 1) {
                const float4 v = rp[q];
                x[4 * q] += v.x;
                x[4 * q + 1] += v.y;
                x[4 * q + 2] += v.z;
                x[4 * q + 3] += v.w;
            }
            w[4 * q] = u.x;
            w[4 * q + 1] = u.y;
            w[4 * q + 2] = u.z;
            w[4 * q + 3] = u.w;
        }
        float squares = 0.0f;
#pragma unroll
        for (int j = 0; j < SL; ++j)
            squares += x[j] * x[j];
        squares = live ? squares : 0.0f;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1)
            squares += __shfl_xor(squares, off, 64);
        if (lane == 0)
            squares_of[wave] = squares;
        if (blockIdx.x == 0 && live && a.side) {
            float4 *sp = reinterpret_cast<float4 *>(a.side + sl * SL);
#pragma unroll
            for (int q = 0; q < SL / 4; ++q)
                sp[q] = float4{x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]};
        }
        __syncthreads();
        float total = 0.0f;
        for (int wv = 0; wv < int(blockDim.x >> 6); ++wv)
            total += squares_of[wv];
        const float reciprocal = 1.0f / sqrtf(total / float(a.k) + a.epsilon);
#pragma unroll
        for (int j = 0; j < SL; ++j)
            x[j] = (x[j] * reciprocal) * w[j];
    }
    unsigned codes[RR][SC::N];
    float scale[RR];
#pragma unroll
    for (int r = 0; r < RR; ++r) {
        // CONV: chunk r / R (B, C, x) of channel row0 + r % R.
        const uint32_t want = CONV ? (r / R) * a.conv.hidden + row0 + r % R : row0 + r;
        const uint32_t row = want < n ? want : n - 1;
        load_slice<SC::N, SC::EB>(codes_of + row * row_bytes + size_t(sl) * SC::bytes, codes[r]);
        const size_t si = size_t(row) * groups + sl / LPG;
        scale[r] = scales16_of ? __half2float(reinterpret_cast<const __half *>(scales16_of)[si])
                              : scales_of[si];
    }
    // Offset correction: sum x over the slice (ternary, INT8).
    float xsum = 0.0f;
#pragma unroll
    for (int j = 0; j < SL; ++j)
        xsum += x[j];
    xsum = F == Format::Ternary ? xsum : F == Format::Int8 ? 128.0f * xsum : 0.0f;
    if constexpr (F == Format::Nf4)
        __syncthreads();  // the level table

    float val[RR];
#pragma unroll
    for (int r = 0; r < RR; ++r) {
        float v = slice_dot<F, SL, SC::N, SC::EB>(codes[r], x, pairs) - xsum;
        // Group sum over its lanes (all end equal), then the group's scale.
        v = quad_add<0xB1>(v);  // quad_perm [1, 0, 3, 2]
        v = quad_add<0x4E>(v);  // quad_perm [2, 3, 0, 1]
#pragma unroll
        for (int off = 4; off < LPG; off <<= 1)
            v += __shfl_xor(v, off, 64);
        v = live ? v * scale[r] : 0.0f;
        // The wave's groups.
#pragma unroll
        for (int off = LPG; off < 64; off <<= 1)
            v += __shfl_xor(v, off, 64);
        val[r] = v;
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RR; ++r)
            red[wave][r] = val[r];
    }
    __syncthreads();
    const int waves = blockDim.x >> 6;
    if constexpr (CONV) {
        // Wave 0: lane r < 3R sums row r (the in-projection value), then
        // lane c < R holds B, C and x of channel row0 + c and finishes
        // conv_step_kernel's arithmetic for it.
        if (wave == 0) {
            const int r = tid < RR ? tid : 0;
            float sum = red[0][r];
            for (int w = 1; w < waves; ++w)
                sum += red[w][r];
            const float cgate = __shfl(sum, (tid + R) & 63, 64);
            const float xval = __shfl(sum, (tid + 2 * R) & 63, 64);
            const uint32_t channel = row0 + uint32_t(tid);
            const ConvStep &cv = a.conv;
            if (tid < R && channel < cv.hidden) {
                const uint32_t rows = cv.width - 1;
                const float u = sum * xval;
                const float *taps = cv.kernel + uint64_t(channel) * cv.width;
                float total = 0.0f;
                for (uint32_t tap = 0; tap < rows; ++tap)
                    total += taps[tap] * cv.history[uint64_t(tap) * cv.hidden + channel];
                total += taps[rows] * u;
                for (uint32_t rr = 0; rr + 1 < rows; ++rr)
                    cv.next[uint64_t(rr) * cv.hidden + channel] =
                        cv.history[uint64_t(rr + 1) * cv.hidden + channel];
                if (rows)
                    cv.next[uint64_t(rows - 1) * cv.hidden + channel] = u;
                cv.out[channel] = total * cgate;
            }
        }
    } else if (tid < R) {
        float sum = red[0][tid];
        for (int w = 1; w < waves; ++w)
            sum += red[w][tid];
        const uint32_t row = row0 + tid;
        if (row < n)
            out[row] = sum;
    }
}

template <Format F, int R, int SL>
void launch_shape(hipStream_t stream, const VArgs &args)
{
    const unsigned waves = (args.k + 64 * SL - 1) / (64 * SL);
    vgemv_kernel<F, R, SL, 0><<<(args.n + R - 1) / R, 64 * waves, 0, stream>>>(args);
}

// The norm variant: 8-wide slices (16-wide measured 1665 against 1681 tok/s
// for 1.2B-shape decode) and norm_rows(F) rows per block (ternary 2: 350M
// decode 2583 -> 2635 against 4; NF4 keeps 4, 1679 against 1654 tok/s for
// the 1.2B shape with 2); `blocks` covers every segment (each a multiple of
// that many rows).
constexpr uint32_t norm_rows(Format f)
{
    return f == Format::Ternary ? 2 : 4;
}

template <Format F>
void launch_norm(hipStream_t stream, const VArgs &args, unsigned blocks)
{
    constexpr int R = int(norm_rows(F));
    const unsigned waves = (args.k + 64 * 8 - 1) / (64 * 8);
    if (args.right)
        vgemv_kernel<F, R, 8, 1><<<blocks, 64 * waves, 0, stream>>>(args);
    else
        vgemv_kernel<F, R, 8, 2><<<blocks, 64 * waves, 0, stream>>>(args);
}

template <Format F>
void launch_format_v(hipStream_t stream, const VArgs &args)
{
    // Ternary rows below 2048 at K < 4096 (the 350M-shape output
    // projections): one row per block (350M decode 2583 -> 2600 against two;
    // four measured 2516).
    if (F == Format::Ternary && args.n < 2048 && args.k < 4096)
        return launch_shape<F, 1, 8>(stream, args);
    if (args.n >= 2048)
        launch_shape<F, 4, 16>(stream, args);
    else
        launch_shape<F, 2, 8>(stream, args);
}

bool aligned16(const void *p)
{
    return reinterpret_cast<uintptr_t>(p) % 16 == 0;
}

}  // namespace

namespace {

// Products whose activations are add + RMS norm of two rows: NF4 at
// 2048 <= K <= 8192 (the LFM2-1.2B conv in-projections and the grouped
// q/k/v launch) and ternary from K = 1024 (the same roles at the 350M
// shape) take the norm variant.  Against the matrix-core GEMV with its norm
// prologue: 1.2B-shape decode 1631 -> 1656 tok/s (NF4, LDS prologue), 350M
// 2450 -> 2499 (ternary, register prologue).  INT8 stays on the matrix
// cores, which were as fast or faster at one plain row for K <= 2048.
constexpr uint32_t kNormMinK = 2048;
constexpr uint32_t kTernaryMinK = 1024;

bool try_norm(hipStream_t stream, const PackedCall &call)
{
    const XForm &t = call.xform;
    const uint32_t min_k = call.format == Format::Ternary ? kTernaryMinK : kNormMinK;
    if (call.format == Format::Int8 || t.kind != XKind::AddRms || call.separate_prologue ||
        call.epilogue != Epilogue::Single || call.m != 1 || call.k < min_k ||
        call.k > kMaxK || call.k % 128 || !t.a || !t.w || !aligned16(t.a) ||
        (t.b && !aligned16(t.b)) || !aligned16(t.w) || (t.side && !aligned16(t.side)))
        return false;
    const uint32_t rows = norm_rows(call.format);
    VArgs args{};
    args.x = t.a;
    args.right = t.b;
    args.weight = t.w;
    args.side = t.side;
    args.epsilon = t.epsilon;
    args.k = call.k;
    unsigned blocks = 0;
    if (call.segments) {
        for (uint32_t i = 0; i < call.segments; ++i) {
            if (call.seg_n[i] == 0 || call.seg_n[i] % rows || !call.seg[i].codes ||
                !call.seg[i].scales)
                return false;
            args.seg_first[i] = blocks;
            args.seg_codes[i] = call.seg[i].codes;
            args.seg_scales[i] = call.seg[i].scales;
            args.seg_scales16[i] = call.seg[i].scales16;
            args.seg_out[i] = call.seg_out[i];
            args.seg_n[i] = call.seg_n[i];
            blocks += call.seg_n[i] / rows;
        }
        args.segments = call.segments;
    } else {
        if (call.n == 0 || call.n > kMaxRows || !call.a.codes || !call.a.scales)
            return false;
        args.codes = call.a.codes;
        args.scales = call.a.scales;
        args.scales16 = call.a.scales16;
        args.out = call.out_a;
        args.n = call.n;
        blocks = (call.n + rows - 1) / rows;
    }
    if (call.format == Format::Ternary)
        launch_norm<Format::Ternary>(stream, args, blocks);
    else
        launch_norm<Format::Nf4>(stream, args, blocks);
    return true;
}

}  // namespace

bool try_vgemv_conv(hipStream_t stream, const PackedCall &call, const ConvStep &conv)
{
    const XForm &t = call.xform;
    const uint32_t min_k = call.format == Format::Ternary ? kTernaryMinK : kNormMinK;
    if (call.format == Format::Int8 || t.kind != XKind::AddRms || call.separate_prologue ||
        call.segments || call.epilogue != Epilogue::Single || call.m != 1 || call.k < min_k ||
        call.k > kMaxK || call.k % 128 || !t.a || !t.w || !aligned16(t.a) ||
        (t.b && !aligned16(t.b)) || !aligned16(t.w) || (t.side && !aligned16(t.side)) ||
        conv.hidden == 0 || call.n != 3 * conv.hidden || conv.width < 1 || !call.a.codes ||
        !call.a.scales)
        return false;
    VArgs args{};
    args.x = t.a;
    args.right = t.b;
    args.weight = t.w;
    args.side = t.side;
    args.epsilon = t.epsilon;
    args.k = call.k;
    args.codes = call.a.codes;
    args.scales = call.a.scales;
    args.scales16 = call.a.scales16;
    args.n = call.n;
    args.conv = conv;
    // One channel (three rows) per block: LFM2 decode 1.2B shape 304.4 ->
    // 293.9 ms per 512 tokens against the projection + conv_step_kernel
    // launches, 350M 96.3 -> 94.0 ms per 256; two channels per block 300.5 /
    // 96.2, four (the norm variant's row count) 314.5 / 101.8.
    const unsigned waves = (args.k + 64 * 8 - 1) / (64 * 8);
    auto go = [&](auto f_tag) {
        constexpr Format F = decltype(f_tag)::value;
        if (args.right)
            vgemv_kernel<F, 1, 8, 1, true><<<conv.hidden, 64 * waves, 0, stream>>>(args);
        else
            vgemv_kernel<F, 1, 8, 2, true><<<conv.hidden, 64 * waves, 0, stream>>>(args);
    };
    if (call.format == Format::Ternary)
        go(std::integral_constant<Format, Format::Ternary>{});
    else
        go(std::integral_constant<Format, Format::Nf4>{});
    return true;
}

bool try_vgemv(hipStream_t stream, const PackedCall &call)
{
    if (try_norm(stream, call))
        return true;
    const float *x = call.xform.kind == XKind::Plain ? call.x : nullptr;
    // NF4 from K = 2048 (its matrix-core GEMV carries the table decode and
    // hi/lo products): 1.2B-shape decode 1662 -> 1667 tok/s, op by op 1297 ->
    // 1320, where the 2048 x 2048 and 6144 x 2048 products move here.
    // Ternary from K = 1024 below 2048 rows (the 350M-shape output
    // projections, 1024 x 1024): 350M decode 2499 -> 2582 tok/s; at 2048 x
    // 2048 and 4608 x 1024 the matrix cores stayed faster (4.2 against
    // 4.7-4.9 us).
    const uint32_t min_k = call.format == Format::Nf4 ? kNormMinK
                           : call.format == Format::Ternary && call.n < 2048 ? kTernaryMinK
                                                                            : kMinK;
    if (call.separate_prologue || call.segments || call.epilogue != Epilogue::Single ||
        call.m != 1 || call.k < min_k || call.k > kMaxK || call.k % 128 || call.n == 0 ||
        call.n > kMaxRows || !call.a.codes || !call.a.scales || !x || !aligned16(x))
        return false;
    VArgs args{};
    args.x = x;
    args.codes = call.a.codes;
    args.scales = call.a.scales;
    args.scales16 = call.a.scales16;
    args.out = call.out_a;
    args.n = call.n;
    args.k = call.k;
    switch (call.format) {
    case Format::Ternary: launch_format_v<Format::Ternary>(stream, args); break;
    case Format::Nf4: launch_format_v<Format::Nf4>(stream, args); break;
    case Format::Int8: launch_format_v<Format::Int8>(stream, args); break;
    }
    return true;
}

}  // namespace mfh
