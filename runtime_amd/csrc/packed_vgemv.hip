// f32 vector-ALU decode GEMV for wide contractions: one activation row,
// 4096 <= K <= 8192 (the FFN down projections, 2048 x 8192 and 1024 x 4608).
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
// latency it replaces.  Measured against the two launches, one row:
// 1024 x 4608 ternary 6.9 -> 4.2 us, 2048 x 8192 7.2 -> 7.05 us (INT8 8.0 ->
// 7.6, NF4 8.1 -> 7.6); LFM2 decode 350M shape 2172 -> 2376 tok/s, 1.2B
// 1567 -> 1596.  Two rows measured slower (2048 x 8192 ternary 9.1 us), and
// so did forming SwiGLU activations here: every block would recompute them
// for all of K.
//
// Layout.  Lane L of wave w owns the 32-wide k slice s = 64 w + L for every
// row of the block: it holds its 32 activations in registers
// and reads the slice's codes of each row from the canonical row-major
// stream (8, 16 or 32 bytes: ternary, NF4, INT8), so a wave reads 512 B - 2 KB
// of one row contiguously.  Four lanes make a 128-group: their partial sums
// add over the lane quad (DPP), the sum is scaled, and the groups add across
// the wave (shuffles) and across the block's waves (LDS, in wave order).
// A block holds R rows (R = 4 from 2048 rows, else 2: at least 512 blocks;
// 2048 x 8192 with R = 1, 2, 8 took 10.2, 7.2, 8.8 us against 7.05, 1024 x
// 4608 with R = 4 5.3 against 4.2) and ceil(K / 2048) waves.
//
// Decode (crates/kernels-simd/src/lib.rs:31-57,113-130,145-183):
//   ternary  level = c - 1, c = 2-bit field (code 3 gives +2, as on the CPU):
//            sum (c - 1) x = sum c x - sum x, with c converted by byte;
//   INT8     level = signed byte b: the byte of code ^ 0x80 is b + 128, so
//            sum b x = sum (b + 128) x - 128 sum x;
//   NF4      a 256-entry LDS table of (low nibble, high nibble) level pairs.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace mfh {
namespace {

constexpr int kSlice = 32;                // k per lane
constexpr uint32_t kWaveK = 64 * kSlice;  // k per wave
constexpr uint32_t kMinK = 4096;
constexpr uint32_t kMaxK = 4 * kWaveK;  // four waves
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
};

// Code bytes of one row's 32-k slice.
template <Format F> struct SliceCodes;
template <> struct SliceCodes<Format::Ternary> { uint2 v; };
template <> struct SliceCodes<Format::Nf4> { uint4 v; };
template <> struct SliceCodes<Format::Int8> { uint4 v[2]; };

template <Format F>
__device__ __forceinline__ SliceCodes<F> load_slice(const uint8_t *p)
{
    SliceCodes<F> c;
    if constexpr (F == Format::Ternary) {
        c.v = *reinterpret_cast<const uint2 *>(p);
    } else if constexpr (F == Format::Nf4) {
        c.v = *reinterpret_cast<const uint4 *>(p);
    } else {
        c.v[0] = reinterpret_cast<const uint4 *>(p)[0];
        c.v[1] = reinterpret_cast<const uint4 *>(p)[1];
    }
    return c;
}

// Byte e of a word as f32 (one v_cvt_f32_ubyte).
__device__ __forceinline__ float byte_f(unsigned w, int e)
{
    return float((w >> (8 * e)) & 0xFFu);
}

// The lane's partial dot over its slice: sum level(code) * x, before the
// ternary / INT8 offset correction (applied by the caller from sum x).
template <Format F>
__device__ __forceinline__ float slice_dot(const SliceCodes<F> &c, const float (&x)[kSlice],
                                           const float2 *pairs)
{
    float dot = 0.0f;
    if constexpr (F == Format::Ternary) {
        // Word q holds k = 16q + 4e + f at byte e, field f.
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const unsigned d = q ? c.v.y : c.v.x;
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                const unsigned t = (d >> (2 * f)) & 0x03030303u;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    dot = fmaf(byte_f(t, e), x[16 * q + 4 * e + f], dot);
            }
        }
    } else if constexpr (F == Format::Nf4) {
        // Byte j = 4q + e holds k = 2j (low nibble) and 2j + 1 (high).
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const unsigned d = q == 0 ? c.v.x : q == 1 ? c.v.y : q == 2 ? c.v.z : c.v.w;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float2 lv = pairs[(d >> (8 * e)) & 0xFFu];
                dot = fmaf(lv.x, x[8 * q + 2 * e], dot);
                dot = fmaf(lv.y, x[8 * q + 2 * e + 1], dot);
            }
        }
    } else {
        // Word q of the 32 bytes holds k = 4q + e at byte e.
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 &u = c.v[h];
                const unsigned d =
                    (q == 0 ? u.x : q == 1 ? u.y : q == 2 ? u.z : u.w) ^ 0x80808080u;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    dot = fmaf(byte_f(d, e), x[16 * h + 4 * q + e], dot);
            }
    }
    return dot;
}

template <int CTRL>
__device__ __forceinline__ float quad_add(float v)
{
    return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <Format F, int R>
__global__ __launch_bounds__(256) void vgemv_kernel(VArgs a)
{
    __shared__ float2 pairs[F == Format::Nf4 ? 256 : 1];
    __shared__ float red[4][R];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if constexpr (F == Format::Nf4) {
        for (int e = tid; e < 256; e += blockDim.x)
            pairs[e] = float2{kLevelsV[e & 15], kLevelsV[e >> 4]};
    }
    const uint32_t slices = a.k / kSlice;
    const uint32_t slice = uint32_t(wave) * 64 + lane;
    const bool live = slice < slices;
    const uint32_t sl = live ? slice : 0;  // dead lanes read slice 0, contribute 0
    const uint32_t row0 = blockIdx.x * R;
    constexpr int wpb = weights_per_byte(F);
    const size_t row_bytes = a.k / wpb;
    const uint32_t groups = a.k / 128;

    // Loads in the order they are needed: activations (from L2), then every
    // row's codes and group scale.
    float x[kSlice];
    const float4 *xp = reinterpret_cast<const float4 *>(a.x + sl * kSlice);
#pragma unroll
    for (int q = 0; q < kSlice / 4; ++q) {
        const float4 v = xp[q];
        x[4 * q] = v.x;
        x[4 * q + 1] = v.y;
        x[4 * q + 2] = v.z;
        x[4 * q + 3] = v.w;
    }
    SliceCodes<F> codes[R];
    float scale[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = row0 + r < a.n ? row0 + r : a.n - 1;
        codes[r] = load_slice<F>(a.codes + row * row_bytes + size_t(sl) * (kSlice / wpb));
        const size_t si = size_t(row) * groups + sl / 4;
        scale[r] = a.scales16 ? __half2float(reinterpret_cast<const __half *>(a.scales16)[si])
                              : a.scales[si];
    }
    // Offset correction: sum x over the slice (ternary, INT8).
    float xsum = 0.0f;
#pragma unroll
    for (int j = 0; j < kSlice; ++j)
        xsum += x[j];
    xsum = F == Format::Ternary ? xsum : F == Format::Int8 ? 128.0f * xsum : 0.0f;
    if constexpr (F == Format::Nf4)
        __syncthreads();  // the level table

    float val[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float v = slice_dot<F>(codes[r], x, pairs) - xsum;
        // Group sum over the lane quad (all four lanes end equal), then the
        // group's scale.
        v = quad_add<0xB1>(v);  // quad_perm [1, 0, 3, 2]
        v = quad_add<0x4E>(v);  // quad_perm [2, 3, 0, 1]
        v = live ? v * scale[r] : 0.0f;
        // The wave's 16 groups.
#pragma unroll
        for (int off = 4; off < 64; off <<= 1)
            v += __shfl_xor(v, off, 64);
        val[r] = v;
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            red[wave][r] = val[r];
    }
    __syncthreads();
    const int waves = blockDim.x >> 6;
    if (tid < R) {
        float sum = red[0][tid];
        for (int w = 1; w < waves; ++w)
            sum += red[w][tid];
        const uint32_t row = row0 + tid;
        if (row < a.n)
            a.out[row] = sum;
    }
}

template <Format F>
void launch_format_v(hipStream_t stream, const VArgs &args)
{
    const unsigned threads = 64 * ((args.k + kWaveK - 1) / kWaveK);
    if (args.n >= 2048)
        vgemv_kernel<F, 4><<<(args.n + 3) / 4, threads, 0, stream>>>(args);
    else
        vgemv_kernel<F, 2><<<(args.n + 1) / 2, threads, 0, stream>>>(args);
}

bool aligned16(const void *p)
{
    return reinterpret_cast<uintptr_t>(p) % 16 == 0;
}

}  // namespace

bool try_vgemv(hipStream_t stream, const PackedCall &call)
{
    const float *x = call.xform.kind == XKind::Plain ? call.x : nullptr;
    if (call.separate_prologue || call.segments || call.epilogue != Epilogue::Single ||
        call.m != 1 || call.k < kMinK || call.k > kMaxK || call.k % 128 || call.n == 0 ||
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
