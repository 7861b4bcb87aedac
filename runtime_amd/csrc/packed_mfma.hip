// Matrix-core decode GEMV (m <= 8) for ternary, NF4 and INT8 streams.
//
// Ternary and INT8 (integer MFMA).  Activation row b is split into 128-wide
// groups; group g is scaled by a power of two so its largest magnitude is
// below 2^30 and rounded to v = rint(x * 2^(30 - e_bg)), a 31-bit integer
// written as four signed digits v = d0*2^24 + d1*2^16 + d2*2^8 + d3.
// Weight codes are exact small integers (ternary code c in {0,1,2}, INT8 in
// [-127, 127]), so v_mfma_i32_16x16x64_i8 forms every per-group digit dot
// sum_k code_k * d_k exactly in int32.  Per group the four digit sums are
// combined, multiplied by the group's weight scale and 2^(e_bg - 30), and
// accumulated in f32 -- the reference's group-then-scale order
// (kernels-simd/src/lib.rs:54,205).  Ternary codes enter through nested bit
// masks and a per-group integer correction (see the operand-field note at
// digits_kernel).  x is represented to within 2^-25 of its group's largest
// magnitude.
//
// NF4 (f16 MFMA).  NF4 levels are not integers, so each level is split into
// two binary16 values L = L_hi + L_lo (22 significant bits) and each
// activation group, scaled by 2^-e_bg, into x = x_hi + x_lo.  A rows are
// (batch, hi/lo), B is the hi plane then the lo plane of the decoded levels,
// both v_mfma_f32_16x16x32_f16 products accumulate in f32 (f16 x f16 products
// are exact in f32), and a per-group epilogue applies scale * 2^e_bg.  Code
// bytes decode through a 256-entry LDS table giving both nibbles' hi and lo
// halves, already packed as MFMA operand dwords.
//
// MFMA operand layout (probed on gfx950 for i8, bf16 and f16): lane
// l = 16*q + i supplies row/column i of k-slot block q; D[i][j] =
// sum_q sum_b A_lane(16q+i)[b] * B_lane(16q+j)[b]; result register r of lane
// l holds D[4*(l/16) + r][l % 16].
//
// Private weight layout ("tiles"): 16 rows x K per tile, ordered so one
// 16-byte load per lane reads 1 KB of contiguous memory per wave:
//   INT8:    [tile][kstep s][lane][16 B]: lane (q,j) row j, k = 64s + 16q + b.
//   ternary: [tile][s/4][lane][4 x 4 B]: dword s%4 holds canonical code bytes
//            [16s + 4q, +4) of row j with bit 7 of every byte flipped (field 3
//            stored as (c + 2) mod 4); byte e, field f is k = 64s + 16q + 4e + f.
//   NF4:     [tile][s/4][lane][4 x 4 B] (s = 32-wide kstep): dword s%4 holds
//            canonical code bytes [16s + 4q, +4) of row j = k 32s + 8q + 0..7.
// Scales: [tile][group][16] as binary16 when every scale is exact in it,
// otherwise f32.
#include <type_traits>
#include <utility>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace mfh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// NF4 levels (kernels-simd/src/lib.rs:111-131 NF4_LEVELS), as literal constants:
// table builders index them with compile-time indices only, so building a
// table needs no memory access.
constexpr float kNf4LevelValues[16] = {
    -1.0f,        -0.6961928f,  -0.52507305f, -0.3949175f,
    -0.28444138f, -0.18477343f, -0.091050036f, 0.0f,
    0.0795803f,   0.1609302f,   0.2461123f,   0.33791524f,
    0.44070983f,  0.562617f,    0.72295684f,  1.0f,
};

// Per-format geometry:
//   kstep: k covered by one MFMA;  kpl: ksteps per 16-byte lane load;
//   lb: ksteps per loop block (integer-MFMA formats);  align: K padding of
//   the tile layout (integer-MFMA formats; NF4 pads to 128, align_of).
template <Format F> struct Geo;
template <> struct Geo<Format::Ternary> {
    static constexpr int kstep = 64, kpl = 4, lb = 4, align = 256;
};
template <> struct Geo<Format::Int8> {
    static constexpr int kstep = 64, kpl = 1, lb = 2, align = 128;
};
template <> struct Geo<Format::Nf4> {
    static constexpr int kstep = 32, kpl = 4;
};

__host__ __device__ inline uint32_t pad_to(uint32_t v, uint32_t a) { return (v + a - 1) / a * a; }

uint32_t align_of(Format f)
{
    return f == Format::Ternary ? 256 : 128;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float silu_mul(float gate, float up)
{
    float sigmoid = 1.0f / (1.0f + expf(-gate));
    return (gate * sigmoid) * up;
}

__device__ __forceinline__ float wave_sum_f(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        v += __shfl_xor(v, off, 64);
    return v;
}

// ---------------------------------------------------------------------------
// Prologue transforms (XForm).  AddRms needs the row's reciprocal RMS before
// any group can be formed: 1 / sqrt(sum(s^2) / k + eps), with s = a + b
// (normalization_rotary.rs:11-83 for the formula).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float add_value(const XForm &t, size_t i)
{
    float v = t.a[i];
    if (t.b)
        v = v + t.b[i];
    return v;
}

__device__ __forceinline__ float rms_reciprocal(float squares, uint32_t k, float epsilon)
{
    return 1.0f / sqrtf(squares / float(k) + epsilon);
}

// Sum `v` over the block (blockDim a multiple of 64), then the reciprocal
// RMS; `scratch` holds blockDim / 64 floats.  Every thread gets the value.
__device__ float block_reciprocal(float squares, uint32_t k, float epsilon, float *scratch)
{
    squares = wave_sum_f(squares);
    __syncthreads();
    if ((threadIdx.x & 63) == 0)
        scratch[threadIdx.x >> 6] = squares;
    __syncthreads();
    float total = 0.0f;
    for (uint32_t w = 0; w < blockDim.x / 64; ++w)
        total += scratch[w];
    return rms_reciprocal(total, k, epsilon);
}

// Element kk of activation row b after the transform of kind K, except
// that AddRms returns s = a + b unscaled and its norm weight in `weight`
// (the caller applies (s * reciprocal) * weight once the row's reciprocal is
// known).  `writer` lanes also store the side output of the element (each
// element has exactly one writer).
template <XKind K>
__device__ __forceinline__ float xform_load(const XForm &t, uint32_t b, uint32_t kk, uint32_t k,
                                            bool writer, float &weight)
{
    const size_t i = size_t(b) * k + kk;
    if constexpr (K == XKind::Plain) {
        return t.a[i];
    } else if constexpr (K == XKind::AddRms) {
        const float v = add_value(t, i);
        if (writer && t.side)
            t.side[i] = v;
        weight = t.w[kk];
        return v;
    } else {
        static_assert(K == XKind::Swiglu, "transform kinds: Plain, AddRms, Swiglu");
        return silu_mul(t.a[i], t.b[i]);
    }
}

// The same with the kind chosen at run time (the separate prologue kernels).
__device__ __forceinline__ float xform_load_any(const XForm &t, uint32_t b, uint32_t kk,
                                                uint32_t k, bool writer, float &weight)
{
    switch (t.kind) {
    case XKind::Plain: return xform_load<XKind::Plain>(t, b, kk, k, writer, weight);
    case XKind::AddRms: return xform_load<XKind::AddRms>(t, b, kk, k, writer, weight);
    default: return xform_load<XKind::Swiglu>(t, b, kk, k, writer, weight);
    }
}

// ---------------------------------------------------------------------------
// Activation prologues: one wave per (128-wide group, batch slot).  Slots at
// or beyond m are written as zeros so every fragment byte is defined.
// ---------------------------------------------------------------------------
struct GroupX {
    float x[2];
    int e;
    bool bad;
};

// This lane's two values of activation group g of batch slot b.
__device__ __forceinline__ void fetch_group(const XForm &t, uint32_t b, uint32_t g, uint32_t m,
                                            uint32_t k, float reciprocal, bool writer,
                                            float (&v)[2])
{
    const uint32_t lane = threadIdx.x & 63;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t kk = g * 128 + h * 64 + lane;
        float weight = 0.0f;
        v[h] = (b < m && kk < k) ? xform_load_any(t, b, kk, k, writer, weight) : 0.0f;
        if (t.kind == XKind::AddRms)
            v[h] = (v[h] * reciprocal) * weight;
    }
}

// The group's exponent (max |x| < 2^e) and non-finite flag, wave-wide.
__device__ __forceinline__ GroupX finish_group(const float (&raw)[2])
{
    GroupX r;
    r.bad = false;
    float mx = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float v = raw[h];
        if (!isfinite(v)) {
            r.bad = true;
            v = 0.0f;
        }
        r.x[h] = v;
        mx = fmaxf(mx, fabsf(v));
    }
    r.bad = __any(r.bad);
    mx = wave_max(mx);
    r.e = 0;
    if (mx > 0.0f)
        frexpf(mx, &r.e);  // mx = f * 2^e with f in [0.5, 1), so |x| < 2^e
    return r;
}

// Ternary operand fields.  Within a 64-wide kstep, k = 16q + 4e + f puts
// weight k in bits [2f, 2f+2) of code byte e of lane block q (f = k % 4).
// The tile layout stores field 3 as (c + 2) mod 4, and the B operand's four
// dwords are w, w & 0xFCFCFCFC, w & 0xF0F0F0F0, w & 0xC0C0C0C0: as signed
// bytes, dword d holds sum_{f >= d} 4^f c'_f with c'_f = c_f for f < 3 and
// c_3 - 2 for field 3.  The matching A dword d holds
// y_d = u_d - u_{d-1}, where u_f = round(v_f / 4^f), so the MFMA sum
// telescopes to sum_f 4^f c'_f u_f.  The prologue's per-group correction
// corr = sum_{f<3} 4^f u_f - 64 sum_{f=3} u_f turns that into
// sum_k (c_k - 1) * 4^f u_k, i.e. sum_k (c_k - 1) v_k to within 2^5 units of
// the 2^30-scaled group maximum per weight.
//
// emit_digits: one wave writes the fragment bytes of activation group g of
// batch slot b; kstep indices are relative to `s0`.  Lane 0 stores the
// group factor 2^(e - 30) (NaN for a non-finite group) and, for ternary, the
// correction.
//
// Fragment layout: kstep s, fragment b / 4, lane block q, row r at
// ((s * nfrag + b / 4) * 4 + q) * rp + r (16 bytes each).  rp = 16 is the
// MFMA lane order; the in-kernel prologue keeps only the live rows
// (rp = 4 * m, nfrag = 1).
template <Format F>
__device__ __forceinline__ void emit_group(const GroupX &gx, uint32_t b, uint32_t g,
                                           uint32_t nfrag, uint32_t rp, uint32_t s0,
                                           int8_t *afrag, float *xf_out, int2 *corr_out)
{
    const uint32_t lane = threadIdx.x & 63;
    if (lane == 0)
        *xf_out = gx.bad ? __builtin_nanf("") : ldexpf(1.0f, gx.e - 30);
    long long corr_sum = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t kk = g * 128 + h * 64 + lane;
        int val = gx.bad ? 0 : int(rintf(ldexpf(gx.x[h], 30 - gx.e)));
        if constexpr (F == Format::Ternary) {
            const int f = int(lane & 3);
            const int u = f == 0 ? val : (val + (1 << (2 * f - 1))) >> (2 * f);
            const int u_prev = __shfl_up(u, 1, 64);
            val = f == 0 ? u : u - u_prev;
            corr_sum += f < 3 ? (static_cast<long long>(u) << (2 * f))
                              : -(static_cast<long long>(u) << 6);
        }
        // Offset form: bytes of val + 0x808080 are the low digits plus 128.
        const int vp = val + 0x808080;
        int d[4];
        d[0] = vp >> 24;
        d[1] = int(int8_t(((vp >> 16) & 255) ^ 0x80));
        d[2] = int(int8_t(((vp >> 8) & 255) ^ 0x80));
        d[3] = int(int8_t((vp & 255) ^ 0x80));
        const uint32_t s = kk / 64 - s0, r = kk % 64;
        const uint32_t q = r / 16, c = r % 16;
        const uint32_t byte = (F == Format::Ternary) ? (4 * (c & 3) + (c >> 2)) : c;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t row = 4 * (b % 4) + i;
            afrag[(((size_t(s) * nfrag + b / 4) * 4 + q) * rp + row) * 16 + byte] = int8_t(d[i]);
        }
    }
    if constexpr (F == Format::Ternary) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            corr_sum += __shfl_xor(corr_sum, off, 64);
        if (lane == 0) {
            // Split as hi * 2^16 + lo to match the epilogue's digit pairs.
            const long long lo = ((corr_sum + 32768) & 65535) - 32768;
            *corr_out = int2{int((corr_sum - lo) >> 16), int(lo)};
        }
    }
}

// The separate prologue kernels: block (x, b) of kPrologueWaves waves forms
// groups [x * kPrologueWaves, +kPrologueWaves) of batch slot b, one wave per
// group; slots at or beyond m get zero fragments.  For AddRms the block
// first reduces the row's squares together.  Every wave writes the side
// outputs of its own elements.
constexpr uint32_t kPrologueWaves = 4;

__device__ __forceinline__ GroupX prologue_group(const XForm &t, uint32_t b, uint32_t g,
                                                 uint32_t m, uint32_t k, float reciprocal)
{
    float raw[2];
    fetch_group(t, b, g, m, k, reciprocal, true, raw);
    return finish_group(raw);
}

__device__ __forceinline__ float prologue_reciprocal(const XForm &t, uint32_t b, uint32_t m,
                                                     uint32_t k, float *scratch)
{
    if (t.kind != XKind::AddRms || b >= m)  // uniform over the block
        return 0.0f;
    float squares = 0.0f;
#pragma unroll 8
    for (uint32_t kk = threadIdx.x; kk < k; kk += blockDim.x) {
        const float v = add_value(t, size_t(b) * k + kk);
        squares += v * v;
    }
    return block_reciprocal(squares, k, t.epsilon, scratch);
}

template <Format F>
__global__ __launch_bounds__(64 * kPrologueWaves) void digits_kernel(XForm t, uint32_t m,
                                                                     uint32_t k, uint32_t groups,
                                                                     uint32_t nfrag,
                                                                     int8_t *afrag, float *xf,
                                                                     int2 *corr, float *zero,
                                                                     uint32_t zero_count)
{
    __shared__ float scratch[kPrologueWaves];
    const uint32_t b = blockIdx.y;
    const uint32_t g = blockIdx.x * kPrologueWaves + (threadIdx.x >> 6);
    // The output a K-split GEMV accumulates into starts at zero.
    const uint32_t stride = gridDim.x * gridDim.y * blockDim.x;
    for (uint32_t i = (blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x;
         i < zero_count; i += stride)
        zero[i] = 0.0f;
    const float reciprocal = prologue_reciprocal(t, b, m, k, scratch);
    if (g >= groups)
        return;
    emit_group<F>(prologue_group(t, b, g, m, k, reciprocal), b, g, nfrag, 16, 0, afrag,
                  xf + b * groups + g, corr + b * groups + g);
}

// The in-kernel prologue (m <= 2).  The block's waves take the 128-groups
// round robin (wave w: groups w, w + W, ...; at most held_groups(K) each)
// and load each batch row's values once, into registers.  AddRms reduces the
// row's squares across the block from those registers, then scales them.
// Each group is then handed to `emit(b, g, group)`; the fragments land in
// one block-wide LDS array that every wave reads for its own K range.  The
// kind is a template parameter so each instantiation holds only its own
// loads.
__host__ __device__ constexpr uint32_t held_groups(XKind kind)
{
    (void)kind;
    return 8;
}
// Each wave forms its groups one after another, so a share above this many
// costs more latency than the separate prologue kernel's launch.
constexpr uint32_t kFusedGroupsPerWave = 2;

template <XKind K, typename Emit>
__device__ __forceinline__ void block_prologue(const XForm &t, uint32_t m, uint32_t k,
                                               uint32_t groups, float *scratch, Emit emit)
{
    constexpr uint32_t kHeld = held_groups(K);
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const bool writer = blockIdx.x == 0;
    for (uint32_t b = 0; b < m; ++b) {
        float v[kHeld][2], w[kHeld][2];
#pragma unroll
        for (uint32_t i = 0; i < kHeld; ++i) {
            const uint32_t g = wave + i * waves;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t kk = g * 128 + h * 64 + lane;
                w[i][h] = 0.0f;
                v[i][h] =
                    (g < groups && kk < k) ? xform_load<K>(t, b, kk, k, writer, w[i][h]) : 0.0f;
            }
        }
        if constexpr (K == XKind::AddRms) {
            float squares = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < kHeld; ++i)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    squares += v[i][h] * v[i][h];
            const float reciprocal = block_reciprocal(squares, k, t.epsilon, scratch);
#pragma unroll
            for (uint32_t i = 0; i < kHeld; ++i)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    v[i][h] = (v[i][h] * reciprocal) * w[i][h];
        }
        // One emission body, not unrolled: group i is always in v[0], and
        // the held values shift down a slot per iteration (static indices
        // keep them in registers).
#pragma nounroll
        for (uint32_t i = 0; i < kHeld; ++i) {
            const uint32_t g = wave + i * waves;
            if (g >= groups)  // wave-uniform
                break;
            emit(b, g, finish_group(v[0]));
#pragma unroll
            for (uint32_t j = 0; j + 1 < kHeld; ++j) {
                v[j][0] = v[j + 1][0];
                v[j][1] = v[j + 1][1];
            }
        }
    }
}

__global__ __launch_bounds__(64 * kPrologueWaves) void halves_kernel(XForm t, uint32_t m,
                                                                     uint32_t k, uint32_t groups,
                                                                     _Float16 *afrag, float *xf,
                                                                     float *zero,
                                                                     uint32_t zero_count)
{
    __shared__ float scratch[kPrologueWaves];
    const uint32_t b = blockIdx.y;
    const uint32_t g = blockIdx.x * kPrologueWaves + (threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63;
    // The output a K-split GEMV accumulates into starts at zero.
    const uint32_t stride = gridDim.x * gridDim.y * blockDim.x;
    for (uint32_t i = (blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x;
         i < zero_count; i += stride)
        zero[i] = 0.0f;
    const float reciprocal = prologue_reciprocal(t, b, m, k, scratch);
    if (g >= groups)
        return;
    const GroupX gx = prologue_group(t, b, g, m, k, reciprocal);
    if (lane == 0)
        xf[b * groups + g] = gx.bad ? __builtin_nanf("") : ldexpf(1.0f, gx.e);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t kk = g * 128 + h * 64 + lane;
        const float v = gx.bad ? 0.0f : ldexpf(gx.x[h], -gx.e);
        const _Float16 hi = _Float16(v);
        const _Float16 lo = _Float16(v - float(hi));
        const uint32_t s = kk / 32, r = kk % 32;
        const uint32_t q = r / 8, pos = r % 8;
        afrag[(size_t(s) * 64 + 16 * q + 2 * b) * 8 + pos] = hi;
        afrag[(size_t(s) * 64 + 16 * q + 2 * b + 1) * 8 + pos] = lo;
    }
}

// NF4 fragment emission of group g of batch row b into the block-wide
// fragment array (rp = 2 * m rows per lane block: hi and lo of each row)
// and its factor 2^e into fxf[b * groups + g].
__device__ __forceinline__ void emit_halves(const GroupX &gx, uint32_t b, uint32_t g,
                                            uint32_t rp, uint32_t groups, _Float16 *frag,
                                            float *fxf)
{
    const uint32_t lane = threadIdx.x & 63;
    if (lane == 0)
        fxf[b * groups + g] = gx.bad ? __builtin_nanf("") : ldexpf(1.0f, gx.e);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t kk = g * 128 + h * 64 + lane;
        const float v = gx.bad ? 0.0f : ldexpf(gx.x[h], -gx.e);
        const _Float16 hi = _Float16(v);
        const _Float16 lo = _Float16(v - float(hi));
        const uint32_t s = kk / 32, r = kk % 32;
        const uint32_t q = r / 8, pos = r % 8;
        frag[((size_t(s) * 4 + q) * rp + 2 * b) * 8 + pos] = hi;
        frag[((size_t(s) * 4 + q) * rp + 2 * b + 1) * 8 + pos] = lo;
    }
}

// Activation fragment sources of the GEMV main loops: at(s, f, nf) is the
// 16-byte operand of this lane for kstep s (relative to the wave's first)
// and fragment f.
template <typename V>
struct GlobalFrag {
    const V *p;  // already offset by the wave's first kstep and the lane
    __device__ __forceinline__ V at(uint32_t s, int f, int nf) const
    {
        return p[(size_t(s) * nf + f) * 64];
    }
};
template <typename V>
struct LdsFrag {
    const V *p;       // block fragments + (first kstep * 4 + q) * rp + j
    uint32_t stride;  // 4 * rp
    bool live;        // j < rp: lanes of dead rows read zeros
    __device__ __forceinline__ V at(uint32_t s, int, int) const
    {
        return live ? p[size_t(s) * stride] : V{};
    }
};

template <bool HALF>
struct ScaleT;
template <> struct ScaleT<true> { typedef __half type; };
template <> struct ScaleT<false> { typedef float type; };

template <bool HALF>
__device__ __forceinline__ float to_f32(typename ScaleT<HALF>::type v)
{
    if constexpr (HALF)
        return __half2float(v);
    else
        return v;
}

struct MfmaArgs {
    const void *afrag;
    const float *xf;
    const int2 *corr;
    const uint8_t *tiles[2];
    const void *scales[2];
    float *out[2];
    XForm xform;  // activation source of the prologue
    uint32_t m, n, k, k_pad;
    uint32_t ksteps_per_wave;
    // K split: kparts blocks per tile group, part p = blockIdx.x / part_blocks
    // taking K steps [p, p + 1) * waves * ksteps_per_wave and adding its
    // sums atomically into the zeroed output (Single epilogue only).
    uint32_t kparts, part_blocks;
    // Segmented launch (one stream, T = 1): blocks [seg_first[i], next) run
    // weight stream i of seg_n[i] rows into seg_out[i]; 0 segments = off.
    uint32_t segments;
    uint32_t seg_first[kMaxSegments];
    const uint8_t *seg_tiles[kMaxSegments];
    const void *seg_scales[kMaxSegments];
    float *seg_out[kMaxSegments];
    uint32_t seg_n[kMaxSegments];
};

// The weight streams, output rows and first tile of this block.
struct Target {
    uint32_t tile0, n;
    const uint8_t *tiles[2];
    const void *scales[2];
    float *out[2];
};

template <int T>
__device__ __forceinline__ Target target_of(const MfmaArgs &a)
{
    Target r;
    uint32_t block = a.kparts > 1 ? blockIdx.x % a.part_blocks : blockIdx.x;
    r.n = a.n;
    for (int st = 0; st < 2; ++st) {
        r.tiles[st] = a.tiles[st];
        r.scales[st] = a.scales[st];
        r.out[st] = a.out[st];
    }
    if (a.segments) {
        uint32_t sg = 0;
        while (sg + 1 < a.segments && block >= a.seg_first[sg + 1])
            ++sg;
        block -= a.seg_first[sg];
        r.tiles[0] = a.seg_tiles[sg];
        r.scales[0] = a.seg_scales[sg];
        r.out[0] = a.seg_out[sg];
        r.n = a.seg_n[sg];
    }
    r.tile0 = block * T;
    return r;
}

// Fixed-order sum of the wave partials through LDS, then the epilogue.
// vals[idx] per lane; idx = (st * T + t) * NB + batch-slot-of-lane.
template <int S, int T, int NB, Epilogue E>
__device__ __forceinline__ void reduce_and_store(uint32_t m, const Target &tg,
                                                 float (&vals)[S][T][NB],
                                                 const uint32_t (&batch)[NB], uint32_t j,
                                                 bool accumulate = false)
{
    const uint32_t tile0 = tg.tile0;
    extern __shared__ float red[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    constexpr int V = S * T * NB;
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                red[(wave * V + (st * T + t) * NB + nb) * 64 + lane] = vals[st][t][nb];
    __syncthreads();
    for (int idx = wave; idx < T * NB; idx += waves) {
        const int t = idx / NB, nb = idx % NB;
        float v[S];
#pragma unroll
        for (int st = 0; st < S; ++st) {
            float sum = 0.0f;
            for (int w2 = 0; w2 < waves; ++w2)
                sum += red[(w2 * V + (st * T + t) * NB + nb) * 64 + lane];
            v[st] = sum;
        }
        const uint32_t b = batch[nb];
        const uint32_t row = (tile0 + t) * 16 + j;
        if (b < m && row < tg.n) {
            const size_t o = size_t(b) * tg.n + row;
            if constexpr (E == Epilogue::Single) {
                // K-split partials: two addends onto zero, so the sum does
                // not depend on their order.
                if (accumulate)
                    atomicAdd(&tg.out[0][o], v[0]);
                else
                    tg.out[0][o] = v[0];
            } else if constexpr (E == Epilogue::Pair) {
                tg.out[0][o] = v[0];
                tg.out[1][o] = v[S - 1];
            } else {
                tg.out[0][o] = silu_mul(v[0], v[S - 1]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Integer-MFMA GEMV (ternary, INT8).  A block owns T consecutive tiles of each
// of S streams; its W waves split K.  Loop blocks of LB ksteps are double
// buffered in registers: the next block's weights and activation fragments
// are in flight while the current one is computed.
// ---------------------------------------------------------------------------
template <Format F, int T, int S, int NF, bool HALF, int LBO = Geo<F>::lb>
struct I8Block {
    // LBO: ksteps per loop block (Geo<F>::lb; 2 for the ternary 128-k
    // pieces of wide_rows_kernel, whose own weight registers leave w unused).
    static constexpr int LB = LBO;
    static constexpr int LOADS = LB / Geo<F>::kpl > 0 ? LB / Geo<F>::kpl : 1;
    static constexpr int GPB = LB / 2;  // 128-groups per loop block
    using ST = typename ScaleT<HALF>::type;
    v4u w[S][T][LOADS];
    ST sc[S][T][GPB];    // weight scales of the block's groups (this lane's row)
    v4i af[LB][NF];
    float xf[GPB][NF];   // activation group factors
    int2 cv[GPB][NF];    // ternary group corrections
};

// Weights and their group scales of loop block `index`.
template <Format F, int T, int S, int NF, bool HALF>
__device__ __forceinline__ void i8_load_w(I8Block<F, T, S, NF, HALF> &blk,
                                          const v4u *const (&wp)[S][T],
                                          const typename ScaleT<HALF>::type *const (&sp)[S][T],
                                          uint32_t index)
{
    using B = I8Block<F, T, S, NF, HALF>;
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int t = 0; t < T; ++t) {
#pragma unroll
            for (int l = 0; l < B::LOADS; ++l) {
                // INT8 weights stream once per launch: non-temporal loads
                // measured about 10 % faster on the 65536-row head and 2-4 %
                // on 8192 x 2048 and 2048 x 8192 (B = 1 and 4), the same on
                // the smaller shapes; ternary and NF4 measured the same or
                // slower with them.
                if constexpr (F == Format::Int8)
                    blk.w[st][t][l] =
                        __builtin_nontemporal_load(&wp[st][t][(index * B::LOADS + l) * 64]);
                else
                    blk.w[st][t][l] = wp[st][t][(index * B::LOADS + l) * 64];
            }
#pragma unroll
            for (int gg = 0; gg < B::GPB; ++gg)
                blk.sc[st][t][gg] = sp[st][t][(index * B::GPB + gg) * 16];
        }
}

// Activation fragments and group constants of loop block `index`.
template <Format F, int T, int S, int NF, bool HALF, typename AP>
__device__ __forceinline__ void i8_load_a(I8Block<F, T, S, NF, HALF> &blk, const AP &ap,
                                          const float *const (&xp)[NF],
                                          const int2 *const (&cp)[NF], uint32_t index)
{
    using B = I8Block<F, T, S, NF, HALF>;
#pragma unroll
    for (int ks = 0; ks < B::LB; ++ks)
#pragma unroll
        for (int f = 0; f < NF; ++f)
            blk.af[ks][f] = ap.at(index * B::LB + ks, f, NF);
#pragma unroll
    for (int gg = 0; gg < B::GPB; ++gg)
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            blk.xf[gg][f] = xp[f][index * B::GPB + gg];
            if constexpr (F == Format::Ternary)
                blk.cv[gg][f] = cp[f][index * B::GPB + gg];
            else
                blk.cv[gg][f] = int2{0, 0};
        }
}

template <Format F, int T, int S, int NF, bool HALF, typename AP>
__device__ __forceinline__ void i8_load(I8Block<F, T, S, NF, HALF> &blk,
                                        const v4u *const (&wp)[S][T],
                                        const typename ScaleT<HALF>::type *const (&sp)[S][T],
                                        const AP &ap, const float *const (&xp)[NF],
                                        const int2 *const (&cp)[NF], uint32_t index)
{
    i8_load_w(blk, wp, sp, index);
    i8_load_a(blk, ap, xp, cp, index);
}

// One loop block: everything it reads was loaded with it (i8_load), so the
// next block's loads stay in flight behind these MFMAs.
template <Format F, int T, int S, int NF, bool HALF>
__device__ __forceinline__ void i8_compute(const I8Block<F, T, S, NF, HALF> &blk,
                                           float (&accf)[S][T][NF])
{
    using B = I8Block<F, T, S, NF, HALF>;
#pragma unroll
    for (int gg = 0; gg < B::GPB; ++gg) {
        v4i acci[S][T][NF];
#pragma unroll
        for (int st = 0; st < S; ++st)
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int f = 0; f < NF; ++f)
                    acci[st][t][f] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int ks = gg * 2 + kk;
#pragma unroll
            for (int st = 0; st < S; ++st)
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    v4i bw;
                    if constexpr (F == Format::Ternary) {
                        // Nested field masks (see the operand-field note above).
                        const unsigned word = blk.w[st][t][0][ks];
                        bw = v4i{int(word), int(word & 0xFCFCFCFCu), int(word & 0xF0F0F0F0u),
                                 int(word & 0xC0C0C0C0u)};
                    } else {
                        const v4u v = blk.w[st][t][ks];
                        bw = v4i{int(v.x), int(v.y), int(v.z), int(v.w)};
                    }
#pragma unroll
                    for (int f = 0; f < NF; ++f)
                        acci[st][t][f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            blk.af[ks][f], bw, acci[st][t][f], 0, 0, 0);
                }
        }
#pragma unroll
        for (int st = 0; st < S; ++st)
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int f = 0; f < NF; ++f) {
                    const v4i d = acci[st][t][f];
                    const int2 cv = blk.cv[gg][f];
                    // |d.x| < 2^21, so the pairs combine exactly in int32.
                    const int hi = (d.x << 8) + d.y - cv.x;
                    const int lo = (d.z << 8) + d.w - cv.y;
                    const float gsum = float(hi) * 65536.0f + float(lo);
                    accf[st][t][f] +=
                        gsum * (to_f32<HALF>(blk.sc[st][t][gg]) * blk.xf[gg][f]);
                }
    }
}

// ---------------------------------------------------------------------------
// Register prologue (m <= 8, activations as stored).  Each wave forms the
// digit fragments of its own loop blocks, one block ahead of the MFMAs,
// from the raw activations: no LDS, no barrier, no separate kernel.
// Lane 16q + 4b + p loads x[4f + b][64s + 16q + 4p + t] (t = 0..3) of every
// kstep s for each fragment f, and it supplies digit row p of batch 4f + b
// in fragment f's MFMA A operand.
// Per group, the exponent and the ternary correction reduce over the 16
// lanes that hold the batch (lane quad, lane blocks); the quad then shares
// its 16 offset values and each lane packs digit p of all of them.  The
// arithmetic is emit_group's value for value, so the fragments, factors and
// corrections are the bytes digits_kernel would write.
// ---------------------------------------------------------------------------
constexpr int kRegPro = 16;
// Largest K range per wave (in 64-wide ksteps) of the register prologue of
// the add + RMS norm, which holds the whole range while the row's squares
// reduce.
constexpr int kRegNormSteps = 4;
// Largest grid for the two-fragment (m > 4) ternary register prologue.
constexpr uint32_t kRegPairBlocks = 320;

template <int LB>
struct RegX {
    v4f v[LB];
};

// Quad lane exchanges (DPP quad_perm): the value of lane l ^ 1, l ^ 2.
__device__ __forceinline__ unsigned quad_xor1(unsigned v)
{
    return unsigned(__builtin_amdgcn_mov_dpp(int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ unsigned quad_xor2(unsigned v)
{
    return unsigned(__builtin_amdgcn_mov_dpp(int(v), 0x4E, 0xF, 0xF, false));
}

// 4 x 4 byte transpose: r[i] byte j = w[j] byte (REV ? 3 - i : i).
// v_perm_b32 selector bytes 0-3 pick bytes of its second operand, 4-7 of
// its first.
template <bool REV>
__device__ __forceinline__ void byte_transpose(const unsigned (&w)[4], unsigned (&r)[4])
{
    // Pairs of rows: (w0.b_i, w1.b_i) for two i per dword.
    const unsigned sa = REV ? 0x06020703u : 0x05010400u;  // i = 0, 1 (REV: bytes 3, 2)
    const unsigned sb = REV ? 0x04000501u : 0x07030602u;  // i = 2, 3 (REV: bytes 1, 0)
    const unsigned a01 = __builtin_amdgcn_perm(w[1], w[0], sa);
    const unsigned b01 = __builtin_amdgcn_perm(w[1], w[0], sb);
    const unsigned a23 = __builtin_amdgcn_perm(w[3], w[2], sa);
    const unsigned b23 = __builtin_amdgcn_perm(w[3], w[2], sb);
    r[0] = __builtin_amdgcn_perm(a23, a01, 0x05040100u);
    r[1] = __builtin_amdgcn_perm(a23, a01, 0x07060302u);
    r[2] = __builtin_amdgcn_perm(b23, b01, 0x05040100u);
    r[3] = __builtin_amdgcn_perm(b23, b01, 0x07060302u);
}

// 4 x 4 transpose across a lane quad: lane p ends with r[P] = register p of
// quad lane P (two butterfly stages).
__device__ __forceinline__ void quad_transpose(unsigned (&r)[4], uint32_t p)
{
    unsigned m[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned other = quad_xor1(r[i ^ 1]);
        m[i] = (p & 1) == unsigned(i & 1) ? r[i] : other;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned other = quad_xor2(m[i ^ 2]);
        r[i] = (p & 2) == unsigned(i & 2) ? m[i] : other;
    }
}

// Loop block `index` of this lane's activation values (zeros past k or for
// batch slots at or beyond m).
template <int LB>
__device__ __forceinline__ void reg_load(RegX<LB> &rx, const float *xrow, bool live, uint32_t k,
                                         uint32_t s0, uint32_t index)
{
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t off = 16 * (lane >> 4) + 4 * (lane & 3);
#pragma unroll
    for (int kk = 0; kk < LB; ++kk) {
        const uint32_t kx = 64 * (s0 + index * LB + kk) + off;
        rx.v[kk] = live && kx < k ? *reinterpret_cast<const v4f *>(xrow + kx)
                                  : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
}

// As reg_load, for the streaming kernels: every load is issued (a dead row
// reads clamped addresses of row 0 and is zeroed afterwards), because a branch
// around a load can make the compiler wait for it before the weight loads that
// follow.
template <int LB>
__device__ __forceinline__ void reg_load_issued(RegX<LB> &rx, const float *xrow, bool live,
                                                uint32_t k, uint32_t index, uint32_t off,
                                                uint32_t kstep)
{
#pragma unroll
    for (int kk = 0; kk < LB; ++kk) {
        const uint32_t kx = kstep * (index * LB + kk) + off;
        const v4f v = *reinterpret_cast<const v4f *>(xrow + (kx < k ? kx : k - 4));
        rx.v[kk] = live && kx < k ? v : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
}

// Fragment f (batch rows 4f..4f+3) of a loop block from this lane's values.
template <Format F, int T, int S, int NF, bool HALF, int LBO>
__device__ __forceinline__ void reg_digits(const RegX<LBO> &rx,
                                           I8Block<F, T, S, NF, HALF, LBO> &blk, int f)
{
    using B = I8Block<F, T, S, NF, HALF, LBO>;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t p = lane & 3, q = lane >> 4;
    const unsigned flip = p ? 0x80808080u : 0u;
#pragma unroll
    for (int gg = 0; gg < B::GPB; ++gg) {
        // Largest magnitude as bits: |x| orders like its bit pattern, and a
        // pattern at or above infinity's marks a non-finite group.
        unsigned mb = 0;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int t = 0; t < 4; ++t)
                mb = max(mb, __float_as_uint(rx.v[2 * gg + kk][t]) & 0x7FFFFFFFu);
        mb = max(mb, quad_xor1(mb));
        mb = max(mb, quad_xor2(mb));
        mb = max(mb, unsigned(__shfl_xor(int(mb), 16, 64)));
        mb = max(mb, unsigned(__shfl_xor(int(mb), 32, 64)));
        const bool bad = mb >= 0x7F800000u;
        int e = 0;
        if (!bad && mb)
            frexpf(__uint_as_float(mb), &e);  // |x| < 2^e
        const float factor = bad ? __builtin_nanf("") : ldexpf(1.0f, e - 30);
        long long corr = 0;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int ks = 2 * gg + kk;
            unsigned vp[4];
            int u_prev = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                int val = bad ? 0 : int(rintf(ldexpf(rx.v[ks][t], 30 - e)));
                if constexpr (F == Format::Ternary) {
                    // Field t of the nested masks (see the operand-field note).
                    const int u = t == 0 ? val : (val + (1 << (2 * t - 1))) >> (2 * t);
                    val = t == 0 ? u : u - u_prev;
                    u_prev = u;
                    corr += t < 3 ? (static_cast<long long>(u) << (2 * t))
                                  : -(static_cast<long long>(u) << 6);
                }
                vp[t] = unsigned(val + 0x808080);
            }
            // d[D] byte t = digit D of value t (digit D is byte 3 - D of the
            // offset form); after the quad transpose d[P] byte t = digit p of
            // quad lane P's value t, i.e. of lane-block value c = 4P + t.
            unsigned d[4];
            byte_transpose<true>(vp, d);
            quad_transpose(d, p);
            unsigned w[4];
            if constexpr (F == Format::Ternary) {
                byte_transpose<false>(d, w);  // ternary byte 4t + P: dword t, byte P
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    w[i] = d[i];             // INT8 byte c = 4P + t: dword P, byte t
            }
            blk.af[ks][f] = v4i{int(w[0] ^ flip), int(w[1] ^ flip), int(w[2] ^ flip),
                                int(w[3] ^ flip)};
        }
        // Lane (q, j) applies batch q's constants: lane 4q holds them.
        blk.xf[gg][f] = __shfl(factor, int(4 * q), 64);
        if constexpr (F == Format::Ternary) {
            corr += static_cast<long long>(quad_xor1(unsigned(corr))) |
                    (static_cast<long long>(quad_xor1(unsigned(corr >> 32))) << 32);
            corr += static_cast<long long>(quad_xor2(unsigned(corr))) |
                    (static_cast<long long>(quad_xor2(unsigned(corr >> 32))) << 32);
            corr += __shfl_xor(corr, 16, 64);
            corr += __shfl_xor(corr, 32, 64);
            // Split as hi * 2^16 + lo to match the epilogue's digit pairs.
            const long long lo = ((corr + 32768) & 65535) - 32768;
            const int hi = int((corr - lo) >> 16);
            blk.cv[gg][f] = int2{__shfl(hi, int(4 * q), 64), __shfl(int(lo), int(4 * q), 64)};
        } else {
            blk.cv[gg][f] = int2{0, 0};
        }
    }
}

// Bytes of dynamic LDS past the reduction area that the in-kernel prologue
// uses: the live rows (4 per batch row) of the digit fragments of all of K,
// then 4 slots of group factors and corrections.
__host__ __device__ constexpr size_t fused_bytes(uint32_t k_pad, uint32_t m)
{
    return size_t(k_pad) * 4 * m + size_t(4) * (k_pad / 128) * 12;
}
// The NF4 kernel's: hi/lo rows (2 per batch row) per 32-wide kstep, then 8
// slots of group factors.
__host__ __device__ constexpr size_t fused_bytes_nf4(uint32_t k_pad, uint32_t m)
{
    return size_t(k_pad) * 4 * m + size_t(8) * (k_pad / 128) * 4;
}

// At most 8 waves per block: two per SIMD leaves 256 VGPRs per wave for the
// double-buffered loop blocks.  One-tile, one-stream, one-fragment kernels
// with the separate or register prologue (at most 110 VGPRs) also run 16
// waves, for the small-N plan (kDeepWaves).  PRO < 0: digits_kernel wrote
// the activation fragments to global scratch.  PRO == kRegPro(+AddRms):
// each lane forms its own fragments in registers.  Otherwise the block first
// forms them in LDS with the in-kernel prologue of transform XKind(PRO)
// (block_prologue) while each wave's first weights are in flight.
template <Format F, int T, int S, int NF, bool HALF, Epilogue E, int PRO>
__global__ __launch_bounds__(T == 1 && S == 1 && NF == 1 && (PRO < 0 || PRO == kRegPro) ? 1024
                                                                                          : 512)
void gemv_i8_kernel(MfmaArgs a)
{
    using B = I8Block<F, T, S, NF, HALF>;
    using ST = typename ScaleT<HALF>::type;
    constexpr int KPL = Geo<F>::kpl;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t q = lane >> 4, j = lane & 15;
    const Target tg = target_of<T>(a);
    const uint32_t tile0 = tg.tile0;
    const uint32_t groups = a.k_pad / 128;
    const uint32_t part = a.kparts > 1 ? blockIdx.x / a.part_blocks : 0;
    const uint32_t s_begin = (part * (blockDim.x >> 6) + wave) * a.ksteps_per_wave;
    const uint32_t nblk = a.ksteps_per_wave / B::LB;
    const uint32_t g_begin = s_begin / 2;
    const size_t tile_vecs = size_t(a.k_pad) / 64 / KPL * 64;

    const v4u *wp[S][T];
    const ST *sp[S][T];
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            wp[st][t] = reinterpret_cast<const v4u *>(tg.tiles[st]) + (tile0 + t) * tile_vecs +
                        (s_begin / KPL) * 64 + lane;
            sp[st][t] = reinterpret_cast<const ST *>(tg.scales[st]) +
                        (size_t(tile0 + t) * groups + g_begin) * 16 + j;
        }
    const GlobalFrag<v4i> ap{reinterpret_cast<const v4i *>(a.afrag) + size_t(s_begin) * NF * 64 +
                             lane};
    const float *xp[NF];
    const int2 *cp[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        xp[f] = a.xf + (4 * f + q) * groups + g_begin;
        cp[f] = a.corr + (4 * f + q) * groups + g_begin;
    }

    float accf[S][T][NF];
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int f = 0; f < NF; ++f)
                accf[st][t][f] = 0.0f;

    B buf0, buf1;
    auto main_loop = [&](auto afp) {
        for (uint32_t i = 0; i < nblk; i += 2) {
            if (i + 1 < nblk)
                i8_load(buf1, wp, sp, afp, xp, cp, i + 1);
            i8_compute(buf0, accf);
            if (i + 1 < nblk) {
                if (i + 2 < nblk)
                    i8_load(buf0, wp, sp, afp, xp, cp, i + 2);
                i8_compute(buf1, accf);
            }
        }
    };
    if constexpr (PRO == kRegPro) {
        // Activation loads go out ahead of the same block's weights, so a
        // block's digits can form while its weights are still arriving.
        const uint32_t b = (lane >> 2) & 3;
        const float *xrow[NF];
        bool live[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            live[f] = 4 * f + b < a.m;
            xrow[f] = a.xform.a + size_t(live[f] ? 4 * f + b : 0) * a.k;
        }
        RegX<B::LB> rx0[NF], rx1[NF];
        auto load_x = [&](RegX<B::LB>(&rx)[NF], uint32_t index) {
#pragma unroll
            for (int f = 0; f < NF; ++f)
                reg_load(rx[f], xrow[f], live[f], a.k, s_begin, index);
        };
        auto digits = [&](const RegX<B::LB>(&rx)[NF], B &blk) {
#pragma unroll
            for (int f = 0; f < NF; ++f)
                reg_digits(rx[f], blk, f);
        };
        if (nblk > 0) {
            load_x(rx0, 0);
            i8_load_w(buf0, wp, sp, 0);
        }
        for (uint32_t i = 0; i < nblk; i += 2) {
            if (i + 1 < nblk) {
                load_x(rx1, i + 1);
                i8_load_w(buf1, wp, sp, i + 1);
            }
            digits(rx0, buf0);
            i8_compute(buf0, accf);
            if (i + 1 < nblk) {
                if (i + 2 < nblk) {
                    load_x(rx0, i + 2);
                    i8_load_w(buf0, wp, sp, i + 2);
                }
                digits(rx1, buf1);
                i8_compute(buf1, accf);
            }
        }
    } else if constexpr (PRO == kRegPro + int(XKind::AddRms)) {
        static_assert(NF == 1, "the register norm prologue serves m <= 4");
        // s = a + b over the wave's whole K range (at most kRegNormSteps
        // ksteps), every wave's squares summed per batch row, then
        // x = (s * reciprocal) * weight as in the separate prologue.
        constexpr int KS = kRegNormSteps;
        constexpr int NB = KS / B::LB;  // loop blocks held
        __shared__ float rms_part[8][4];  // [wave][batch slot]
        const XForm &t = a.xform;
        const uint32_t b = (lane >> 2) & 3;
        const bool live = b < a.m;
        const size_t row = size_t(live ? b : 0) * a.k;
        const uint32_t steps = a.ksteps_per_wave;
        const uint32_t off = 16 * (lane >> 4) + 4 * (lane & 3);
        auto at = [&](int ks) { return 64 * (s_begin + ks) + off; };
        v4f xs[KS], ys[KS], ws[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const bool in = uint32_t(ks) < steps && at(ks) < a.k;
            xs[ks] = ys[ks] = ws[ks] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if (in && live)
                xs[ks] = *reinterpret_cast<const v4f *>(t.a + row + at(ks));
            if (in && live && t.b)
                ys[ks] = *reinterpret_cast<const v4f *>(t.b + row + at(ks));
            if (in)
                ws[ks] = *reinterpret_cast<const v4f *>(t.w + at(ks));
        }
        if (nblk > 0)
            i8_load_w(buf0, wp, sp, 0);
        if (nblk > 1)
            i8_load_w(buf1, wp, sp, 1);
        float squares = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (t.b)
                xs[ks] = xs[ks] + ys[ks];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                squares += xs[ks][e] * xs[ks][e];
        }
        squares += __shfl_xor(squares, 1, 64);
        squares += __shfl_xor(squares, 2, 64);
        squares += __shfl_xor(squares, 16, 64);
        squares += __shfl_xor(squares, 32, 64);
        if ((lane & 0x33) == 0)  // lane 4b: one per batch slot
            rms_part[wave][b] = squares;
        __syncthreads();
        float total = 0.0f;
        for (uint32_t w = 0; w < blockDim.x / 64; ++w)
            total += rms_part[w][b];
        const float reciprocal = rms_reciprocal(total, a.k, t.epsilon);
        RegX<B::LB> rx[NB];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (blockIdx.x == 0 && t.side && live && uint32_t(ks) < steps && at(ks) < a.k)
                *reinterpret_cast<v4f *>(t.side + row + at(ks)) = xs[ks];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                rx[ks / B::LB].v[ks % B::LB][e] = (xs[ks][e] * reciprocal) * ws[ks][e];
        }
        if (nblk > 0) {
            reg_digits(rx[0], buf0, 0);
            i8_compute(buf0, accf);
        }
        if constexpr (NB > 1) {
            if (nblk > 1) {
                reg_digits(rx[1], buf1, 0);
                i8_compute(buf1, accf);
            }
        }
    } else if constexpr (PRO >= 0) {
        static_assert(NF == 1, "the in-kernel prologue serves m <= 2");
        extern __shared__ float lds_dyn[];
        __shared__ float rms_scratch[8];
        const uint32_t waves = blockDim.x >> 6;
        const uint32_t rp = 4 * a.m;
        // Fragments: k_pad / 64 ksteps x 4 lane blocks x rp rows x 16 bytes.
        int8_t *frag = reinterpret_cast<int8_t *>(lds_dyn + size_t(waves) * S * T * NF * 64);
        float *fxf = reinterpret_cast<float *>(frag + size_t(a.k_pad) * rp);
        int2 *fcorr = reinterpret_cast<int2 *>(fxf + 4 * groups);
        if (nblk > 0)
            i8_load_w(buf0, wp, sp, 0);
        for (uint32_t i = a.m * groups + threadIdx.x; i < 4 * groups; i += blockDim.x) {
            fxf[i] = 0.0f;
            fcorr[i] = int2{0, 0};
        }
        block_prologue<XKind(PRO)>(a.xform, a.m, a.k, groups, rms_scratch,
                                   [&](uint32_t b, uint32_t g, const GroupX &gx) {
                                       emit_group<F>(gx, b, g, 1, rp, 0, frag,
                                                     fxf + b * groups + g, fcorr + b * groups + g);
                                   });
        __syncthreads();
        xp[0] = fxf + q * groups + g_begin;
        cp[0] = fcorr + q * groups + g_begin;
        const LdsFrag<v4i> lap{reinterpret_cast<const v4i *>(frag) + (size_t(s_begin) * 4 + q) * rp +
                                   j,
                               4 * rp, j < rp};
        if (nblk > 0)
            i8_load_a(buf0, lap, xp, cp, 0);
        main_loop(lap);
    } else {
        if (nblk > 0)
            i8_load(buf0, wp, sp, ap, xp, cp, 0);
        main_loop(ap);
    }

    uint32_t batch[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f)
        batch[f] = 4 * f + q;
    reduce_and_store<S, T, NF, E>(a.m, tg, accf, batch, j, a.kparts > 1);
}

// ---------------------------------------------------------------------------
// Streaming ternary GEMV for wide matrices (the LM head, plain activations,
// m <= 8).  Each wave owns one whole tile (16 rows x all of K), so there is
// no cross-wave reduction and no second round of waves: the grid is one
// block of kStreamWaves waves per kStreamWaves tiles.  Loads leave in the
// order they are needed, because the vector memory counter retires them in
// order: the tile's scale block (one coalesced load), the activations of the
// wave's share of the prologue, then the first weight loads of the tile (one
// 16-byte load per lane per 256 k), the rest following kStreamTernaryAhead
// loads ahead of the products.  While the weights are in flight the block forms
// the activation fragments of all of K in LDS: wave w takes fragment w / KL,
// K block w % KL (256 k) and forms it with the register prologue's
// arithmetic (reg_digits, the bytes digits_kernel writes; batch slots at or
// beyond m become zero rows).  After one barrier each wave runs its tile's
// MFMAs with the fragments, group constants and scales read from LDS.
// Group sums are formed and scaled exactly as in i8_compute and accumulated
// over the groups in order.
// ---------------------------------------------------------------------------
constexpr int kStreamWaves = 16;
// Weight loads a wave keeps in flight ahead of its products: a wave that
// issues all of its loads first stalls at the issue of the later ones and
// only computes once they have nearly all arrived.  Measured at 65536 x 2048,
// one row: ternary (one load = 256 k) 9.9 us with all eight ahead, 9.5 /
// 8.8 / 8.1 / 8.2 with one to four; NF4 (one load = 128 k) 28.4 us with all
// sixteen, 24.4 with eight, 21.5 / 20.0 / 21.5 / 21.9 with one to four.
constexpr int kStreamTernaryAhead = 3;
// The same for a wave of the one- or two-row kernel that has no prologue
// pass (it waits at the barrier while the others form the digits): 65536 x
// 2048, one row, 7.34-7.43 us with three, 7.21-7.28 with five or six,
// 7.70-7.82 with eight (interleaved runs on one device).
constexpr int kStreamTernaryIdleAhead = 6;
constexpr int kStreamNf4Ahead = 2;
// Widest grids only: below this many tiles the one-tile-per-block plans
// keep more waves busy.  At 512 tiles (8192 x 2048, us per launch, A/B on
// one device) the streaming kernels measured 4.1 -> 4.3 at one row, 5.6 ->
// 6.0 at four, 8.6 -> 9.0 at eight; at 768 (12288 x 2048) 4.9 -> 4.4 at
// one, 7.5 -> 6.1 at four.
constexpr uint32_t kStreamMinTiles = 768;
// Two rows from 512 tiles: 8192 x 2048 5.5 -> 5.1 us, 8192 x 1024 3.8 -> 3.7
// (one, four and eight rows measured slower there).
constexpr uint32_t kStreamTwoRowMinTiles = 512;
// Fewest blocks a streaming launch spreads its tiles over.
constexpr uint32_t kStreamMinBlocks = 256;

struct StreamArgs {
    const float *x;  // [m, k] plain activations, 16-byte aligned
    const uint8_t *tiles;
    const void *scales;
    float *out;
    uint32_t m, n, k, n_tiles;
    // wide_row_kernel only.  NORM: x is the add + RMS norm of x + b (b may
    // be null) with weight w.  argmax (may be null): one greedy-selection
    // candidate per block.
    const float *b = nullptr, *w = nullptr;
    float epsilon = 0.0f;
    Candidate *argmax = nullptr;
    // wide_row_kernel at one tile per block, MERGE: x is merged from the
    // decode attention's key-range records (XKind::GqaMerge) at a.x.
    uint32_t ranges = 0, head_dim = 0;
};

// One (batch slot, group) record of the prologue: the correction pair and
// the group factor, read with one 16-byte LDS load.
struct StreamRecord {
    int2 corr;
    float xf;
    float pad;
};

template <int NF, int KL, bool HALF, int W>
__global__ __launch_bounds__(64 * W) void stream_ternary_kernel(StreamArgs a)
{
    using ST = typename ScaleT<HALF>::type;
    using B = I8Block<Format::Ternary, 1, 1, NF, HALF>;
    constexpr int G = 2 * KL;   // 128-groups of K (the tile width is 256 * KL)
    constexpr int KS = 4 * KL;  // 64-wide ksteps
    // Prologue units (fragment, 256-k block), wave w taking w, w + W, ...
    constexpr int UNITS = NF * KL;
    constexpr int PER = (UNITS + W - 1) / W;
    // Scale block of a tile: G * 16 values, one SV vector per lane for the
    // first SLANES lanes.
    typedef typename std::conditional<HALF, uint2, v4u>::type SV;
    constexpr int SLANES = G * 16 * (HALF ? 2 : 4) / int(sizeof(SV));
    // Fragments [kstep][fragment][lane] (the MFMA A operand of every lane),
    // records [slot][group] with one spare record per slot (a slot stride of
    // G + 1 records puts the four lane blocks' reads of one group in
    // different banks; at G records they fell in the same ones: 65536 x
    // 2048 at B = 8 13.1-14.1 -> 11.9-12.8 us with the records read one
    // group ahead), each wave's scale block.
    __shared__ v4i frag[KS * NF * 64];
    __shared__ StreamRecord rec[4 * NF * (G + 1)];
    __shared__ SV scale_lds[W * SLANES];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t q = lane >> 4, j = lane & 15;
    const uint32_t tile_id = blockIdx.x * W + wave;
    const uint32_t tile = tile_id < a.n_tiles ? tile_id : a.n_tiles - 1;

    // 1. The tile's scale block.
    SV sv{};
    if (lane < uint32_t(SLANES))
        sv = reinterpret_cast<const SV *>(a.scales)[size_t(tile) * SLANES + lane];
    __builtin_amdgcn_sched_barrier(0);
    // 2. The activations of this wave's prologue units (fragment pf, K block
    // pu): lane 16q + 4b + p holds x[4 pf + b][256 pu + 64 kk + 16q + 4p + t].
    RegX<4> rx[PER];
#pragma unroll
    for (int pi = 0; pi < PER; ++pi) {
        const uint32_t u = wave + W * pi;
        const bool former = u < uint32_t(UNITS);
        const uint32_t pf = u / KL, pu = u % KL;
        const uint32_t pb = 4 * pf + ((lane >> 2) & 3);
        const bool row_live = former && pb < a.m;
        reg_load_issued(rx[pi], a.x + size_t(row_live ? pb : 0) * a.k, row_live, a.k, pu,
                        16 * (lane >> 4) + 4 * (lane & 3), 64);
    }
    __builtin_amdgcn_sched_barrier(0);
    // 3. The first kStreamTernaryAhead weight loads of the tile; the load
    // of K block l + kStreamTernaryAhead leaves when block l's products
    // begin.  Each
    // weight byte is read once: non-temporal loads keep the activations and
    // scales of the next calls in the caches.
    v4u w[KL];
    const v4u *wp = reinterpret_cast<const v4u *>(a.tiles) + size_t(tile) * KL * 64 + lane;
    constexpr int AHEAD = KL < kStreamTernaryAhead ? KL : kStreamTernaryAhead;
#pragma unroll
    for (int l = 0; l < AHEAD; ++l)
        w[l] = __builtin_nontemporal_load(&wp[l * 64]);
    __builtin_amdgcn_sched_barrier(0);

    // 4. The prologue units' fragments and records, then the scale block,
    // into LDS.
#pragma unroll
    for (int pi = 0; pi < PER; ++pi) {
        const uint32_t u = wave + W * pi;
        if (u >= uint32_t(UNITS))
            continue;
        const uint32_t pf = u / KL, pu = u % KL;
        B blk;
        auto emit = [&](auto f_tag) {
            constexpr int F = decltype(f_tag)::value;
            reg_digits(rx[pi], blk, F);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                frag[((4 * pu + ks) * NF + F) * 64 + lane] = blk.af[ks][F];
            if (j == 0) {
#pragma unroll
                for (int gg = 0; gg < 2; ++gg)
                    rec[(4 * F + q) * (G + 1) + 2 * pu + gg] =
                        StreamRecord{blk.cv[gg][F], blk.xf[gg][F], 0.0f};
            }
        };
        if (NF == 1 || pf == 0)
            emit(std::integral_constant<int, 0>{});
        else
            emit(std::integral_constant<int, NF - 1>{});
    }
    if (lane < uint32_t(SLANES))
        scale_lds[wave * SLANES + lane] = sv;
    __syncthreads();

    // 5. The tile's products.  The fragments of the next group are read
    // while the current group's MFMAs run; the compiler barrier keeps reads
    // from being hoisted further.
    const v4i *ap = frag + lane;
    const ST *scl = reinterpret_cast<const ST *>(scale_lds + wave * SLANES) + j;
    auto read_group = [&](int g, v4i (&av)[2][NF]) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int f = 0; f < NF; ++f)
                av[kk][f] = ap[((2 * g + kk) * NF + f) * 64];
    };
    float accf[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f)
        accf[f] = 0.0f;
    v4i cur[2][NF], next[2][NF];
    // Each group's records are read with its fragments, one group ahead.
    StreamRecord rcur[NF], rnext[NF];
    auto read_records = [&](int g, StreamRecord (&rv)[NF]) {
#pragma unroll
        for (int f = 0; f < NF; ++f)
            rv[f] = rec[(4 * f + q) * (G + 1) + g];
    };
    read_group(0, cur);
    read_records(0, rcur);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (g % 2 == 0 && g / 2 + AHEAD < KL)
            w[g / 2 + AHEAD] = __builtin_nontemporal_load(&wp[(g / 2 + AHEAD) * 64]);
        if (g + 1 < G) {
            read_group(g + 1, next);
            read_records(g + 1, rnext);
        }
        v4i acci[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f)
            acci[f] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int s = 2 * g + kk;
            const unsigned word = w[s / 4][s % 4];
            const v4i bw = v4i{int(word), int(word & 0xFCFCFCFCu), int(word & 0xF0F0F0F0u),
                               int(word & 0xC0C0C0C0u)};
#pragma unroll
            for (int f = 0; f < NF; ++f)
                acci[f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur[kk][f], bw, acci[f], 0, 0, 0);
        }
        const float scale = to_f32<HALF>(scl[g * 16]);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const StreamRecord r = rcur[f];
            const v4i d = acci[f];
            // |d.x| < 2^21, so the pairs combine exactly in int32.
            const int hi = (d.x << 8) + d.y - r.corr.x;
            const int lo = (d.z << 8) + d.w - r.corr.y;
            const float gsum = float(hi) * 65536.0f + float(lo);
            accf[f] += gsum * (scale * r.xf);
            // Keep the accumulation here: otherwise it sinks into the
            // guarded store below and every group's MFMA results stay live.
            asm volatile("" : "+v"(accf[f]));
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int f = 0; f < NF; ++f)
                cur[kk][f] = next[kk][f];
#pragma unroll
        for (int f = 0; f < NF; ++f)
            rcur[f] = rnext[f];
        __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t row = tile_id * 16 + j;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const uint32_t b = 4 * f + q;
        if (tile_id < a.n_tiles && b < a.m && row < a.n)
            a.out[size_t(b) * a.n + row] = accf[f];
    }
}

// ---------------------------------------------------------------------------
// Streaming ternary GEMV for one or two activation rows (MB = m), the LM
// head's decode case.  Two changes to stream_ternary_kernel remove work that
// the four-row layout wastes when fewer rows are live:
// - Prologue: lane 16q + 4 slot + p forms the digits of one (batch row,
//   kstep) slot -- slot = kstep offset (MB = 1) or kstep offset + 2 * batch
//   (MB = 2) -- so one pass of the register prologue's arithmetic forms four
//   ksteps (MB = 1) or two ksteps of both rows (MB = 2) where the four-row
//   layout formed one.  The two ksteps of a 128-group are the slots that
//   differ in lane bit 2, so a group's exponent and correction reduce over
//   the lane quad, that bit (DPP row_half_mirror) and the lane blocks.  The
//   bytes are emit_group's.
// - Products: IL = 4 / MB consecutive groups accumulate into one MFMA result,
//   group g in A rows [4 MB (g % IL), +4 MB) (the other rows zero), so lane
//   block q' of the result holds the digit sums of group base + q' / MB,
//   batch row q' % MB, and the digit combine runs once per IL groups.  A lane
//   reads its fragment rows for the groups of its own row block and zeros
//   (an all-zero LDS region at the same offsets) for the others.
// Each lane accumulates its groups in order; the IL partial sums of a row
// are added at the end (row-swap exchanges), which reorders the f32
// additions over groups but not the exact in-group sums.
// ---------------------------------------------------------------------------
// Calls f(integral_constant<int, i>) for i = 0 .. N-1 in order, so every
// index f derives from i is a compile-time constant.
template <typename F, int... I>
__device__ __forceinline__ void unroll_each(F &&f, std::integer_sequence<int, I...>)
{
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void unroll_groups(F &&f)
{
    unroll_each(f, std::make_integer_sequence<int, N>{});
}

// Reductions across lane rows on the VALU (gfx950 v_permlane16/32_swap):
// after the swap of two copies, lane l holds (value of l, value of l ^ 16)
// (or ^ 32) in some order, the same order for both lanes of the pair, so a
// commutative combine gives both lanes the identical result.
__device__ __forceinline__ unsigned max_xor16(unsigned v)
{
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return max(unsigned(r[0]), unsigned(r[1]));
}
__device__ __forceinline__ unsigned max_xor32(unsigned v)
{
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max(unsigned(r[0]), unsigned(r[1]));
}
__device__ __forceinline__ long long sum_xor16(long long v)
{
    const auto lo = __builtin_amdgcn_permlane16_swap(unsigned(v), unsigned(v), false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap(unsigned(v >> 32), unsigned(v >> 32), false,
                                                      false);
    return ((static_cast<long long>(hi[0]) << 32) | unsigned(lo[0])) +
           ((static_cast<long long>(hi[1]) << 32) | unsigned(lo[1]));
}
__device__ __forceinline__ long long sum_xor32(long long v)
{
    const auto lo = __builtin_amdgcn_permlane32_swap(unsigned(v), unsigned(v), false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap(unsigned(v >> 32), unsigned(v >> 32), false,
                                                      false);
    return ((static_cast<long long>(hi[0]) << 32) | unsigned(lo[0])) +
           ((static_cast<long long>(hi[1]) << 32) | unsigned(lo[1]));
}
__device__ __forceinline__ float sum_xor16(float v)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ unsigned half_mirror(unsigned v)
{
    // DPP row_half_mirror: lane i of each 8-lane half reads lane 7 - i.
    return unsigned(__builtin_amdgcn_mov_dpp(int(v), 0x141, 0xF, 0xF, false));
}

template <int MB, int KL, bool HALF, int W>
__global__ __launch_bounds__(64 * W) void stream_ternary_rows_kernel(StreamArgs a)
{
    using ST = typename ScaleT<HALF>::type;
    constexpr int IL = 4 / MB;          // groups per MFMA accumulation
    constexpr int RB = 4 * MB;          // A rows of one group's block
    constexpr int G = 2 * KL;           // 128-groups of K
    constexpr int KS = 4 * KL;          // 64-wide ksteps
    constexpr int PASS_KS = 4 / MB;     // ksteps one prologue pass forms
    constexpr int PASSES = KS / PASS_KS;
    static_assert(G % IL == 0, "whole accumulations");
    typedef typename std::conditional<HALF, uint2, v4u>::type SV;
    constexpr int SLANES = G * 16 * (HALF ? 2 : 4) / int(sizeof(SV));
    // Fragments [kstep][lane block][row 4b + p] (16 B each), records
    // [batch][group], each wave's scale block.
    __shared__ v4i frag[KS * 4 * RB];
    __shared__ v4i zeros[KS * 4 * RB];
    __shared__ StreamRecord rec[MB * G];
    __shared__ SV scale_lds[W * SLANES];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t q = lane >> 4, j = lane & 15, p = lane & 3, slot = (lane >> 2) & 3;
    const uint32_t tile_id = blockIdx.x * W + wave;
    const uint32_t tile = tile_id < a.n_tiles ? tile_id : a.n_tiles - 1;

    // 1. The tile's scale block.
    SV sv{};
    if (lane < uint32_t(SLANES))
        sv = reinterpret_cast<const SV *>(a.scales)[size_t(tile) * SLANES + lane];
    __builtin_amdgcn_sched_barrier(0);
    // 2. The values of this wave's prologue passes (wave w takes passes w,
    // w + W, ...): slot -> (batch b, kstep s).
    constexpr int PER = (PASSES + W - 1) / W;
    const uint32_t pb = MB == 1 ? 0 : slot >> 1;
    v4f xv[PER];
#pragma unroll
    for (int pi = 0; pi < PER; ++pi) {
        const uint32_t pass = wave + W * pi < uint32_t(PASSES) ? wave + W * pi : 0;
        const uint32_t ps = pass * PASS_KS + (MB == 1 ? slot : slot & 1);
        const uint32_t kx = 64 * ps + 16 * q + 4 * p;
        xv[pi] = *reinterpret_cast<const v4f *>(a.x + size_t(pb) * a.k + (kx < a.k ? kx : 0));
    }
    __builtin_amdgcn_sched_barrier(0);
    // Steps 3-5 with AHEAD_W weight loads in flight: a wave with a prologue
    // pass keeps kStreamTernaryAhead, a wave without one (it only waits at
    // the barrier) kStreamTernaryIdleAhead.  The choice is wave-uniform and
    // every wave reaches the one barrier of either copy.
    auto rest = [&](auto ahead_tag) {
        constexpr int AHEAD_W = decltype(ahead_tag)::value;
        // 3. The first weight loads of the tile.
        v4u w[KL];
        const v4u *wp = reinterpret_cast<const v4u *>(a.tiles) + size_t(tile) * KL * 64 + lane;
        constexpr int AHEAD = KL < AHEAD_W ? KL : AHEAD_W;
#pragma unroll
        for (int l = 0; l < AHEAD; ++l)
            w[l] = __builtin_nontemporal_load(&wp[l * 64]);
        __builtin_amdgcn_sched_barrier(0);

        // 4. The prologue passes (the register prologue's arithmetic, per slot),
        // then the scale block, into LDS.
#pragma unroll
        for (int pi = 0; pi < PER; ++pi) {
            const uint32_t pass = wave + W * pi;
            if (pass >= uint32_t(PASSES))
                continue;
            const uint32_t ps = pass * PASS_KS + (MB == 1 ? slot : slot & 1);
            const bool inb = 64 * ps + 16 * q + 4 * p < a.k;
            float v[4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
                v[t] = inb ? xv[pi][t] : 0.0f;
            unsigned mb = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t)
                mb = max(mb, __float_as_uint(v[t]) & 0x7FFFFFFFu);
            mb = max(mb, quad_xor1(mb));
            mb = max(mb, quad_xor2(mb));
            mb = max(mb, half_mirror(mb));
            mb = max_xor16(mb);
            mb = max_xor32(mb);
            const bool bad = mb >= 0x7F800000u;
            int e = 0;
            if (!bad && mb)
                frexpf(__uint_as_float(mb), &e);  // |x| < 2^e
            const float factor = bad ? __builtin_nanf("") : ldexpf(1.0f, e - 30);
            long long corr = 0;
            unsigned vp[4];
            int u_prev = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                int val = bad ? 0 : int(rintf(ldexpf(v[t], 30 - e)));
                // Field t of the nested masks (see the operand-field note).
                const int u = t == 0 ? val : (val + (1 << (2 * t - 1))) >> (2 * t);
                val = t == 0 ? u : u - u_prev;
                u_prev = u;
                corr += t < 3 ? (static_cast<long long>(u) << (2 * t))
                              : -(static_cast<long long>(u) << 6);
                vp[t] = unsigned(val + 0x808080);
            }
            unsigned d[4], wd[4];
            byte_transpose<true>(vp, d);
            quad_transpose(d, p);
            byte_transpose<false>(d, wd);
            const unsigned flip = p ? 0x80808080u : 0u;
            frag[(ps * 4 + q) * RB + 4 * pb + p] =
                v4i{int(wd[0] ^ flip), int(wd[1] ^ flip), int(wd[2] ^ flip), int(wd[3] ^ flip)};
            corr += static_cast<long long>(quad_xor1(unsigned(corr))) |
                    (static_cast<long long>(quad_xor1(unsigned(corr >> 32))) << 32);
            corr += static_cast<long long>(quad_xor2(unsigned(corr))) |
                    (static_cast<long long>(quad_xor2(unsigned(corr >> 32))) << 32);
            corr += static_cast<long long>(half_mirror(unsigned(corr))) |
                    (static_cast<long long>(half_mirror(unsigned(corr >> 32))) << 32);
            corr = sum_xor16(corr);
            corr = sum_xor32(corr);
            // Split as hi * 2^16 + lo to match the epilogue's digit pairs.
            const long long lo = ((corr + 32768) & 65535) - 32768;
            const int hi = int((corr - lo) >> 16);
            if (lane < 16 && p == 0 && (slot & 1) == 0)
                rec[pb * G + ps / 2] = StreamRecord{int2{hi, int(lo)}, factor, 0.0f};
        }
        for (uint32_t i = threadIdx.x; i < uint32_t(KS * 4 * RB); i += 64 * W)
            zeros[i] = v4i{0, 0, 0, 0};
        if (lane < uint32_t(SLANES))
            scale_lds[wave * SLANES + lane] = sv;
        __syncthreads();

        // 5. The tile's products.  Lane (q, i) supplies A row i: row block
        // i / RB takes the groups g with g % IL == i / RB.
        const uint32_t phase = j / RB;
        const ST *scl = reinterpret_cast<const ST *>(scale_lds + wave * SLANES) + j;
        // Per phase, the lane's fragment base: its own compact rows for its row
        // block's phase, the zero region (same offsets) for the others.  Every
        // read is then one unconditional 16-byte LDS load.
        const v4i *abase[IL];
#pragma unroll
        for (int ph = 0; ph < IL; ++ph)
            abase[ph] = (phase == uint32_t(ph) ? frag : zeros) + q * RB + j % RB;
        v4i cur[2], next[2];
        auto read_group = [&](auto g_tag, v4i (&av)[2]) {
            constexpr int g = decltype(g_tag)::value;
            av[0] = abase[g % IL][(2 * g) * 4 * RB];
            av[1] = abase[g % IL][(2 * g + 1) * 4 * RB];
        };
        // Lane block q' of each accumulation holds group base + q' / MB, batch
        // row q' % MB.
        const uint32_t my_group = q / MB, my_batch = q % MB;
        float accf = 0.0f;
        v4i acci = v4i{0, 0, 0, 0};
        read_group(std::integral_constant<int, 0>{}, cur);
        unroll_groups<G>([&](auto g_tag) {
            constexpr int g = decltype(g_tag)::value;
            if constexpr (g % 2 == 0 && g / 2 + AHEAD < KL)
                w[g / 2 + AHEAD] = __builtin_nontemporal_load(&wp[(g / 2 + AHEAD) * 64]);
            if constexpr (g + 1 < G)
                read_group(std::integral_constant<int, g + 1>{}, next);
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int s = 2 * g + kk;
                const unsigned word = w[s / 4][s % 4];
                const v4i bw = v4i{int(word), int(word & 0xFCFCFCFCu), int(word & 0xF0F0F0F0u),
                                   int(word & 0xC0C0C0C0u)};
                acci = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur[kk], bw, acci, 0, 0, 0);
            }
            cur[0] = next[0];
            cur[1] = next[1];
            if constexpr (g % IL == IL - 1) {
                const uint32_t gg = uint32_t(g - (IL - 1)) + my_group;
                const StreamRecord r = rec[my_batch * G + gg];
                const float scale = to_f32<HALF>(scl[gg * 16]);
                // |d.x| < 2^21, so the pairs combine exactly in int32.
                const int hi = (acci.x << 8) + acci.y - r.corr.x;
                const int lo = (acci.z << 8) + acci.w - r.corr.y;
                const float gsum = float(hi) * 65536.0f + float(lo);
                accf += gsum * (scale * r.xf);
                // Keep the accumulation here: otherwise it sinks into the
                // guarded store below and every group's MFMA results stay live.
                asm volatile("" : "+v"(accf));
                acci = v4i{0, 0, 0, 0};
            }
            __builtin_amdgcn_sched_barrier(0);
        });
        // The IL partial sums of each batch row: lane blocks q' with equal
        // q' % MB.
        if constexpr (MB == 1)
            accf = sum_xor16(accf);
        accf = sum_xor32(accf);
        const uint32_t row = tile_id * 16 + j;
        if (q < uint32_t(MB) && tile_id < a.n_tiles && q < a.m && row < a.n)
            a.out[size_t(q) * a.n + row] = accf;
    };
    if (wave < uint32_t(PASSES))
        rest(std::integral_constant<int, kStreamTernaryAhead>{});
    else
        rest(std::integral_constant<int, kStreamTernaryIdleAhead>{});
}

// ---------------------------------------------------------------------------
// NF4 GEMV on f16 MFMA.  One loop block = one 16-byte lane load per tile =
// four 32-wide ksteps = one 128-weight group.
// ---------------------------------------------------------------------------
// One table copy: interleaved copies that spread the lanes of a read over
// distinct banks measured slower (65536 x 2048 at one row: 4, 16 and 32
// copies 27.2, 31.3 and 45.6 us against 25.4) -- the build work and LDS
// footprint cost more than the bank conflicts they remove.
constexpr uint32_t kLutCopies = 1;

// Table entry for one code byte: x = hi halves of (low nibble, high nibble),
// y = lo halves, each a packed f16 pair for consecutive k.  The levels are
// literal constants picked by selects, so no memory access delays the
// table: a per-lane constant-memory load issued after the weight loads
// would wait for all of them (loads retire in order), and one issued before
// them made every decode GEMV wait a memory round trip before its first
// load.
__device__ __forceinline__ uint2 nf4_lut_entry(uint32_t e)
{
    const float *lv = kNf4LevelValues;
    float l0 = lv[0], l1 = lv[0];
#pragma unroll
    for (int c = 1; c < 16; ++c) {
        l0 = (e & 15u) == uint32_t(c) ? lv[c] : l0;
        l1 = (e >> 4) == uint32_t(c) ? lv[c] : l1;
    }
    const _Float16 h0 = _Float16(l0), h1 = _Float16(l1);
    const _Float16 r0 = _Float16(l0 - float(h0)), r1 = _Float16(l1 - float(h1));
    return uint2{unsigned(__builtin_bit_cast(unsigned short, h0)) |
                     (unsigned(__builtin_bit_cast(unsigned short, h1)) << 16),
                 unsigned(__builtin_bit_cast(unsigned short, r0)) |
                     (unsigned(__builtin_bit_cast(unsigned short, r1)) << 16)};
}

template <int T, int S, bool HALF>
struct Nf4Block {
    v4u w[S][T];
    typename ScaleT<HALF>::type sc[S][T];  // the group's weight scales (this lane's row)
    v8h af[4];
    float xf[2];  // the group's activation factors of batch rows 2q, 2q + 1
};

template <int T, int S, bool HALF, typename AP>
__device__ __forceinline__ void nf4_load(Nf4Block<T, S, HALF> &blk, const v4u *const (&wp)[S][T],
                                         const typename ScaleT<HALF>::type *const (&sp)[S][T],
                                         const AP &ap, const float *const (&xp)[2],
                                         uint32_t index)
{
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            blk.w[st][t] = wp[st][t][index * 64];
            blk.sc[st][t] = sp[st][t][index * 16];
        }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
        blk.af[ks] = ap.at(index * 4 + ks, 0, 1);
    blk.xf[0] = xp[0][index];
    blk.xf[1] = xp[1][index];
}

// The activation half of nf4_load (fragments and group factors), for a
// block whose weights were loaded ahead of the in-kernel prologue.
template <int T, int S, bool HALF, typename AP>
__device__ __forceinline__ void nf4_load_a(Nf4Block<T, S, HALF> &blk, const AP &ap,
                                           const float *const (&xp)[2], uint32_t index)
{
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
        blk.af[ks] = ap.at(index * 4 + ks, 0, 1);
    blk.xf[0] = xp[0][index];
    blk.xf[1] = xp[1][index];
}

template <int T, int S, bool HALF>
__device__ __forceinline__ void nf4_compute(const Nf4Block<T, S, HALF> &blk,
                                            float (&accf)[S][T][2], const uint2 *lut)
{
    v4f acc[S][T];
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int t = 0; t < T; ++t)
            acc[st][t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int st = 0; st < S; ++st)
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const unsigned word = blk.w[st][t][ks];
                v4u hi, lo;
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const uint2 e = lut[((word >> (8 * p)) & 255u) * kLutCopies];
                    hi[p] = e.x;
                    lo[p] = e.y;
                }
                acc[st][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    blk.af[ks], __builtin_bit_cast(v8h, hi), acc[st][t], 0, 0, 0);
                acc[st][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    blk.af[ks], __builtin_bit_cast(v8h, lo), acc[st][t], 0, 0, 0);
            }
    }
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            // Rows 4q + {0,1} are batch 2q (hi, lo), rows 4q + {2,3} batch 2q+1.
            const float sc = to_f32<HALF>(blk.sc[st][t]);
            accf[st][t][0] += (acc[st][t].x + acc[st][t].y) * (sc * blk.xf[0]);
            accf[st][t][1] += (acc[st][t].z + acc[st][t].w) * (sc * blk.xf[1]);
        }
}

// Weights and group scales of NF4 loop block `index`.
template <int T, int S, bool HALF>
__device__ __forceinline__ void nf4_load_w(Nf4Block<T, S, HALF> &blk,
                                           const v4u *const (&wp)[S][T],
                                           const typename ScaleT<HALF>::type *const (&sp)[S][T],
                                           uint32_t index)
{
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            blk.w[st][t] = wp[st][t][index * 64];
            blk.sc[st][t] = sp[st][t][index * 16];
        }
}

// NF4 register prologue (m <= 8).  Lane 16q + 2b + h supplies half h (0:
// hi, 1: lo) of batch b in the f16 A operand, eight values
// k = 32s + 8q + 0..7 per 32-wide kstep s.  The lane pair splits them:
// lane h loads values 4h..4h+3 (k offset nf4_reg_offset), splits them
// into binary16 hi and lo, keeps its own half and sends its partner the
// other (DPP).  The group exponent reduces over the batch's eight lanes
// (the pair and the lane blocks).  The arithmetic is halves_kernel's value
// for value.
__device__ __forceinline__ uint32_t nf4_reg_offset()
{
    const uint32_t lane = threadIdx.x & 63;
    return 8 * (lane >> 4) + 4 * (lane & 1);
}

__device__ __forceinline__ void nf4_reg_load(RegX<4> &rx, const float *xrow, bool live,
                                             uint32_t k, uint32_t s0, uint32_t index)
{
    const uint32_t off = nf4_reg_offset();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const uint32_t kx = 32 * (s0 + index * 4 + kk) + off;
        rx.v[kk] = live && kx < k ? *reinterpret_cast<const v4f *>(xrow + kx)
                                  : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
}

__device__ __forceinline__ unsigned pack_halves(_Float16 lo_k, _Float16 hi_k)
{
    return unsigned(__builtin_bit_cast(unsigned short, lo_k)) |
           (unsigned(__builtin_bit_cast(unsigned short, hi_k)) << 16);
}

template <int T, int S, bool HALF>
__device__ __forceinline__ void nf4_reg_halves(const RegX<4> &rx, Nf4Block<T, S, HALF> &blk)
{
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t h = lane & 1, q = lane >> 4;
    unsigned mb = 0;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int t = 0; t < 4; ++t)
            mb = max(mb, __float_as_uint(rx.v[kk][t]) & 0x7FFFFFFFu);
    mb = max(mb, quad_xor1(mb));
    mb = max(mb, unsigned(__shfl_xor(int(mb), 16, 64)));
    mb = max(mb, unsigned(__shfl_xor(int(mb), 32, 64)));
    const bool bad = mb >= 0x7F800000u;
    int e = 0;
    if (!bad && mb)
        frexpf(__uint_as_float(mb), &e);  // |x| < 2^e
    const float factor = bad ? __builtin_nanf("") : ldexpf(1.0f, e);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        unsigned mine[2], recv[2];
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
            const float v0 = bad ? 0.0f : ldexpf(rx.v[kk][2 * pr], -e);
            const float v1 = bad ? 0.0f : ldexpf(rx.v[kk][2 * pr + 1], -e);
            const _Float16 h0 = _Float16(v0), h1 = _Float16(v1);
            const _Float16 l0 = _Float16(v0 - float(h0)), l1 = _Float16(v1 - float(h1));
            const unsigned hi_pair = pack_halves(h0, h1), lo_pair = pack_halves(l0, l1);
            mine[pr] = h ? lo_pair : hi_pair;
            recv[pr] = quad_xor1(h ? hi_pair : lo_pair);  // the partner's half h
        }
        // Values 0..3 of the lane block come from lane h = 0, 4..7 from h = 1.
        const v4u d = h ? v4u{recv[0], recv[1], mine[0], mine[1]}
                        : v4u{mine[0], mine[1], recv[0], recv[1]};
        blk.af[kk] = __builtin_bit_cast(v8h, d);
    }
    // Lane (q, j) applies the factors of batches 2q and 2q + 1: lanes 4q and
    // 4q + 2 hold them.
    blk.xf[0] = __shfl(factor, int(4 * q), 64);
    blk.xf[1] = __shfl(factor, int(4 * q + 2), 64);
}

// Block shapes as gemv_i8_kernel's; one-tile single-stream kernels with the
// separate or register prologue (at most 116 VGPRs) also run 16 waves.
template <int T, int S, bool HALF, Epilogue E, int PRO>
__global__ __launch_bounds__(T == 1 && S == 1 && (PRO < 0 || PRO == kRegPro) ? 1024 : 512)
void gemv_nf4_kernel(MfmaArgs a)
{
    using ST = typename ScaleT<HALF>::type;
    // kLutCopies interleaved copies of the 256-entry table; lane l reads copy
    // l % kLutCopies, so the lanes of one LDS cycle spread over distinct banks.
    // Built after the first loads are issued (it needs no memory access);
    // a barrier orders it before the first product.
    __shared__ uint2 lut_all[256 * kLutCopies];
    auto build_table = [&] {
        for (uint32_t i = threadIdx.x; i < 256 * kLutCopies; i += blockDim.x)
            lut_all[i] = nf4_lut_entry(i / kLutCopies);
    };
    const uint2 *lut = lut_all + (threadIdx.x % kLutCopies);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t q = lane >> 4, j = lane & 15;
    const Target tg = target_of<T>(a);
    const uint32_t tile0 = tg.tile0;
    const uint32_t groups = a.k_pad / 128;
    const uint32_t part = a.kparts > 1 ? blockIdx.x / a.part_blocks : 0;
    const uint32_t s_begin =
        (part * (blockDim.x >> 6) + wave) * a.ksteps_per_wave;  // 32-wide ksteps
    const uint32_t nblk = a.ksteps_per_wave / 4;
    const uint32_t g_begin = s_begin / 4;
    const size_t tile_vecs = size_t(a.k_pad) / 128 * 64;

    const v4u *wp[S][T];
    const ST *sp[S][T];
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            wp[st][t] = reinterpret_cast<const v4u *>(tg.tiles[st]) + (tile0 + t) * tile_vecs +
                        g_begin * 64 + lane;
            sp[st][t] = reinterpret_cast<const ST *>(tg.scales[st]) +
                        (size_t(tile0 + t) * groups + g_begin) * 16 + j;
        }
    const float *xp[2] = {a.xf + (2 * q) * groups + g_begin, a.xf + (2 * q + 1) * groups + g_begin};

    float accf[S][T][2];
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int t = 0; t < T; ++t)
            accf[st][t][0] = accf[st][t][1] = 0.0f;

    // buf0 holds loop block 0 on entry.
    Nf4Block<T, S, HALF> buf0, buf1;
    auto main_loop = [&](const auto &ap) {
        for (uint32_t i = 0; i < nblk; i += 2) {
            if (i + 1 < nblk)
                nf4_load(buf1, wp, sp, ap, xp, i + 1);
            nf4_compute(buf0, accf, lut);
            if (i + 1 < nblk) {
                if (i + 2 < nblk)
                    nf4_load(buf0, wp, sp, ap, xp, i + 2);
                nf4_compute(buf1, accf, lut);
            }
        }
    };
    if constexpr (PRO == kRegPro) {
        const uint32_t b = (lane >> 1) & 7;
        const bool live = b < a.m;
        const float *xrow = a.xform.a + size_t(live ? b : 0) * a.k;
        RegX<4> rx0, rx1;
        if (nblk > 0) {
            nf4_reg_load(rx0, xrow, live, a.k, s_begin, 0);
            nf4_load_w(buf0, wp, sp, 0);
        }
        build_table();
        __syncthreads();
        for (uint32_t i = 0; i < nblk; i += 2) {
            if (i + 1 < nblk) {
                nf4_reg_load(rx1, xrow, live, a.k, s_begin, i + 1);
                nf4_load_w(buf1, wp, sp, i + 1);
            }
            nf4_reg_halves(rx0, buf0);
            nf4_compute(buf0, accf, lut);
            if (i + 1 < nblk) {
                if (i + 2 < nblk) {
                    nf4_reg_load(rx0, xrow, live, a.k, s_begin, i + 2);
                    nf4_load_w(buf0, wp, sp, i + 2);
                }
                nf4_reg_halves(rx1, buf1);
                nf4_compute(buf1, accf, lut);
            }
        }
    } else if constexpr (PRO >= 0) {
        extern __shared__ float lds_dyn[];
        __shared__ float rms_scratch[8];
        const uint32_t waves = blockDim.x >> 6;
        const uint32_t rp = 2 * a.m;
        _Float16 *frag = reinterpret_cast<_Float16 *>(lds_dyn + size_t(waves) * S * T * 2 * 64);
        // Fragments: k_pad / 32 ksteps x 4 lane blocks x rp rows x 8 halves.
        float *fxf = reinterpret_cast<float *>(frag + size_t(a.k_pad) * rp);
        // The first weights go out before the prologue's activation loads:
        // their latencies overlap instead of adding up.
        if (nblk > 0)
            nf4_load_w(buf0, wp, sp, 0);
        build_table();  // ordered before the products by the barrier below
        for (uint32_t i = a.m * groups + threadIdx.x; i < 8 * groups; i += blockDim.x)
            fxf[i] = 0.0f;
        block_prologue<XKind(PRO)>(a.xform, a.m, a.k, groups, rms_scratch,
                                   [&](uint32_t b, uint32_t g, const GroupX &gx) {
                                       emit_halves(gx, b, g, rp, groups, frag, fxf);
                                   });
        __syncthreads();
        xp[0] = fxf + (2 * q) * groups + g_begin;
        xp[1] = fxf + (2 * q + 1) * groups + g_begin;
        const LdsFrag<v8h> lap{reinterpret_cast<const v8h *>(frag) + (size_t(s_begin) * 4 + q) * rp +
                                   j,
                               4 * rp, j < rp};
        if (nblk > 0)
            nf4_load_a(buf0, lap, xp, 0);
        main_loop(lap);
    } else {
        const GlobalFrag<v8h> gap{reinterpret_cast<const v8h *>(a.afrag) + size_t(s_begin) * 64 +
                                  lane};
        if (nblk > 0)
            nf4_load(buf0, wp, sp, gap, xp, 0);
        build_table();
        __syncthreads();
        main_loop(gap);
    }
    const uint32_t batch[2] = {2 * q, 2 * q + 1};
    reduce_and_store<S, T, 2, E>(a.m, tg, accf, batch, j, a.kparts > 1);
}

// ---------------------------------------------------------------------------
// Streaming NF4 GEMV for wide matrices (the LM head, plain activations,
// m <= 8), laid out as stream_ternary_kernel: each wave owns one whole tile
// (16 rows x all of K) and the block forms the f16 activation fragments of
// all of K once, in LDS, for its kStreamWaves tiles.  Loads leave in the
// order they are needed: the tile's scale block, the activations of the
// wave's prologue group (wave w forms 128-group w with nf4_reg_halves'
// arithmetic; batch slots at or beyond m become zero rows), then the first
// weight loads of the tile (16 bytes per lane per group), the rest following
// kStreamNf4Ahead groups ahead of the products.  After the barriers each wave
// runs its tile's MFMAs kstep by kstep, reading the next kstep's fragment and
// table entries while the current kstep's MFMAs run.  Group sums are formed
// and scaled exactly as in nf4_compute and accumulated over the groups in
// order.
// ---------------------------------------------------------------------------
constexpr uint32_t kStreamLutCopies = 32;
// The code-byte table with C copies of each entry (C = 32, 16 or 8): the
// cells of one byte value lie 8 C bytes apart, and a lane's cell address is
// (code byte) * 256 + 8 * spread * (lane % C), shifted right by `shift`
// (one byte permute and one shift).  Kernels of one block per row tile
// (below the head size) fill 8 copies: their blocks are short, and the
// 64 KB fill of 32 copies sat on every block's path (1.2B-shape decode 2289
// -> 2337 tok/s, NF4 4608 x 1024 at one row 4.48 -> 3.70 us, 8192 x 2048
// 5.44 -> 4.88; the head, 13.8 us with 32, takes 17.1 with 8).
template <uint32_t C>
struct LutLayout {
    static_assert(C == 32 || C == 16 || C == 8, "table copies");
    static constexpr uint32_t copies = C;
    static constexpr uint32_t shift = C == 32 ? 0 : C == 16 ? 1 : 2;
    static constexpr uint32_t spread = 1u << shift;
};
constexpr uint32_t kSmallLutCopies = 8;

template <int G, bool HALF>
__global__ __launch_bounds__(64 * kStreamWaves) void stream_nf4_kernel(StreamArgs a)
{
    using ST = typename ScaleT<HALF>::type;
    constexpr int KS = 4 * G;  // 32-wide ksteps
    static_assert(G <= kStreamWaves, "one prologue group per wave");
    typedef typename std::conditional<HALF, uint2, v4u>::type SV;
    constexpr int SLANES = G * 16 * (HALF ? 2 : 4) / int(sizeof(SV));
    static_assert(SLANES <= 64, "one scale vector per lane");
    // Fragments [kstep][lane], group factors [batch slot][group], each
    // wave's scale block, and the code-byte table: 256 B per byte value,
    // kStreamLutCopies copies of its (hi, lo) word pair.  Lane l reads copy
    // l % 32 with one 8-byte load, so the 32 lanes of each half-wave read 256
    // distinct bytes of banks, and a byte's cell address is one byte permute
    // of the code word.  (Two 4-byte reads per byte measured half the rate:
    // 4-byte LDS reads run at about 265 GB/s per CU whatever their pattern,
    // 8-byte ones at about 515, scattered table reads included.)
    __shared__ v8h frag[KS * 64];
    __shared__ float xfs[8 * G];
    __shared__ SV scale_lds[kStreamWaves * SLANES];
    __shared__ unsigned lut[256 * 2 * kStreamLutCopies];
    __shared__ uint2 entries[256];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t q = lane >> 4, j = lane & 15;
    const uint32_t tile_id = blockIdx.x * kStreamWaves + wave;
    const uint32_t tile = tile_id < a.n_tiles ? tile_id : a.n_tiles - 1;

    // 1. The tile's scale block.
    SV sv{};
    if (lane < uint32_t(SLANES))
        sv = reinterpret_cast<const SV *>(a.scales)[size_t(tile) * SLANES + lane];
    __builtin_amdgcn_sched_barrier(0);
    // 2. The activations of this wave's prologue group (lane 16q + 2b + h:
    // batch slot b).
    const bool former = wave < uint32_t(G);
    const uint32_t pb = (lane >> 1) & 7;
    const bool row_live = former && pb < a.m;
    RegX<4> rx;
    reg_load_issued(rx, a.x + size_t(row_live ? pb : 0) * a.k, row_live, a.k,
                    former ? wave : 0, nf4_reg_offset(), 32);
    __builtin_amdgcn_sched_barrier(0);
    // 3. The first kStreamNf4Ahead weight loads of the tile (each byte is
    // read once); the load of group g + kStreamNf4Ahead leaves when group g's
    // products begin.
    v4u w[G];
    const v4u *wp = reinterpret_cast<const v4u *>(a.tiles) + size_t(tile) * G * 64 + lane;
    constexpr int AHEAD = G < kStreamNf4Ahead ? G : kStreamNf4Ahead;
#pragma unroll
    for (int g = 0; g < AHEAD; ++g)
        w[g] = __builtin_nontemporal_load(&wp[g * 64]);
    __builtin_amdgcn_sched_barrier(0);

    // 4. The table, the prologue group's fragments and factors and the
    // scale block, into LDS.  Only the fragment rows of live batch slots
    // (j < 2m) are written; a lane of a dead slot reads a live row of its
    // lane block instead (its output rows are never stored, and the read
    // shares the live lane's address).
    const uint32_t rp = 2 * a.m;
    const bool row_read = j < rp;
    if (threadIdx.x < 256)
        entries[threadIdx.x] = nf4_lut_entry(threadIdx.x);
    __syncthreads();
    for (uint32_t v = threadIdx.x; v < 256 * 2 * kStreamLutCopies / 4; v += blockDim.x) {
        const uint2 e = entries[v / (2 * kStreamLutCopies / 4)];
        reinterpret_cast<v4u *>(lut)[v] = v4u{e.x, e.y, e.x, e.y};
    }
    if (former) {
        Nf4Block<1, 1, HALF> blk;
        nf4_reg_halves(rx, blk);
        if (row_read) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                frag[(4 * wave + ks) * 64 + lane] = blk.af[ks];
        }
        if (j == 0) {
            xfs[(2 * q) * G + wave] = blk.xf[0];
            xfs[(2 * q + 1) * G + wave] = blk.xf[1];
        }
    }
    if (lane < uint32_t(SLANES))
        scale_lds[wave * SLANES + lane] = sv;
    __syncthreads();

    // 5. The tile's products.
    const ST *scl = reinterpret_cast<const ST *>(scale_lds + wave * SLANES) + j;
    struct Step {
        v8h af;
        v4u hi, lo;
    };
    const v8h *ap = frag + 16 * q + (row_read ? j : j % rp);
    // Byte 0 of the cell address: the lane's copy.
    const unsigned copy_byte = 8 * (lane % kStreamLutCopies);
    const char *cells = reinterpret_cast<const char *>(lut);
    auto read_step = [&](int s, Step &st) {
        st.af = ap[s * 64];
        const unsigned word = w[s / 4][s % 4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            // (code byte p) * 256 + copy_byte.
            const unsigned at = __builtin_amdgcn_perm(word, copy_byte, 0x0C0C0000u | ((4u + p) << 8));
            const uint2 e = *reinterpret_cast<const uint2 *>(cells + at);
            st.hi[p] = e.x;
            st.lo[p] = e.y;
        }
    };
    float accf[2] = {0.0f, 0.0f};
    Step cur, next;
    read_step(0, cur);
    v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        if (s % 4 == 0 && s / 4 + AHEAD < G)
            w[s / 4 + AHEAD] = __builtin_nontemporal_load(&wp[(s / 4 + AHEAD) * 64]);
        if (s + 1 < KS)
            read_step(s + 1, next);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.af, __builtin_bit_cast(v8h, cur.hi), acc,
                                                     0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.af, __builtin_bit_cast(v8h, cur.lo), acc,
                                                     0, 0, 0);
        if (s % 4 == 3) {
            // Rows 4q + {0,1} are batch 2q (hi, lo), rows 4q + {2,3} batch 2q+1.
            const int g = s / 4;
            const float sc = to_f32<HALF>(scl[g * 16]);
            accf[0] += (acc.x + acc.y) * (sc * xfs[(2 * q) * G + g]);
            accf[1] += (acc.z + acc.w) * (sc * xfs[(2 * q + 1) * G + g]);
            // Keep the accumulation here (see stream_ternary_kernel).
            asm volatile("" : "+v"(accf[0]), "+v"(accf[1]));
            acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
        cur = next;
        __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t row = tile_id * 16 + j;
#pragma unroll
    for (int f = 0; f < 2; ++f) {
        const uint32_t b = 2 * q + f;
        if (tile_id < a.n_tiles && b < a.m && row < a.n)
            a.out[size_t(b) * a.n + row] = accf[f];
    }
}

// ---------------------------------------------------------------------------
// Wide-matrix GEMV at one activation row (the LM heads at decode): each wave
// owns one 256-wide slice of K ("part" p of P = K / 256) and streams that
// slice of R tiles, so a block of 16 waves covers TS = 16 / P tiles per
// round, R rounds: 16 contiguous KB of codes per round for ternary, 32 for
// NF4, 64 for INT8.  The activation operand never goes through LDS:
// - One pass of the register prologue's arithmetic over the slice gives
//   lane 16q + j exactly the A operand row j it supplies for one kstep:
//   integer formats: lane 16q + 4s + p holds digit p of kstep s (s = 0..3,
//   two 128-groups); NF4: lane 16q + 2s + h holds half h of kstep s
//   (s = 0..7, two groups).  For kstep s the wave feeds A = (own kstep == s
//   ? own fragment : 0), so row j of the MFMA result holds kstep s's sums
//   in rows 4s + p (2s + h): one accumulation covers the whole slice.
// - The group exponents, factors and ternary corrections reduce over the
//   lanes of a group (quad, half-row mirror, row swaps) once per wave, for
//   all of its R tiles.
// Per tile, lane block q' holds ksteps q' (2q', 2q' + 1 for NF4); a row swap
// adds the two halves of each group, the group sum is scaled as elsewhere
// (digit combine or hi + lo, times scale * factor), and a second swap adds
// the slice's two groups.  The slices' partial sums meet in LDS and are
// added in slice order once every wave is done.  The in-group sums are
// exact as in the other kernels; only the order of the f32 additions over
// groups differs.
// ---------------------------------------------------------------------------
// 16-byte lane loads in flight per wave.  Two measured faster than three
// once the kernels' register use fell to 56-62 VGPRs (INT8 65536x2048 B=1
// 22.1-22.3 -> 21.5-21.7 us, 65536x1024 12.0-12.2 -> 11.6-11.7, 8192x2048
// 4.85-4.92 -> 4.65-4.73; four and five in between), with LFM2 decode and
// the ternary products unchanged.
constexpr int kWideAhead = 2;
// NF4 in wide_row_kernel: ksteps between a kstep's table reads and its
// products (a ring of that many B-operand pairs in registers).
constexpr int kNf4TableAhead = 1;
// The NF4 head: two measured slightly faster than three (mean of eight
// 100-launch bursts 15.2 against 15.7 us; four to six slower).
constexpr int kWideAheadNf4 = 2;
// The same in the norm variant, whose block barrier holds back the loads
// issued after it: 1.2B-shape decode 2298 tok/s with 3, 2307 with 6, 2285
// with all (16).
constexpr int kWideAheadNorm = 6;

// The packed one-row operand layout (wide_row_kernel, wide_pair_kernel):
// lane 16q + 4s + p holds x[64 s + 16 q + 4 p + t], t = 0..3, of a 256-k
// slice (s: the slice's kstep, which lane bit 3 splits into its two
// 128-groups).  The group's exponent (|x| < 2^e) reduces over lane bits 0-2
// and the lane blocks; `bad` marks a group holding a non-finite value.
__device__ __forceinline__ void packed_group_exponent(const float (&v)[4], int &e, bool &bad)
{
    unsigned mb = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t)
        mb = max(mb, __float_as_uint(v[t]) & 0x7FFFFFFFu);
    mb = max(mb, quad_xor1(mb));
    mb = max(mb, quad_xor2(mb));
    mb = max(mb, half_mirror(mb));
    mb = max_xor16(mb);
    mb = max_xor32(mb);
    bad = mb >= 0x7F800000u;
    e = 0;
    if (!bad && mb)
        frexpf(__uint_as_float(mb), &e);  // |x| < 2^e
}

// Integer formats, packed layout: the lane's A fragment for its own kstep
// (digit p = lane & 3 of the quad's 16 values, as reg_digits forms it) and,
// for ternary, the group correction split as hi * 2^16 + lo (zero for INT8).
template <Format F>
__device__ __forceinline__ v4i packed_digits(const float (&v)[4], int e, bool bad, int2 &cv)
{
    const uint32_t p = threadIdx.x & 3;
    long long corr = 0;
    unsigned vp[4];
    int u_prev = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        int val = bad ? 0 : int(rintf(ldexpf(v[t], 30 - e)));
        if constexpr (F == Format::Ternary) {
            // Field t of the nested masks (see the operand-field note).
            const int u = t == 0 ? val : (val + (1 << (2 * t - 1))) >> (2 * t);
            val = t == 0 ? u : u - u_prev;
            u_prev = u;
            corr += t < 3 ? (static_cast<long long>(u) << (2 * t))
                          : -(static_cast<long long>(u) << 6);
        }
        vp[t] = unsigned(val + 0x808080);
    }
    unsigned d[4], wd[4];
    byte_transpose<true>(vp, d);
    quad_transpose(d, p);
    if constexpr (F == Format::Ternary) {
        byte_transpose<false>(d, wd);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            wd[i] = d[i];
    }
    const unsigned flip = p ? 0x80808080u : 0u;
    cv = int2{0, 0};
    if constexpr (F == Format::Ternary) {
        corr += static_cast<long long>(quad_xor1(unsigned(corr))) |
                (static_cast<long long>(quad_xor1(unsigned(corr >> 32))) << 32);
        corr += static_cast<long long>(quad_xor2(unsigned(corr))) |
                (static_cast<long long>(quad_xor2(unsigned(corr >> 32))) << 32);
        corr += static_cast<long long>(half_mirror(unsigned(corr))) |
                (static_cast<long long>(half_mirror(unsigned(corr >> 32))) << 32);
        corr = sum_xor16(corr);
        corr = sum_xor32(corr);
        const long long lo = ((corr + 32768) & 65535) - 32768;
        cv = int2{int((corr - lo) >> 16), int(lo)};
    }
    return v4i{int(wd[0] ^ flip), int(wd[1] ^ flip), int(wd[2] ^ flip), int(wd[3] ^ flip)};
}

template <Format F>
struct WideGeo {
    // Lane loads per (tile, slice) and ksteps per lane load.
    static constexpr int loads = F == Format::Ternary ? 1 : F == Format::Nf4 ? 2 : 4;
    static constexpr int ksteps_per_load = F == Format::Int8 ? 1 : 4;
    static constexpr int ksteps = loads * ksteps_per_load;  // 4, 8, 4
};

// One decode token's attention output at k .. k + 3 (one head, head_dim a
// multiple of 4) merged from its key ranges' (m, l, acc) records by
// gqa_combine_kernel's formula: weights e^(m_s - M) over the non-empty
// ranges (l != 0), M their largest m, divided by the weighted sum of l.  The
// sums run serially in range order (the combine kernel's run as block
// reductions, so the two round differently in the last bits); a NaN in any
// record reaches the output.  Every record is loaded before any is used
// (one memory round trip).
__device__ __forceinline__ void gqa_merge4(const float *records, uint32_t ranges,
                                           uint32_t head_dim, uint32_t k, float (&v)[4])
{
    constexpr int S = int(kGqaMergeMaxRanges);
    const uint32_t head = k / head_dim, dim = k % head_dim;
    const uint32_t stride = head_dim + 2;
    const float *rec = records + size_t(head) * ranges * stride;
    float m[S], l[S];
    float2 lo[S], hi[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const bool live = uint32_t(s) < ranges;
        const float *r = rec + (live ? s : 0) * stride;
        m[s] = r[0];
        l[s] = live ? r[1] : 0.0f;
        // acc[dim .. dim + 3]: 8-byte aligned (stride and dim are even).
        lo[s] = *reinterpret_cast<const float2 *>(r + 2 + dim);
        hi[s] = *reinterpret_cast<const float2 *>(r + 4 + dim);
    }
    float maximum = -__builtin_inff();
#pragma unroll
    for (int s = 0; s < S; ++s)
        if (l[s] != 0.0f)
            maximum = fmaxf(maximum, m[s]);
    float denominator = 0.0f, acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < S; ++s) {
        if (l[s] == 0.0f)
            continue;  // an empty (or absent) range: weight 0, acc 0
        const float w = expf(m[s] - maximum);
        denominator += l[s] * w;
        acc[0] += lo[s].x * w;
        acc[1] += lo[s].y * w;
        acc[2] += hi[s].x * w;
        acc[3] += hi[s].y * w;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
        v[t] = acc[t] / denominator;
}

template <Format F, bool HALF, int P, int R, int W = 16, bool NORM = false, bool ARGMAX = false,
          bool MERGE = false>
__global__ __launch_bounds__(64 * W) void wide_row_kernel(StreamArgs a)
{
    static_assert(!MERGE || (R == 1 && !NORM), "the merge prologue: one tile per block");
    using ST = typename ScaleT<HALF>::type;
    constexpr int TS = W / P;                      // tiles per round
    constexpr int L = WideGeo<F>::loads;
    constexpr int KPL = WideGeo<F>::ksteps_per_load;
    constexpr int KSU = WideGeo<F>::ksteps;
    constexpr int NL = R * L;                       // lane loads per wave
    constexpr int AHW = NORM ? kWideAheadNorm : F == Format::Nf4 ? kWideAheadNf4 : kWideAhead;
    constexpr int AH = NL < AHW ? NL : AHW;
    constexpr int G = 2 * P;                        // 128-groups per tile
    constexpr bool NF4 = F == Format::Nf4;
    __shared__ float partial[TS * R * P * 16];
    // One block per tile below the head size: the small table.
    using LUT = LutLayout<R == 1 ? kSmallLutCopies : kStreamLutCopies>;
    __shared__ unsigned lut[NF4 ? 256 * 2 * LUT::copies : 1];
    __shared__ uint2 entries[NF4 ? 256 : 1];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t q = lane >> 4, j = lane & 15;
    const uint32_t part = wave % P, tslot = wave / P;
    const uint32_t tile0 = blockIdx.x * (TS * R) + tslot;
    auto tile_of = [&](int i) {
        const uint32_t t = tile0 + uint32_t(TS * i);
        return t < a.n_tiles ? t : a.n_tiles - 1;
    };

    // 1. The slice's activations: one float4 per lane.
    const uint32_t kx = NF4 ? 256 * part + 32 * ((lane >> 1) & 7) + 8 * q + 4 * (lane & 1)
                            : 256 * part + 64 * ((lane >> 2) & 3) + 16 * q + 4 * (lane & 3);
    const bool inb = kx < a.k;
    v4f xv;
    if constexpr (MERGE) {
        float mv[4];
        gqa_merge4(a.x, a.ranges, a.head_dim, inb ? kx : 0, mv);
        xv = v4f{mv[0], mv[1], mv[2], mv[3]};
    } else {
        xv = *reinterpret_cast<const v4f *>(a.x + (inb ? kx : 0));
    }
    v4f bv{0.0f, 0.0f, 0.0f, 0.0f}, wv{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (NORM) {
        if (a.b)
            bv = *reinterpret_cast<const v4f *>(a.b + (inb ? kx : 0));
        wv = *reinterpret_cast<const v4f *>(a.w + (inb ? kx : 0));
    }
    // 2. The group scales of this lane's combine (group 2p + q'/2, row j):
    // tile i's is loaded one tile ahead (the first two here).  Then the first
    // weight loads.  Byte offsets from the tile base are 32-bit
    // (try_wide_row keeps the codes below 4 GiB).
    const uint32_t my_group = 2 * part + (q >> 1);
    auto scale_of = [&](int i) {
        return reinterpret_cast<const ST *>(a.scales)[(tile_of(i) * G + my_group) * 16 + j];
    };
    ST sc[R];
    sc[0] = scale_of(0);
    if constexpr (R > 1)
        sc[1] = scale_of(1);
    __builtin_amdgcn_sched_barrier(0);
    v4u w[NL];
    auto issue = [&](auto n_tag) {
        constexpr int n = decltype(n_tag)::value;
        const uint32_t off = ((tile_of(n / L) * (P * L) + part * L + n % L) * 64 + lane) * 16;
        w[n] = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(a.tiles + off));
    };
    unroll_groups<AH>(issue);
    __builtin_amdgcn_sched_barrier(0);

    // 3. NF4: the code-byte table (as stream_nf4_kernel's).
    if constexpr (NF4) {
        if (threadIdx.x < 256)
            entries[threadIdx.x] = nf4_lut_entry(threadIdx.x);
        __syncthreads();
        for (uint32_t v = threadIdx.x; v < 256 * 2 * LUT::copies / 4; v += blockDim.x) {
            const uint2 e = entries[v / (2 * LUT::copies / 4)];
            reinterpret_cast<v4u *>(lut)[v] = v4u{e.x, e.y, e.x, e.y};
        }
    }

    // 4. The slice's operands and group constants.  NORM: every tile slot's
    // waves hold all of K, and each slot sums its slices' squares (wave
    // sums, then slice order).
    float v[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
        v[t] = inb ? xv[t] : 0.0f;
    if constexpr (NORM) {
        __shared__ float squares_part[W];
        float sv[4], squares = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            sv[t] = a.b ? v[t] + (inb ? bv[t] : 0.0f) : v[t];
            squares += sv[t] * sv[t];
        }
        squares = wave_sum_f(squares);
        if (lane == 0)
            squares_part[wave] = squares;
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int pp = 0; pp < P; ++pp)
            total += squares_part[tslot * P + pp];
        const float reciprocal = rms_reciprocal(total, a.k, a.epsilon);
#pragma unroll
        for (int t = 0; t < 4; ++t)
            v[t] = inb ? (sv[t] * reciprocal) * wv[t] : 0.0f;
    }
    int e;
    bool bad;
    packed_group_exponent(v, e, bad);
    typedef typename std::conditional<NF4, v8h, v4i>::type AT;
    AT af;
    float factor;
    int2 cv = int2{0, 0};
    if constexpr (NF4) {
        factor = bad ? __builtin_nanf("") : ldexpf(1.0f, e);
        const uint32_t h = lane & 1;
        unsigned mine[2], recv[2];
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
            const float v0 = bad ? 0.0f : ldexpf(v[2 * pr], -e);
            const float v1 = bad ? 0.0f : ldexpf(v[2 * pr + 1], -e);
            const _Float16 h0 = _Float16(v0), h1 = _Float16(v1);
            const _Float16 l0 = _Float16(v0 - float(h0)), l1 = _Float16(v1 - float(h1));
            const unsigned hi_pair = pack_halves(h0, h1), lo_pair = pack_halves(l0, l1);
            mine[pr] = h ? lo_pair : hi_pair;
            recv[pr] = quad_xor1(h ? hi_pair : lo_pair);  // the partner's half h
        }
        const v4u d = h ? v4u{recv[0], recv[1], mine[0], mine[1]}
                        : v4u{mine[0], mine[1], recv[0], recv[1]};
        af = __builtin_bit_cast(v8h, d);
    } else {
        factor = bad ? __builtin_nanf("") : ldexpf(1.0f, e - 30);
        af = packed_digits<F>(v, e, bad, cv);
    }
    // The combine of lane block q' uses group q' / 2 of the slice, whose
    // constants lanes 8 (q' / 2) .. hold.
    const int src_lane = 8 * int(q >> 1);
    const float my_factor = __shfl(factor, src_lane, 64);
    const int2 my_corr = int2{__shfl(cv.x, src_lane, 64), __shfl(cv.y, src_lane, 64)};
    // Operands per kstep: own fragment for the lane's kstep, zero otherwise.
    // NF4 takes two per kstep, in the k-slot order of nf4_entries: slots
    // (hi, lo) of code byte 2c and of byte 2c + 1 for operand c, so the A
    // operand repeats each activation pair for its hi and lo slots.
    // NF4 selects them per kstep from the lane's own pair (registers).
    const uint32_t own = NF4 ? j >> 1 : j >> 2;
    constexpr int OPS = NF4 ? 2 : 1;
    const v4u dq = __builtin_bit_cast(v4u, af);
    const v4u own0 = NF4 ? v4u{dq.x, dq.x, dq.y, dq.y} : dq;
    const v4u own1 = v4u{dq.z, dq.z, dq.w, dq.w};
    auto operand = [&](int s2, int o) {
        const v4u z{0, 0, 0, 0};
        return __builtin_bit_cast(AT, own == uint32_t(s2) ? (o == 0 ? own0 : own1) : z);
    };
    AT as[NF4 ? 1 : KSU][1];
    if constexpr (!NF4) {
#pragma unroll
        for (int s2 = 0; s2 < KSU; ++s2)
            as[s2][0] = operand(s2, 0);
    }
    if constexpr (NF4)
        __syncthreads();  // the table
    const unsigned copy_byte = 8 * LUT::spread * (lane % LUT::copies);
    const char *cells = reinterpret_cast<const char *>(lut);

    // NF4 B operands of one kstep's code word: the table entries (hi pair,
    // lo pair) of code bytes 0, 1 and of bytes 2, 3, each operand exactly
    // the two 8-byte reads (no register moves).
    auto nf4_entries = [&](unsigned word, v4u &b0, v4u &b1) {
        uint2 ent[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            // (code byte b) * 256 + copy_byte.
            const unsigned at =
                __builtin_amdgcn_perm(word, copy_byte, 0x0C0C0000u | ((4u + b) << 8)) >>
                LUT::shift;
            ent[b] = *reinterpret_cast<const uint2 *>(cells + at);
        }
        b0 = v4u{ent[0].x, ent[0].y, ent[1].x, ent[1].y};
        b1 = v4u{ent[2].x, ent[2].y, ent[3].x, ent[3].y};
    };
    // NF4: the table entries of kstep t are read TA ksteps ahead of its
    // products, into ring slot t % TA (the code words of those ksteps are
    // in loads already issued: TA <= KPL and AH >= 2).
    constexpr int NKS = NL * KPL;  // ksteps per wave
    constexpr int TA = NF4 ? (kNf4TableAhead < NKS ? kNf4TableAhead : NKS) : 1;
    static_assert(!NF4 || (TA <= KPL && AH >= 2), "NF4 table reads run ahead of the loads");
    v4u pb0[TA], pb1[TA];
    if constexpr (NF4) {
        unroll_groups<TA>([&](auto d_tag) {
            constexpr int d = decltype(d_tag)::value;
            nf4_entries(w[d / KPL][d % KPL], pb0[d], pb1[d]);
        });
    }

    // 5. The tiles: products of the slice, then the combine.
    typedef typename std::conditional<NF4, v4f, v4i>::type CT;
    unroll_groups<R>([&](auto i_tag) {
        constexpr int i = decltype(i_tag)::value;
        if constexpr (i + 2 < R)
            sc[i + 2] = scale_of(i + 2);
        CT acc = CT{};
        unroll_groups<L>([&](auto l_tag) {
            constexpr int l = decltype(l_tag)::value;
            constexpr int n = i * L + l;
            if constexpr (n + AH < NL)
                issue(std::integral_constant<int, n + AH>{});
            unroll_groups<KPL>([&](auto ks_tag) {
                constexpr int ks = decltype(ks_tag)::value;
                constexpr int s2 = l * KPL + ks;  // kstep within the slice
                if constexpr (F == Format::Int8) {
                    const v4u wv = w[n];
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        as[s2][0], v4i{int(wv.x), int(wv.y), int(wv.z), int(wv.w)}, acc, 0, 0, 0);
                } else if constexpr (F == Format::Ternary) {
                    const unsigned word = w[n][ks];
                    const v4i bw = v4i{int(word), int(word & 0xFCFCFCFCu),
                                       int(word & 0xF0F0F0F0u), int(word & 0xC0C0C0C0u)};
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(as[s2][0], bw, acc, 0, 0, 0);
                } else {
                    // This kstep's entries were read TA ksteps ago; read
                    // kstep t + TA's into the freed slot before the products.
                    constexpr int t = n * KPL + ks, slot = t % TA;
                    const v4u b0 = pb0[slot], b1 = pb1[slot];
                    if constexpr (t + TA < NKS)
                        nf4_entries(w[(t + TA) / KPL][(t + TA) % KPL], pb0[slot], pb1[slot]);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        operand(s2, 0), __builtin_bit_cast(v8h, b0), acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        operand(s2, OPS - 1), __builtin_bit_cast(v8h, b1), acc, 0, 0, 0);
                }
            });
            __builtin_amdgcn_sched_barrier(0);
        });
        float gsum;
        if constexpr (NF4) {
            // Rows 4q' + r: kstep 2q' + r / 2, half r % 2.  Add the group's
            // other two ksteps (lane block q' ^ 1).
            gsum = sum_xor16((acc.x + acc.y) + (acc.z + acc.w));
        } else {
            // Rows 4q' + r: digit r of kstep q'.  The group's two ksteps are
            // lane blocks q' and q' ^ 1; integer sums combine exactly.
            int d[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const auto pr = __builtin_amdgcn_permlane16_swap(unsigned(acc[r]), unsigned(acc[r]),
                                                                 false, false);
                d[r] = int(pr[0]) + int(pr[1]);
            }
            // |d[0]| < 2^21, so the pairs combine exactly in int32.
            const int hi = (d[0] << 8) + d[1] - my_corr.x;
            const int lo = (d[2] << 8) + d[3] - my_corr.y;
            gsum = float(hi) * 65536.0f + float(lo);
        }
        float total = gsum * (to_f32<HALF>(sc[i]) * my_factor);
        total = sum_xor32(total);  // the slice's two groups
        if (q == 0)
            partial[((tslot + TS * i) * P + part) * 16 + j] = total;
    });

    // 6. The slices of each tile, added in order; ARGMAX (with `argmax` set),
    // the block's greedy-selection candidate (non-finite outputs poison it).
    __syncthreads();
    float sum = 0.0f;
    uint32_t stored = UINT32_MAX;  // the output row this thread wrote
    if (threadIdx.x < uint32_t(TS * R * 16)) {
        const uint32_t tl = threadIdx.x / 16, r = threadIdx.x % 16;
        sum = partial[(tl * P) * 16 + r];
#pragma unroll
        for (int pp = 1; pp < P; ++pp)
            sum += partial[(tl * P + pp) * 16 + r];
        const uint32_t t = blockIdx.x * (TS * R) + (tl % TS) + TS * (tl / TS);
        const uint32_t row = t * 16 + r;
        if (t < a.n_tiles && row < a.n) {
            a.out[row] = sum;
            stored = row;
        }
    }
    if (ARGMAX && a.argmax) {  // uniform
        Candidate cand{-__builtin_inff(), UINT32_MAX, 0};
        if (stored != UINT32_MAX) {
            if (isfinite(sum)) {
                cand.value = sum;
                cand.index = stored;
            } else {
                cand.poisoned = 1;
            }
        }
        constexpr int CW = (TS * R * 16 + 63) / 64;  // waves holding candidates
        __shared__ Candidate wave_cand[CW];
        if (wave < uint32_t(CW)) {
#pragma unroll
            for (int offset = 32; offset > 0; offset >>= 1)
                merge(cand, __shfl_xor(cand.value, offset, 64),
                      __shfl_xor(cand.index, offset, 64), __shfl_xor(cand.poisoned, offset, 64));
            if (lane == 0)
                wave_cand[wave] = cand;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w2 = 1; w2 < CW; ++w2)
                merge(cand, wave_cand[w2].value, wave_cand[w2].index, wave_cand[w2].poisoned);
            a.argmax[blockIdx.x] = cand;
        }
    }
}

// Wide-matrix GEMV at two to eight activation rows, integer formats
// (launch_wide_rows: INT8, and ternary below the head size): the plan of
// wide_row_kernel (one wave per 256-k slice across R tiles, the
// slices' sums added in slice order through LDS) with the register
// prologue's fragment layout.  Lane 16q + 4b + p loads x[4f + b] at
// k = 256 part + 64 s + 16q + 4p + 0..3 for the slice's four ksteps s and
// forms digit p of them (reg_digits), so one MFMA per kstep, fragment and
// tile serves four rows; each of the slice's two 128-groups keeps its own
// accumulator.  Output lane block q holds batch 4f + q: the group sums,
// scales and slice order are wide_row_kernel's, so each row's result is the
// one-row kernel's bit for bit.  Rows at or beyond m read row 0 and are
// zeroed.  HS = 2 splits each slice into two 128-k pieces, one group each,
// on two waves (half the weight loads and digits per wave, none
// duplicated; a ternary piece reads half of each 16-byte lane load); the
// block adds the two pieces of a slice before adding the slices in order,
// the one-row kernel's sum.
template <Format F, bool HALF, int P, int R, int NF, int W = 16, int HS = 1, int SPW = 1>
__global__ __launch_bounds__(64 * W) void wide_rows_kernel(StreamArgs a)
{
    static_assert(F != Format::Nf4, "integer formats");
    static_assert(HS == 1 || HS == 2, "whole or half slices");
    static_assert(SPW == 1 || (HS == 1 && R == 1), "several slices per wave: one tile, whole slices");
    using ST = typename ScaleT<HALF>::type;
    // Ternary pieces read half of each 16-byte lane load (8 bytes: two
    // ksteps, one 128-group).
    constexpr bool HALFLOAD = F == Format::Ternary && HS == 2;
    constexpr int PW = P * HS / SPW;                // waves per tile
    constexpr int TS = W / PW;                      // tiles per round
    constexpr int LS = WideGeo<F>::loads;           // lane loads per (tile, slice)
    constexpr int L = HALFLOAD ? 1 : LS / HS;       // ... per (tile, piece)
    constexpr int KPL = HALFLOAD ? 2 : WideGeo<F>::ksteps_per_load;
    constexpr int NL = R * L * SPW;                 // lane loads per wave
    constexpr int AH = NL < kWideAhead ? NL : kWideAhead;
    constexpr int G = 2 * P;                        // 128-groups per tile
    constexpr int GW = 2 / HS;                      // 128-groups per piece
    constexpr int LB = Geo<F>::lb < 4 / HS ? Geo<F>::lb : 4 / HS;  // ksteps per digit block
    constexpr int NB = 4 / HS / LB;                 // digit blocks per piece
    using Blk = I8Block<F, 1, 1, NF, HALF, LB>;
    constexpr int MB = 4 * NF;                      // batch rows held
    __shared__ float partial[TS * R * PW * MB * 16];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t q = lane >> 4, j = lane & 15;
    const uint32_t wpart = wave % PW, tslot = wave / PW;
    const uint32_t tile0 = blockIdx.x * (TS * R) + tslot;
    auto tile_of = [&](int i) {
        const uint32_t t = tile0 + uint32_t(TS * i);
        return t < a.n_tiles ? t : a.n_tiles - 1;
    };

    // 1. The piece's activations: one float4 per kstep and fragment (K is
    // 256 P, so every address lies in the row).  With several slices per
    // wave (slice wpart * SPW + sp), each slice's values are loaded one
    // slice ahead of its digits.
    const uint32_t b = (lane >> 2) & 3;
    RegX<LB> rx[NF][NB];
    auto load_x = [&](uint32_t part) {
        const uint32_t off = (256 / HS) * part + 16 * q + 4 * (lane & 3);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const uint32_t row = 4 * f + b;
            const bool live = row < a.m;
            const float *xrow = a.x + size_t(live ? row : 0) * a.k + off;
#pragma unroll
            for (int bi = 0; bi < NB; ++bi)
#pragma unroll
                for (int kk = 0; kk < LB; ++kk) {
                    const v4f v = *reinterpret_cast<const v4f *>(xrow + 64 * (bi * LB + kk));
                    rx[f][bi].v[kk] = live ? v : v4f{0.0f, 0.0f, 0.0f, 0.0f};
                }
        }
    };
    load_x(wpart * SPW);
    // 2. The group scales of every tile and slice (this lane's row j), then
    // the first weight loads.
    ST sc[R * SPW][GW];
#pragma unroll
    for (int i = 0; i < R * SPW; ++i)
#pragma unroll
        for (int gs = 0; gs < GW; ++gs)
            sc[i][gs] = reinterpret_cast<const ST *>(
                a.scales)[(size_t(tile_of(SPW == 1 ? i : 0)) * G +
                           GW * (wpart * SPW + (SPW == 1 ? 0 : i)) + gs) *
                              16 +
                          j];
    __builtin_amdgcn_sched_barrier(0);
    v4u w[NL];
    auto issue = [&](auto n_tag) {
        constexpr int n = decltype(n_tag)::value;
        // SPW > 1 (one tile): load n is load n % L of slice n / L.
        const uint32_t part = SPW == 1 ? wpart : wpart * SPW + n / L;
        constexpr int ti = SPW == 1 ? n / L : 0;
        if constexpr (HALFLOAD) {
            typedef unsigned v2u __attribute__((ext_vector_type(2)));
            const v2u *src = reinterpret_cast<const v2u *>(
                                 reinterpret_cast<const v4u *>(a.tiles) +
                                 (size_t(tile_of(ti)) * (P * LS) + (part / 2) * LS) * 64 + lane) +
                             part % 2;
            const v2u u = __builtin_nontemporal_load(src);
            w[n] = v4u{u.x, u.y, 0u, 0u};
        } else {
            const v4u *src = reinterpret_cast<const v4u *>(a.tiles) +
                             (size_t(tile_of(ti)) * (P * LS) + part * L + n % L) * 64 + lane;
            w[n] = __builtin_nontemporal_load(src);
        }
    };
    unroll_groups<AH>(issue);
    __builtin_amdgcn_sched_barrier(0);

    // 3. Digits, group factors and corrections of the piece (of each slice
    // in turn), then 4. the tiles: products of the piece per group and the
    // combine.  Several slices per wave add in slice order.
    Blk blk[NB];
    float wave_sum[NF];
    unroll_groups<R * SPW>([&](auto i_tag) {
        constexpr int i = decltype(i_tag)::value;  // tile (SPW == 1) or slice
        if constexpr (SPW == 1 ? i == 0 : true) {
#pragma unroll
            for (int bi = 0; bi < NB; ++bi)
#pragma unroll
                for (int f = 0; f < NF; ++f)
                    reg_digits(rx[f][bi], blk[bi], f);
            if constexpr (SPW > 1 && i + 1 < SPW)
                load_x(wpart * SPW + i + 1);  // the next slice's values
        }
        v4i acc[GW][NF];
#pragma unroll
        for (int gs = 0; gs < GW; ++gs)
#pragma unroll
            for (int f = 0; f < NF; ++f)
                acc[gs][f] = v4i{0, 0, 0, 0};
        unroll_groups<L>([&](auto l_tag) {
            constexpr int l = decltype(l_tag)::value;
            constexpr int n = i * L + l;
            if constexpr (n + AH < NL)
                issue(std::integral_constant<int, n + AH>{});
#pragma unroll
            for (int ks = 0; ks < KPL; ++ks) {
                const int s2 = l * KPL + ks;  // kstep within the slice
                v4i bw;
                if constexpr (F == Format::Ternary) {
                    const unsigned word = w[n][ks];
                    bw = v4i{int(word), int(word & 0xFCFCFCFCu), int(word & 0xF0F0F0F0u),
                             int(word & 0xC0C0C0C0u)};
                } else {
                    const v4u wv = w[n];
                    bw = v4i{int(wv.x), int(wv.y), int(wv.z), int(wv.w)};
                }
#pragma unroll
                for (int f = 0; f < NF; ++f)
                    acc[s2 / 2][f] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        blk[s2 / LB].af[s2 % LB][f], bw, acc[s2 / 2][f], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            // Each group's product is rounded before the add (no fused
            // multiply-add), as the one-row kernel's cross-lane sum.
#pragma clang fp contract(off)
            float g[GW];
#pragma unroll
            for (int gs = 0; gs < GW; ++gs) {
                // Rows 4q + r: digit r of batch 4f + q.
                const v4i d = acc[gs][f];
                const int2 cv = blk[gs * 2 / LB].cv[gs % (LB / 2)][f];
                const float xf = blk[gs * 2 / LB].xf[gs % (LB / 2)][f];
                // |d.x| < 2^21, so the pairs combine exactly in int32.
                const int hi = (d.x << 8) + d.y - cv.x;
                const int lo = (d.z << 8) + d.w - cv.y;
                const float gsum = float(hi) * 65536.0f + float(lo);
                g[gs] = gsum * (to_f32<HALF>(sc[i][gs]) * xf);
            }
            const float value = GW == 2 ? g[0] + g[GW - 1] : g[0];
            if constexpr (SPW == 1)
                partial[(((tslot + TS * i) * PW + wpart) * MB + 4 * f + q) * 16 + j] = value;
            else
                wave_sum[f] = i == 0 ? value : wave_sum[f] + value;
        }
    });
    if constexpr (SPW > 1) {
#pragma unroll
        for (int f = 0; f < NF; ++f)
            partial[((tslot * PW + wpart) * MB + 4 * f + q) * 16 + j] = wave_sum[f];
    }

    // 5. The slices of each (tile, batch row), added in order (each slice
    // the sum of its pieces).
    __syncthreads();
    for (uint32_t v = threadIdx.x; v < uint32_t(TS * R * MB * 16); v += blockDim.x) {
        const uint32_t tl = v / (MB * 16), bb = (v / 16) % MB, r = v % 16;
        auto slice = [&](int pp) {
            const float *at = partial + ((tl * PW + HS * pp) * MB + bb) * 16 + r;
            return HS == 2 ? at[0] + at[MB * 16] : at[0];
        };
        float sum = slice(0);
#pragma unroll
        for (int pp = 1; pp < P / SPW; ++pp)
            sum += slice(pp);
        const uint32_t t = blockIdx.x * (TS * R) + (tl % TS) + TS * (tl / TS);
        const uint32_t row = t * 16 + r;
        if (bb < a.m && t < a.n_tiles && row < a.n)
            a.out[size_t(bb) * a.n + row] = sum;
    }
}

// One-row wide GEMV for the decode projections (m = 1): the packed one-row
// operand layout of wide_row_kernel with one block of P waves per row tile,
// each wave SPW consecutive 256-k slices (K = 256 P SPW), over S weight
// streams: one (Single), two (Pair, SwigluPair), or three row regions of
// one matrix (the convolution in-projection: rows c, h + c and 2h + c of
// channel c, finished by conv_step_kernel's arithmetic).  The activation
// transform forms x in the slices: Plain; AddRms (s = a + b, the block sums
// the squares of its waves in wave order, x = (s * reciprocal) * weight,
// block 0 writes s to the side output); Swiglu (x = silu(a) * b).  Each
// (stream, slice) sums its two 128-groups as wide_row_kernel; a wave adds
// its slices in order, and the block adds the waves in order.
struct WideArgs {
    XForm xform;  // Plain: a = x
    const uint8_t *tiles[2];
    const void *scales[2];
    float *out[2];
    uint32_t n, k;
    uint32_t stream_tiles;  // S = 3: region s starts at tile s * stream_tiles
    ConvStep conv;          // S = 3
};

template <Format F, bool HALF, int P, int SPW, int S, XKind PRO, Epilogue E>
__global__ __launch_bounds__(64 * P) void wide_one_kernel(WideArgs a)
{
    static_assert(S == 1 || S == 2 || S == 3, "one, two or three weight streams");
    static_assert((S == 2) == (E != Epilogue::Single), "two streams for the pair epilogues");
    using ST = typename ScaleT<HALF>::type;
    constexpr bool NF4 = F == Format::Nf4;
    constexpr int L = WideGeo<F>::loads;             // lane loads per (tile, slice)
    constexpr int KPL = WideGeo<F>::ksteps_per_load;
    constexpr int G = 2 * P * SPW;                   // 128-groups per tile
    __shared__ float partial[S * P * 16];
    __shared__ float squares_part[P];
    using LUT = LutLayout<kSmallLutCopies>;  // one block per tile
    __shared__ unsigned lut[NF4 ? 256 * 2 * LUT::copies : 1];
    __shared__ uint2 entries[NF4 ? 256 : 1];
    const uint32_t lane = threadIdx.x & 63, part = threadIdx.x >> 6;
    const uint32_t q = lane >> 4, j = lane & 15;
    const XForm &t = a.xform;
    auto tile_of = [&](int st) {
        return S == 3 ? blockIdx.x + uint32_t(st) * a.stream_tiles : blockIdx.x;
    };
    auto tiles_of = [&](int st) { return S == 3 ? a.tiles[0] : a.tiles[st]; };
    auto scales_of = [&](int st) { return S == 3 ? a.scales[0] : a.scales[st]; };

    // 1. The slices' activations (and transform operands): one float4 each.
    uint32_t kx[SPW];
    v4f av[SPW], bv[SPW], wv[SPW];
#pragma unroll
    for (int sp = 0; sp < SPW; ++sp) {
        const uint32_t slice = part * SPW + sp;
        kx[sp] = NF4 ? 256 * slice + 32 * ((lane >> 1) & 7) + 8 * q + 4 * (lane & 1)
                     : 256 * slice + 64 * ((lane >> 2) & 3) + 16 * q + 4 * (lane & 3);
        av[sp] = *reinterpret_cast<const v4f *>(t.a + kx[sp]);
        bv[sp] = wv[sp] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (PRO == XKind::Swiglu)
            bv[sp] = *reinterpret_cast<const v4f *>(t.b + kx[sp]);
        if constexpr (PRO == XKind::AddRms) {
            if (t.b)
                bv[sp] = *reinterpret_cast<const v4f *>(t.b + kx[sp]);
            wv[sp] = *reinterpret_cast<const v4f *>(t.w + kx[sp]);
        }
    }
    // 2. Group scales (group 2 slice + q / 2, row j) and every weight load.
    ST sc[S][SPW];
    v4u w[S][SPW][L];
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int sp = 0; sp < SPW; ++sp)
            sc[st][sp] = reinterpret_cast<const ST *>(scales_of(st))
                [(size_t(tile_of(st)) * G + 2 * (part * SPW + sp) + (q >> 1)) * 16 + j];
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int sp = 0; sp < SPW; ++sp)
#pragma unroll
            for (int l = 0; l < L; ++l)
                w[st][sp][l] = __builtin_nontemporal_load(
                    reinterpret_cast<const v4u *>(tiles_of(st)) +
                    (size_t(tile_of(st)) * (P * SPW * L) + (part * SPW + sp) * L + l) * 64 +
                    lane);

    // 3. NF4: the code-byte table (as wide_row_kernel's).
    if constexpr (NF4) {
        if (threadIdx.x < 256)
            entries[threadIdx.x] = nf4_lut_entry(threadIdx.x);
        __syncthreads();
        for (uint32_t v = threadIdx.x; v < 256 * 2 * LUT::copies / 4; v += blockDim.x) {
            const uint2 e = entries[v / (2 * LUT::copies / 4)];
            reinterpret_cast<v4u *>(lut)[v] = v4u{e.x, e.y, e.x, e.y};
        }
    }

    // 4. The transform.
    float v[SPW][4];
    if constexpr (PRO == XKind::AddRms) {
        v4f sv[SPW];
        float squares = 0.0f;
#pragma unroll
        for (int sp = 0; sp < SPW; ++sp) {
            sv[sp] = t.b ? av[sp] + bv[sp] : av[sp];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                squares += sv[sp][e] * sv[sp][e];
        }
        squares = wave_sum_f(squares);
        if (lane == 0)
            squares_part[part] = squares;
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int pp = 0; pp < P; ++pp)
            total += squares_part[pp];
        const float reciprocal = rms_reciprocal(total, a.k, t.epsilon);
#pragma unroll
        for (int sp = 0; sp < SPW; ++sp) {
            if (blockIdx.x == 0 && t.side)
                *reinterpret_cast<v4f *>(t.side + kx[sp]) = sv[sp];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[sp][e] = (sv[sp][e] * reciprocal) * wv[sp][e];
        }
    } else {
#pragma unroll
        for (int sp = 0; sp < SPW; ++sp)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[sp][e] = PRO == XKind::Swiglu ? silu_mul(av[sp][e], bv[sp][e]) : av[sp][e];
    }

    // 5. Operands and group constants per slice.  Lane block q's combine
    // uses group q / 2 of the slice, whose constants lanes 8 (q / 2) .. hold.
    typedef typename std::conditional<NF4, v8h, v4i>::type AT;
    const int src_lane = 8 * int(q >> 1);
    v4u dq[SPW];
    float my_factor[SPW];
    int2 my_corr[SPW];
#pragma unroll
    for (int sp = 0; sp < SPW; ++sp) {
        int e;
        bool bad;
        packed_group_exponent(v[sp], e, bad);
        float factor;
        int2 cv = int2{0, 0};
        if constexpr (NF4) {
            factor = bad ? __builtin_nanf("") : ldexpf(1.0f, e);
            const uint32_t h = lane & 1;
            unsigned mine[2], recv[2];
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {
                const float v0 = bad ? 0.0f : ldexpf(v[sp][2 * pr], -e);
                const float v1 = bad ? 0.0f : ldexpf(v[sp][2 * pr + 1], -e);
                const _Float16 h0 = _Float16(v0), h1 = _Float16(v1);
                const _Float16 l0 = _Float16(v0 - float(h0)), l1 = _Float16(v1 - float(h1));
                const unsigned hi_pair = pack_halves(h0, h1), lo_pair = pack_halves(l0, l1);
                mine[pr] = h ? lo_pair : hi_pair;
                recv[pr] = quad_xor1(h ? hi_pair : lo_pair);  // the partner's half h
            }
            dq[sp] = h ? v4u{recv[0], recv[1], mine[0], mine[1]}
                       : v4u{mine[0], mine[1], recv[0], recv[1]};
        } else {
            factor = bad ? __builtin_nanf("") : ldexpf(1.0f, e - 30);
            dq[sp] = __builtin_bit_cast(v4u, packed_digits<F>(v[sp], e, bad, cv));
        }
        my_factor[sp] = __shfl(factor, src_lane, 64);
        my_corr[sp] = int2{__shfl(cv.x, src_lane, 64), __shfl(cv.y, src_lane, 64)};
    }
    // Operand of kstep s2 (NF4: two per kstep, the lane's activation pair
    // repeated for its hi and lo slots): the own fragment, zero otherwise.
    const uint32_t own = NF4 ? j >> 1 : j >> 2;
    auto operand = [&](int sp, int s2, int o) {
        const v4u d = dq[sp];
        const v4u z{0, 0, 0, 0};
        const v4u pick = NF4 ? (o == 0 ? v4u{d.x, d.x, d.y, d.y} : v4u{d.z, d.z, d.w, d.w}) : d;
        return __builtin_bit_cast(AT, own == uint32_t(s2) ? pick : z);
    };
    if constexpr (NF4)
        __syncthreads();  // the table
    const unsigned copy_byte = 8 * LUT::spread * (lane % LUT::copies);
    const char *cells = reinterpret_cast<const char *>(lut);
    auto nf4_entries = [&](unsigned word, v4u &b0, v4u &b1) {
        uint2 ent[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const unsigned at =
                __builtin_amdgcn_perm(word, copy_byte, 0x0C0C0000u | ((4u + b) << 8)) >>
                LUT::shift;
            ent[b] = *reinterpret_cast<const uint2 *>(cells + at);
        }
        b0 = v4u{ent[0].x, ent[0].y, ent[1].x, ent[1].y};
        b1 = v4u{ent[2].x, ent[2].y, ent[3].x, ent[3].y};
    };

    // 6. Products per (stream, slice), the combine, the wave's slice sum.
#pragma unroll
    for (int st = 0; st < S; ++st) {
        float wave_total = 0.0f;
#pragma unroll
        for (int sp = 0; sp < SPW; ++sp) {
            typedef typename std::conditional<NF4, v4f, v4i>::type CT;
            CT acc = CT{};
            v4u nb0{}, nb1{};
            if constexpr (NF4)
                nf4_entries(w[st][sp][0][0], nb0, nb1);
#pragma unroll
            for (int l = 0; l < L; ++l)
#pragma unroll
                for (int ks = 0; ks < KPL; ++ks) {
                    const int s2 = l * KPL + ks;  // kstep within the slice
                    if constexpr (F == Format::Int8) {
                        const v4u wv2 = w[st][sp][l];
                        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            operand(sp, s2, 0),
                            v4i{int(wv2.x), int(wv2.y), int(wv2.z), int(wv2.w)}, acc, 0, 0, 0);
                    } else if constexpr (F == Format::Ternary) {
                        const unsigned word = w[st][sp][l][ks];
                        const v4i bw = v4i{int(word), int(word & 0xFCFCFCFCu),
                                           int(word & 0xF0F0F0F0u), int(word & 0xC0C0C0C0u)};
                        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(operand(sp, s2, 0), bw, acc,
                                                                    0, 0, 0);
                    } else {
                        const v4u b0 = nb0, b1 = nb1;
                        if (ks + 1 < KPL)
                            nf4_entries(w[st][sp][l][ks + 1], nb0, nb1);
                        else if (l + 1 < L)
                            nf4_entries(w[st][sp][l + 1][0], nb0, nb1);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            operand(sp, s2, 0), __builtin_bit_cast(v8h, b0), acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            operand(sp, s2, 1), __builtin_bit_cast(v8h, b1), acc, 0, 0, 0);
                    }
                }
            float gsum;
            if constexpr (NF4) {
                // Rows 4q' + r: kstep 2q' + r / 2, half r % 2; the group's
                // other two ksteps are lane block q' ^ 1.
                gsum = sum_xor16((acc.x + acc.y) + (acc.z + acc.w));
            } else {
                // Rows 4q' + r: digit r of kstep q'; the group's two ksteps
                // are lane blocks q' and q' ^ 1.
                int d[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const auto pr = __builtin_amdgcn_permlane16_swap(
                        unsigned(acc[r]), unsigned(acc[r]), false, false);
                    d[r] = int(pr[0]) + int(pr[1]);
                }
                const int hi = (d[0] << 8) + d[1] - my_corr[sp].x;
                const int lo = (d[2] << 8) + d[3] - my_corr[sp].y;
                gsum = float(hi) * 65536.0f + float(lo);
            }
            float total = gsum * (to_f32<HALF>(sc[st][sp]) * my_factor[sp]);
            total = sum_xor32(total);  // the slice's two groups
            wave_total = sp == 0 ? total : wave_total + total;
        }
        if (q == 0)
            partial[(st * P + part) * 16 + j] = wave_total;
    }

    // 7. The waves of each stream, added in order; the epilogue.
    __syncthreads();
    if (threadIdx.x < 16) {
        const uint32_t r = threadIdx.x;
        float sum[S];
#pragma unroll
        for (int st = 0; st < S; ++st) {
            sum[st] = partial[(st * P) * 16 + r];
#pragma unroll
            for (int pp = 1; pp < P; ++pp)
                sum[st] += partial[(st * P + pp) * 16 + r];
        }
        const uint32_t row = blockIdx.x * 16 + r;
        if constexpr (S == 3) {
            // Channel `row`: B, C and x of the in-projection, then the
            // one-token convolution (conv_step_kernel's arithmetic).
            const ConvStep &cv = a.conv;
            if (row < cv.hidden) {
                const uint32_t rows = cv.width - 1;
                const float u = sum[0] * sum[2];
                const float *taps = cv.kernel + uint64_t(row) * cv.width;
                float total = 0.0f;
                for (uint32_t tap = 0; tap < rows; ++tap)
                    total += taps[tap] * cv.history[uint64_t(tap) * cv.hidden + row];
                total += taps[rows] * u;
                for (uint32_t rr = 0; rr + 1 < rows; ++rr)
                    cv.next[uint64_t(rr) * cv.hidden + row] =
                        cv.history[uint64_t(rr + 1) * cv.hidden + row];
                if (rows)
                    cv.next[uint64_t(rows - 1) * cv.hidden + row] = u;
                cv.out[row] = total * sum[1];
            }
        } else if (row < a.n) {
            if constexpr (E == Epilogue::Single) {
                a.out[0][row] = sum[0];
            } else if constexpr (E == Epilogue::Pair) {
                a.out[0][row] = sum[0];
                a.out[1][row] = sum[1];
            } else {
                a.out[0][row] = silu_mul(sum[0], sum[1]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Repack canonical codes into tiles, and scales into [tile][group][16].
// ---------------------------------------------------------------------------
template <Format F>
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t *codes, uint8_t *tiles,
                                                     uint32_t n, uint32_t k, uint32_t k_pad,
                                                     uint32_t n_tiles)
{
    constexpr uint32_t KPL = Geo<F>::kpl, KSTEP = Geo<F>::kstep;
    const uint32_t loads_per_tile = k_pad / KSTEP / KPL;
    const size_t total = size_t(n_tiles) * loads_per_tile * 64;
    const uint32_t row_bytes = k / weights_per_byte(F);
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += size_t(gridDim.x) * 256) {
        const uint32_t lane = uint32_t(i % 64);
        const uint32_t u = uint32_t((i / 64) % loads_per_tile);
        const uint32_t tile = uint32_t(i / 64 / loads_per_tile);
        const uint32_t q = lane / 16, jj = lane % 16;
        const uint32_t row = tile * 16 + jj;
        // Padding decodes to weight 0 in every format.
        const unsigned pad = F == Format::Ternary ? 0x55555555u : F == Format::Nf4 ? 0x77777777u : 0u;
        unsigned out[4] = {pad, pad, pad, pad};
        if (row < n) {
            const uint8_t *src = codes + size_t(row) * row_bytes;
            if constexpr (F == Format::Int8) {
                const uint32_t byte0 = 64 * u + 16 * q;
                if (byte0 < row_bytes) {
                    uint4 v = *reinterpret_cast<const uint4 *>(src + byte0);
                    out[0] = v.x;
                    out[1] = v.y;
                    out[2] = v.z;
                    out[3] = v.w;
                }
            } else {
                // Ternary 64-wide and NF4 32-wide ksteps both span 16 code bytes.
                for (int kk = 0; kk < 4; ++kk) {
                    const uint32_t byte0 = 16 * (u * 4 + kk) + 4 * q;
                    if (byte0 < row_bytes)
                        out[kk] = *reinterpret_cast<const unsigned *>(src + byte0) ^
                                  (F == Format::Ternary ? 0x80808080u : 0u);  // field 3 + 2
                }
            }
        }
        reinterpret_cast<uint4 *>(tiles)[i] = uint4{out[0], out[1], out[2], out[3]};
    }
}

template <bool HALF>
__global__ __launch_bounds__(256) void tile_scales_kernel(const float *scales, void *out,
                                                          uint32_t n, uint32_t groups,
                                                          uint32_t groups_pad, uint32_t n_tiles)
{
    const size_t total = size_t(n_tiles) * groups_pad * 16;
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += size_t(gridDim.x) * 256) {
        const uint32_t jj = uint32_t(i % 16);
        const uint32_t g = uint32_t((i / 16) % groups_pad);
        const uint32_t tile = uint32_t(i / 16 / groups_pad);
        const uint32_t row = tile * 16 + jj;
        const float v = (row < n && g < groups) ? scales[size_t(row) * groups + g] : 0.0f;
        if constexpr (HALF)
            reinterpret_cast<__half *>(out)[i] = __float2half(v);
        else
            reinterpret_cast<float *>(out)[i] = v;
    }
}

unsigned grid_for(size_t count)
{
    size_t blocks = (count + 255) / 256;
    return unsigned(blocks < 65536 ? (blocks ? blocks : 1) : 65536);
}

struct Plan {
    int tiles_per_block;
    int waves;
};

// Tiles per block T and waves per block W (which split K).  Prefer the widest
// T that still yields >= 2048 waves; each wave covers whole loop blocks.
// `wide` tries 8 waves before 4, which halves each wave's share of the
// in-kernel prologue (used when the narrower plan's share is too large).
Plan plan_for(uint32_t n_tiles, uint32_t ksteps, uint32_t lb, int max_t, bool wide)
{
    auto fits = [&](uint32_t w) { return ksteps % (w * lb) == 0; };
    const int order[2] = {wide ? 8 : 4, wide ? 4 : 8};
    for (int t : {4, 2, 1}) {
        if (t > max_t || n_tiles % t)
            continue;
        for (int w : order)
            if (fits(w) && uint64_t(n_tiles / t) * w >= 2048)
                return Plan{t, w};
    }
    for (int w : {8, 6, 4, 3, 2, 1})
        if (fits(w))
            return Plan{1, w};
    return Plan{1, 1};
}

// Small-N shapes fall back to one tile per block and 8 waves over K with too
// few waves to fill the chip (n_tiles * 8 < 2048): there 16 waves per block
// halve every wave's K range (2048 x 8192 INT8 at one row: 9.48 -> 8.13 us;
// 2048 x 2048 NF4: 5.13 -> 4.63 us).  Only kernels declared for 1024 lanes
// take it (one tile, one stream, one fragment; separate or register
// prologue).
constexpr int kDeepWaves = 16;
// Largest grid (blocks) that takes the two-part K split.
constexpr uint32_t kSplitMaxBlocks = 128;
// Row tiles from which an INT8 product at one or two rows is an LM head
// (65536 rows: 4096 tiles) and streams one tile per block.
constexpr uint32_t kHeadTiles = 4096;
constexpr uint32_t kNf4MidTiles = 1024;

// Whether float ranges [a, a + na) and [b, b + nb) share memory.
bool overlaps(const float *a, size_t na, const float *b, size_t nb)
{
    return a < b + nb && b < a + na;
}
Plan deepen(Plan p, uint32_t n_tiles, uint32_t ksteps, uint32_t lb)
{
    if (p.tiles_per_block == 1 && p.waves == 8 && uint64_t(n_tiles) * 8 < 2048 &&
        ksteps % (kDeepWaves * lb) == 0)
        p.waves = kDeepWaves;
    return p;
}

template <int S, int NB>
size_t reduce_lds_bytes(int waves, int t)
{
    return size_t(waves) * S * t * NB * 64 * sizeof(float);
}

// Kernel instantiations by prologue: pro < 0 is the separate prologue
// kernel, otherwise the in-kernel one with that XKind.  Single products
// serve every kind, the two-stream epilogues the plain and norm prologues
// (fused_kind_served).
bool fused_kind_served(Epilogue e, XKind kind)
{
    return e == Epilogue::Single || kind == XKind::Plain || kind == XKind::AddRms;
}

template <Format F, int T, int S, int NF, bool HALF, Epilogue E, int PRO>
void launch_i8_kernel(hipStream_t stream, const MfmaArgs &args, unsigned blocks, int waves)
{
    size_t lds = reduce_lds_bytes<S, NF>(waves, T);
    if constexpr (PRO >= 0 && PRO < kRegPro)
        lds += fused_bytes(args.k_pad, args.m);
    gemv_i8_kernel<F, T, S, NF, HALF, E, PRO><<<blocks, 64 * waves, lds, stream>>>(args);
}

template <Format F, int T, int S, int NF, bool HALF, Epilogue E>
void launch_i8_pro(hipStream_t stream, const MfmaArgs &args, unsigned blocks, int waves, int pro)
{
    if constexpr (NF == 1) {
        switch (pro) {
        case kRegPro:
            return launch_i8_kernel<F, T, S, NF, HALF, E, kRegPro>(stream, args, blocks, waves);
        case kRegPro + int(XKind::AddRms):
            return launch_i8_kernel<F, T, S, NF, HALF, E, kRegPro + int(XKind::AddRms)>(
                stream, args, blocks, waves);
        case int(XKind::Plain):
            return launch_i8_kernel<F, T, S, NF, HALF, E, 0>(stream, args, blocks, waves);
        case int(XKind::AddRms):
            return launch_i8_kernel<F, T, S, NF, HALF, E, 1>(stream, args, blocks, waves);
        case int(XKind::Swiglu):
            if constexpr (E == Epilogue::Single)
                return launch_i8_kernel<F, T, S, NF, HALF, E, 2>(stream, args, blocks, waves);
            break;
        default:
            break;
        }
    } else if constexpr (S == 1) {
        // Two fragments: gemv_i8_format picks the register prologue only for
        // single products, else the separate one (pro < 0).
        if (pro == kRegPro)
            return launch_i8_kernel<F, T, S, NF, HALF, E, kRegPro>(stream, args, blocks, waves);
    }
    launch_i8_kernel<F, T, S, NF, HALF, E, -1>(stream, args, blocks, waves);
}

template <Format F, int T, int S, int NF, bool HALF>
void launch_i8(hipStream_t stream, const MfmaArgs &args, Epilogue e, unsigned blocks, int waves,
               int pro)
{
    if constexpr (S == 1)
        launch_i8_pro<F, T, 1, NF, HALF, Epilogue::Single>(stream, args, blocks, waves, pro);
    else if (e == Epilogue::Pair)
        launch_i8_pro<F, T, 2, NF, HALF, Epilogue::Pair>(stream, args, blocks, waves, pro);
    else
        launch_i8_pro<F, T, 2, NF, HALF, Epilogue::SwigluPair>(stream, args, blocks, waves, pro);
}

template <Format F, int T, int S>
void launch_i8_nf(hipStream_t stream, const MfmaArgs &args, Epilogue e, unsigned blocks, int waves,
                  int nf, bool half, int pro)
{
    if (nf == 1) {
        if (half)
            launch_i8<F, T, S, 1, true>(stream, args, e, blocks, waves, pro);
        else
            launch_i8<F, T, S, 1, false>(stream, args, e, blocks, waves, pro);
    } else {
        // Two fragments: the separate prologue or the plain register one
        // (the LDS and norm prologues serve one fragment only).
        if (half)
            launch_i8<F, T, S, 2, true>(stream, args, e, blocks, waves, pro);
        else
            launch_i8<F, T, S, 2, false>(stream, args, e, blocks, waves, pro);
    }
}

template <int T, int S, bool HALF, Epilogue E, int PRO>
void launch_nf4_kernel(hipStream_t stream, const MfmaArgs &args, unsigned blocks, int waves)
{
    size_t lds = reduce_lds_bytes<S, 2>(waves, T);
    if constexpr (PRO >= 0 && PRO < kRegPro)
        lds += fused_bytes_nf4(args.k_pad, args.m);
    gemv_nf4_kernel<T, S, HALF, E, PRO><<<blocks, 64 * waves, lds, stream>>>(args);
}

template <int T, int S, bool HALF, Epilogue E>
void launch_nf4_pro(hipStream_t stream, const MfmaArgs &args, unsigned blocks, int waves, int pro)
{
    switch (pro) {
    case kRegPro:
        return launch_nf4_kernel<T, S, HALF, E, kRegPro>(stream, args, blocks, waves);
    case int(XKind::Plain):
        return launch_nf4_kernel<T, S, HALF, E, 0>(stream, args, blocks, waves);
    case int(XKind::AddRms):
        return launch_nf4_kernel<T, S, HALF, E, 1>(stream, args, blocks, waves);
    case int(XKind::Swiglu):
        if constexpr (E == Epilogue::Single)
            return launch_nf4_kernel<T, S, HALF, E, 2>(stream, args, blocks, waves);
        break;
    default:
        break;
    }
    launch_nf4_kernel<T, S, HALF, E, -1>(stream, args, blocks, waves);
}

template <int T, int S>
void launch_nf4_variant(hipStream_t stream, const MfmaArgs &args, Epilogue e, unsigned blocks,
                        int waves, bool half, int pro)
{
    auto go = [&](auto half_tag) {
        constexpr bool H = decltype(half_tag)::value;
        if constexpr (S == 1)
            launch_nf4_pro<T, 1, H, Epilogue::Single>(stream, args, blocks, waves, pro);
        else if (e == Epilogue::Pair)
            launch_nf4_pro<T, 2, H, Epilogue::Pair>(stream, args, blocks, waves, pro);
        else
            launch_nf4_pro<T, 2, H, Epilogue::SwigluPair>(stream, args, blocks, waves, pro);
    };
    if (half)
        go(std::true_type{});
    else
        go(std::false_type{});
}

struct Scratch {
    void *afrag;
    float *xf;
    int2 *corr;
};

Scratch carve(void *scratch, uint32_t k_pad)
{
    // afrag: k_pad * 16 bytes per 4-batch integer fragment (two fragments at
    // most); the f16 NF4 fragment takes k_pad * 32 bytes.  Same bound.
    char *p = static_cast<char *>(scratch);
    Scratch s;
    s.afrag = p;
    p += size_t(k_pad) * 32;
    s.xf = reinterpret_cast<float *>(p);
    p += size_t(8) * (k_pad / 128) * sizeof(float);
    s.corr = reinterpret_cast<int2 *>(p);
    return s;
}

// Largest grid that takes the in-kernel prologue (see gemv_i8_format).
constexpr unsigned kFusedMaxBlocks = 512;

// Tiles of the call: one stream's, or every segment's (each padded to 64
// rows as repacked).  Segment first-block table for T = 1.
uint32_t call_tiles(const PackedCall &call)
{
    if (!call.segments)
        return pad_to(call.n, 64) / 16;
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < call.segments; ++i)
        tiles += pad_to(call.seg_n[i], 64) / 16;
    return tiles;
}

void set_segments(MfmaArgs &args, const PackedCall &call)
{
    args.segments = call.segments;
    uint32_t first = 0;
    for (uint32_t i = 0; i < call.segments; ++i) {
        args.seg_first[i] = first;
        args.seg_tiles[i] = call.seg[i].tiles;
        args.seg_scales[i] = call.seg[i].tiled_scales;
        args.seg_out[i] = call.seg_out[i];
        args.seg_n[i] = call.seg_n[i];
        first += pad_to(call.seg_n[i], 64) / 16;
    }
}

template <int NF, int KL>
void launch_stream_ternary(hipStream_t stream, const StreamArgs &args, bool half)
{
    // Waves per block: the most that still leave at least kStreamMinBlocks
    // blocks (one tile each wave), so small grids spread over the CUs.
    auto go = [&](auto w_tag) {
        constexpr int W = decltype(w_tag)::value;
        const unsigned blocks = (args.n_tiles + W - 1) / W;
        if (half)
            stream_ternary_kernel<NF, KL, true, W><<<blocks, 64 * W, 0, stream>>>(args);
        else
            stream_ternary_kernel<NF, KL, false, W><<<blocks, 64 * W, 0, stream>>>(args);
    };
    // (n_tiles >= kStreamMinTiles, so at least 192 blocks of four waves.)
    // Measured at 16384 x 1024, one row: 16 waves per block 5.3 us, 4 waves
    // 4.6-4.8 us.
    static_assert(kStreamMinTiles >= 3 * kStreamMinBlocks && kStreamTwoRowMinTiles >= 512,
                  "at least 192 blocks (128 at two rows)");
    if (args.n_tiles >= 16 * kStreamMinBlocks)
        go(std::integral_constant<int, 16>{});
    else if (args.n_tiles >= 8 * kStreamMinBlocks)
        go(std::integral_constant<int, 8>{});
    else
        go(std::integral_constant<int, 4>{});
}

template <int MB, int KL>
void launch_stream_ternary_rows(hipStream_t stream, const StreamArgs &args, bool half)
{
    // Waves per block as launch_stream_ternary.
    auto go = [&](auto w_tag) {
        constexpr int W = decltype(w_tag)::value;
        const unsigned blocks = (args.n_tiles + W - 1) / W;
        if (half)
            stream_ternary_rows_kernel<MB, KL, true, W><<<blocks, 64 * W, 0, stream>>>(args);
        else
            stream_ternary_rows_kernel<MB, KL, false, W><<<blocks, 64 * W, 0, stream>>>(args);
    };
    if (args.n_tiles >= 16 * kStreamMinBlocks)
        go(std::integral_constant<int, 16>{});
    else if (args.n_tiles >= 8 * kStreamMinBlocks)
        go(std::integral_constant<int, 8>{});
    else
        go(std::integral_constant<int, 4>{});
}

// Serves the call with the streaming kernel when it applies; false leaves
// it to the K-split plans.
bool try_stream_ternary(hipStream_t stream, const PackedCall &call, uint32_t n_tiles)
{
    const uint32_t k_pad = pad_to(call.k, 256);
    const uint32_t kl = k_pad / 256;
    if (call.separate_prologue || call.xform.kind != XKind::Plain || call.segments ||
        call.epilogue != Epilogue::Single || call.m == 0 || call.m > 8 ||
        n_tiles < (call.m == 2 ? kStreamTwoRowMinTiles : kStreamMinTiles) || (kl != 4 && kl != 8) ||
        reinterpret_cast<uintptr_t>(call.x) % 16 != 0)
        return false;
    StreamArgs args{};
    args.x = call.x;
    args.tiles = call.a.tiles;
    args.scales = call.a.tiled_scales;
    args.out = call.out_a;
    args.m = call.m;
    args.n = call.n;
    args.k = call.k;
    args.n_tiles = n_tiles;
    const bool half = call.a.tiled_half;
    auto go = [&](auto nf_tag) {
        constexpr int NF = decltype(nf_tag)::value;
        if (kl == 4)
            launch_stream_ternary<NF, 4>(stream, args, half);
        else
            launch_stream_ternary<NF, 8>(stream, args, half);
    };
    if (call.m <= 2) {
        auto rows = [&](auto mb_tag) {
            constexpr int MB = decltype(mb_tag)::value;
            if (kl == 4)
                launch_stream_ternary_rows<MB, 4>(stream, args, half);
            else
                launch_stream_ternary_rows<MB, 8>(stream, args, half);
        };
        if (call.m == 1)
            rows(std::integral_constant<int, 1>{});
        else
            rows(std::integral_constant<int, 2>{});
    } else if (call.m <= 4) {
        go(std::integral_constant<int, 1>{});
    } else {
        go(std::integral_constant<int, 2>{});
    }
    return true;
}

// Tiles per wave (R) of wide_row_kernel, measured at 65536 rows, one row
// (us per launch, 1 GiB rotation): INT8 K = 2048 R = 4 21.8-22.4 against
// R = 8 22.3-22.7 (the four-tile K-split plan 24.2-29.0); K = 1024 R = 2-4
// 12.1-12.5.  NF4 K = 2048 R = 8 14.8-20.4 against R = 4 18.6-22.3 (two
// blocks per CU do not fit its registers) and the streaming kernel
// 18.4-21.8; K = 1024 R = 4 8.9-10.5 against 10.9-12.1.  Ternary K = 1024
// R = 4 5.6-5.9 against the rows kernel's 5.9-6.2; at K = 2048 the rows
// kernel (7.5 us) beats R = 8 (8.1-8.6), which keeps it.
// Below kHeadTiles row tiles (the decode projections) one tile per wave and
// one block of P waves per tile (W = P, R = 1).  Measured at one row (us per
// launch, rotation) against the plans they replace: ternary 2048 x 2048
// 4.10 -> 3.29-3.37, 8192 x 2048 5.84 -> 4.07, 4608 x 1024 4.26 -> 3.37
// (K-split register prologue); NF4 2048 x 2048 4.97 -> 3.68, 8192 x 2048
// 7.13 -> 4.88 (f32 vector GEMV); INT8 8192 x 2048 6.09 -> 4.84, 2048 x 2048
// 3.71 -> 3.59.  LFM2 greedy decode, 1.2B shape 2073 -> 2168 tok/s (op by
// op 1439 -> 1585), 350M 3053 -> 3047 (op by op 1741 -> 1923).
// Returns the number of argmax candidates written (one per block), 0 where
// the launched kernel writes none.
template <Format F, bool HALF, int P>
unsigned launch_wide_row(hipStream_t stream, const StreamArgs &args, bool norm, bool merge)
{
    constexpr int TS = 16 / P;
    // NF4 from kNf4MidTiles tiles to below the head size: blocks of 16
    // waves, R tiles per wave with R the largest of 4, 2, 1 that leaves at
    // least 256 blocks (the 32-copy table filled once per R rounds).
    // Measured at one row (us per launch, A/B on one device) against one
    // block per tile: 16384 x 2048 7.1 -> 5.9, 32768 x 2048 12.0 -> 8.5,
    // 49152 x 2048 16.4-18.5 -> 14.6-15.3, 32768 x 1024 7.5 -> 6.0, 16384 x
    // 1024 the same; INT8 measured the same or slower (32768 x 1024 6.9 ->
    // 7.2, 49152 x 2048 16.4 -> 17.8) and keeps one block per tile, and so
    // does NF4 below 1024 tiles (R = 1 on 16-wave blocks: 12288 x 2048 6.1
    // -> 7.2, 10240 x 2048 6.0 -> 7.0, 8192 x 1024 3.9 -> 4.6).
    if constexpr (F == Format::Nf4) {
        if (args.n_tiles < kHeadTiles && args.n_tiles >= kNf4MidTiles && !merge) {
            auto mid = [&](auto r_tag) {
                constexpr int RM = decltype(r_tag)::value;
                const unsigned blocks = (args.n_tiles + TS * RM - 1) / (TS * RM);
                wide_row_kernel<F, HALF, P, RM><<<blocks, 1024, 0, stream>>>(args);
                return args.argmax ? 0u : blocks;
            };
            if (args.n_tiles >= 4 * TS * 256)
                return mid(std::integral_constant<int, 4>{});
            if (args.n_tiles >= 2 * TS * 256)
                return mid(std::integral_constant<int, 2>{});
            return mid(std::integral_constant<int, 1>{});
        }
    }
    if (args.n_tiles < kHeadTiles) {
        if (merge)
            wide_row_kernel<F, HALF, P, 1, P, false, false, true><<<args.n_tiles, 64 * P, 0,
                                                                   stream>>>(args);
        else
            wide_row_kernel<F, HALF, P, 1, P><<<args.n_tiles, 64 * P, 0, stream>>>(args);
        return 0;
    }
    // Tiles per wave at the head: eight at K = 2048, four at K = 1024 (one
    // row, us per launch, A/B on one device: INT8 65536 x 2048 R = 4 / 8
    // 21.1-21.2 / 20.9-21.0; 65536 x 1024 R = 2 / 4 / 8 12.0 / 11.6 / 13.5,
    // ternary 6.5 / 5.7-5.8 / 7.4; R = 1 slower everywhere).
    constexpr int R = P == 8 ? 8 : 4;
    const unsigned blocks = (args.n_tiles + TS * R - 1) / (TS * R);
    // The norm comes with the argmax candidates (the LM head of the fused
    // decode step); NF4 heads keep the separate norm and selection (folded,
    // the 128-VGPR NF4 head spilled).
    if constexpr (F != Format::Nf4) {
        if (norm) {
            wide_row_kernel<F, HALF, P, R, 16, true, true><<<blocks, 1024, 0, stream>>>(args);
            return blocks;
        }
    }
    wide_row_kernel<F, HALF, P, R><<<blocks, 1024, 0, stream>>>(args);
    return args.argmax ? 0u : blocks;
}

// At the head size, tiles per wave R = P, so each block's 16 waves cover 16
// tiles.  Measured at 65536 rows, INT8, B = 2 / 4 / 8 (us per launch, 1 GiB
// rotation): K = 2048 R = 8 22.1 / 22.0 / 22.9, R = 4 22.6 / 23.0 / 25.3,
// R = 2 24.1 / 24.7 / 30.3 (the K-split plans 28.4 / 25.6 / 28.7); K = 1024
// R = 4 12.3 / 12.5 / 13.3, R = 8 15.1 / 15.2 / 16.1.  The ternary head
// stays on the streaming kernels: its digit prologue (the field
// telescoping), repeated by every wave of a slice, cost more than it saved
// (65536 x 2048, B = 2 / 4 / 8: R = 8 8.9 / 9.3 / 14.2 us against 8.1 / 8.9
// / 14.3).

template <Format F, bool HALF, int P, int NF>
void launch_wide_rows(hipStream_t stream, const StreamArgs &args)
{
    // Below the head size one block of P waves per tile, as wide_row_kernel.
    // Measured at B = 2 / 4 / 8 (us per launch) against the K-split
    // register-prologue plans: ternary 2048 x 2048 4.15 / 4.18 / 6.13 ->
    // 3.82 / 3.83 / 5.34, 8192 x 2048 5.79 / 5.76 / 9.00 -> 5.33 / 5.38 /
    // 8.31, 4608 x 1024 4.24 / 4.25 / 6.12 -> 3.78 / 3.75 / 5.39; INT8
    // 2048 x 2048 3.74 / 3.87 / 5.82 -> 3.69 / 3.71 / 4.86, 8192 x 2048 6.07
    // / 6.22 / 8.16 -> 5.05 / 5.14 / 7.12 (1024 x 1024: 3.25 / 3.22 / 3.94 ->
    // 3.51 / 3.46 / 3.70).
    if (args.n_tiles < kHeadTiles) {
        // Two waves per slice, one 128-k piece each.  Measured at B = 2 / 4
        // / 8 (us per launch, A/B on one device) against one wave per
        // slice: INT8 2048 x 2048 3.84 / 3.96 / 4.84 -> 3.62 / 3.53 / 4.31,
        // 4608 x 1024 - / 3.78 / 4.41 -> - / 3.48 / 4.15, 8192 x 2048 5.1 /
        // 5.1 / 7.27 -> 5.1 / 5.1 / 6.64, 1024 x 1024 the same (B = 5 at
        // 2048 x 2048 4.81 -> 4.27-4.48); ternary (against the fragments of
        // a slice split over two waves at five to eight rows) 1024 x 1024
        // 3.73 / - / 3.93 -> 3.48 / - / 3.7-4.0, 4608 x 1024 3.95 / 3.98 /
        // 5.27 -> 3.68 / 3.73 / 5.07, 2048 x 2048 3.93 / 4.04 / 5.45 -> 3.82
        // / 3.91 / 5.24, 8192 x 2048 5.37 / 5.58 / 8.49 -> 5.40 / 5.46 /
        // 8.20.
        // INT8 from 512 blocks' worth of tiles at two tiles per wave (1024
        // tiles at K = 2048, 2048 at K = 1024) to below the head size:
        // blocks of 16 waves, two tiles per wave up to 256 blocks, four
        // beyond.  Measured at B = 2 / 4-5 / 8 (us per launch, A/B on one
        // device) against one block per tile: 16384 x 2048 8.5 / 8.6 / 11.4
        // -> 7.7 / 7.8 / 8.8, 20480 x 2048 10.1 / 13.2 (B = 5) / - -> 9.3 /
        // 10.5 / -, 24576 x 2048 11.5 / 16.2 (B = 5) / - -> 10.2 / 11.1 / -,
        // 32768 x 2048 14.6 / - / 21.2-23.6 -> 12.2 / - / 13.2, 40960 x
        // 2048 - / 18.4-19.6 / 26.5-29.3 -> - / 18.3 / 21.1, 32768 x 1024
        // at B = 8 11.2 -> 8.8, 49152 x 1024 at B = 4 11.1 -> 10.4; one
        // tile per wave at 16384 x 1024 measured slower (B = 2 / 4 / 8 4.9
        // / 5.0 / 6.5 -> 5.4 / 5.4 / 7.5), and 320 blocks of two tiles per
        // wave slower than 160 of four (20480 x 2048, B = 5 10.5 -> 14.2).
        constexpr int TS = 16 / P;
        if (F != Format::Int8 || args.n_tiles < 2 * TS * 256) {
            wide_rows_kernel<F, HALF, P, 1, NF, 2 * P, 2><<<args.n_tiles, 128 * P, 0, stream>>>(
                args);
            return;
        }
        if constexpr (F == Format::Int8) {
            auto mid = [&](auto r_tag) {
                constexpr int RM = decltype(r_tag)::value;
                const unsigned blocks = (args.n_tiles + TS * RM - 1) / (TS * RM);
                wide_rows_kernel<F, HALF, P, RM, NF><<<blocks, 1024, 0, stream>>>(args);
            };
            if (args.n_tiles <= 2 * TS * 256)
                mid(std::integral_constant<int, 2>{});
            else
                mid(std::integral_constant<int, 4>{});
        }
        return;
    }
    constexpr int R = P;
    constexpr int TS = 16 / P;
    const unsigned blocks = (args.n_tiles + TS * R - 1) / (TS * R);
    wide_rows_kernel<F, HALF, P, R, NF><<<blocks, 1024, 0, stream>>>(args);
}

// Serves products at K = 1024 or 2048: one row with wide_row_kernel, two
// to eight rows with wide_rows_kernel (INT8, and ternary below the head
// size); false leaves it to the other plans.  The ternary head keeps the
// streaming kernels at K = 2048 and from two rows.
template <Format F>
bool try_wide_row(hipStream_t stream, const PackedCall &call, uint32_t n_tiles)
{
    const bool head = n_tiles >= kHeadTiles;
    const uint32_t max_m = F == Format::Int8 || (F == Format::Ternary && !head) ? 8 : 1;
    const XForm &t = call.xform;
    auto aligned = [](const void *ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
    // The add + RMS norm: one row at the head size (the LM head after the
    // last block), no side output.
    const bool norm = t.kind == XKind::AddRms;
    if (norm && (F == Format::Nf4 || !head || call.m != 1 || t.side || !t.w || !aligned(t.w) ||
                 (t.b && !aligned(t.b))))
        return false;
    // The attention merge: one row below the head size (an attention output
    // projection), at most kGqaMergeMaxRanges ranges of whole heads.
    const bool merge = t.kind == XKind::GqaMerge;
    if (merge && (head || call.m != 1 || t.ranges == 0 || t.ranges > kGqaMergeMaxRanges ||
                  t.head_dim == 0 || t.head_dim % 4 || call.k % t.head_dim))
        return false;
    const float *x = norm || merge ? t.a : call.x;
    // INT8, K = 8192 at two to four rows below the head size: sixteen waves
    // of two slices each (wide_rows_kernel SPW = 2).  Measured (us per
    // launch, A/B on one device) against the K-split plans: 2048 x 8192 B =
    // 2 / 4 8.43 / 8.89 -> 7.69 / 7.89, 8192 x 8192 B = 4 16.4 -> 15.9; at
    // eight rows slower (9.8 -> 11.6), and slower for ternary at every row
    // count (B = 2 7.45 -> 8.26, B = 8 8.65 -> 14.5).
    const bool k8192 = F == Format::Int8 && call.k == 8192 && call.m > 1 && call.m <= 4 && !head;
    if (call.separate_prologue || (t.kind != XKind::Plain && !norm && !merge) || call.segments ||
        call.epilogue != Epilogue::Single || call.m == 0 || call.m > max_m ||
        (call.k != 1024 && call.k != 2048 && !k8192) ||
        (F == Format::Ternary && head && call.k != 1024) || !x || !aligned(x))
        return false;
    // wide_row_kernel addresses the repacked codes with 32-bit byte offsets.
    if (uint64_t(n_tiles) * 16 * call.k * (F == Format::Int8 ? 8 : F == Format::Nf4 ? 4 : 2) / 8 >=
        (uint64_t(1) << 32))
        return false;
    StreamArgs args{};
    args.x = x;
    if (norm) {
        args.b = t.b;
        args.w = t.w;
        args.epsilon = t.epsilon;
    }
    if (merge) {
        args.ranges = t.ranges;
        args.head_dim = t.head_dim;
    }
    if (call.m == 1)
        args.argmax = call.argmax;
    args.tiles = call.a.tiles;
    args.scales = call.a.tiled_scales;
    args.out = call.out_a;
    args.m = call.m;
    args.n = call.n;
    args.k = call.k;
    args.n_tiles = n_tiles;
    const bool half = call.a.tiled_half;
    if constexpr (F != Format::Nf4) {
        if (k8192) {
            auto go = [&](auto nf_tag) {
                constexpr int NF = decltype(nf_tag)::value;
                if (half)
                    wide_rows_kernel<F, true, 32, 1, NF, 16, 1, 2>
                        <<<args.n_tiles, 1024, 0, stream>>>(args);
                else
                    wide_rows_kernel<F, false, 32, 1, NF, 16, 1, 2>
                        <<<args.n_tiles, 1024, 0, stream>>>(args);
            };
            go(std::integral_constant<int, 1>{});
            return true;
        }
        if (call.m > 1) {
            auto rows = [&](auto p_tag, auto nf_tag) {
                constexpr int P = decltype(p_tag)::value, NF = decltype(nf_tag)::value;
                if (half)
                    launch_wide_rows<F, true, P, NF>(stream, args);
                else
                    launch_wide_rows<F, false, P, NF>(stream, args);
            };
            using One = std::integral_constant<int, 1>;
            using Two = std::integral_constant<int, 2>;
            if (call.k == 2048)
                call.m <= 4 ? rows(std::integral_constant<int, 8>{}, One{})
                            : rows(std::integral_constant<int, 8>{}, Two{});
            else
                call.m <= 4 ? rows(std::integral_constant<int, 4>{}, One{})
                            : rows(std::integral_constant<int, 4>{}, Two{});
            return true;
        }
    }
    unsigned blocks;
    if (call.k == 2048)
        blocks = half ? launch_wide_row<F, true, 8>(stream, args, norm, merge)
                      : launch_wide_row<F, false, 8>(stream, args, norm, merge);
    else
        blocks = half ? launch_wide_row<F, true, 4>(stream, args, norm, merge)
                      : launch_wide_row<F, false, 4>(stream, args, norm, merge);
    if (blocks && args.argmax && call.argmax_count)
        *call.argmax_count = blocks;
    return true;
}

template <Format F, bool HALF, int P, int SPW, int S, XKind PRO, Epilogue E>
void launch_wide_one(hipStream_t stream, const WideArgs &args, uint32_t blocks)
{
    wide_one_kernel<F, HALF, P, SPW, S, PRO, E><<<blocks, 64 * P, 0, stream>>>(args);
}

// Kernel shape of a one-row wide product: (P waves, SPW slices) for K, or
// false.
bool wide_one_shape(uint32_t k, int &p, int &spw)
{
    switch (k) {
    case 1024: p = 4; spw = 1; return true;
    case 2048: p = 8; spw = 1; return true;
    case 4608: p = 9; spw = 2; return true;
    case 8192: p = 16; spw = 2; return true;
    default: return false;
    }
}

// Dispatch over (HALF, K shape) for one (S, PRO, E) combination.
template <Format F, int S, XKind PRO, Epilogue E>
void wide_one_go(hipStream_t stream, const WideArgs &args, uint32_t blocks, bool half, int p)
{
    auto go = [&](auto half_tag) {
        constexpr bool H = decltype(half_tag)::value;
        if constexpr (S == 1 && E == Epilogue::Single && PRO != XKind::AddRms) {
            // Plain and SwiGLU singles: the long contractions (down
            // projections); K = 1024 and 2048 plain rows take wide_row_kernel.
            if constexpr (PRO == XKind::Swiglu) {
                if (p == 9)
                    return launch_wide_one<F, H, 9, 2, S, PRO, E>(stream, args, blocks);
            }
            if (p == 16)
                return launch_wide_one<F, H, 16, 2, S, PRO, E>(stream, args, blocks);
        }
        if constexpr (PRO != XKind::Swiglu || S == 1) {
            if (p == 4)
                return launch_wide_one<F, H, 4, 1, S, PRO, E>(stream, args, blocks);
            if (p == 8)
                return launch_wide_one<F, H, 8, 1, S, PRO, E>(stream, args, blocks);
        }
    };
    if (half)
        go(std::true_type{});
    else
        go(std::false_type{});
}

// Whether the one-row wide kernel serves this call (ternary and NF4, m = 1,
// K one of wide_one_shape's, 16-byte aligned operands).
bool wide_one_ok(const PackedCall &call, int &p, int &spw)
{
    const XForm &t = call.xform;
    auto aligned = [](const void *ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
    if (call.format == Format::Int8 || call.separate_prologue || call.segments || call.m != 1 ||
        !wide_one_shape(call.k, p, spw) || !call.a.tiles)
        return false;
    const bool single = call.epilogue == Epilogue::Single;
    if (!single && (!call.b.tiles || call.a.tiled_half != call.b.tiled_half))
        return false;
    // Two slices per wave serve the long single contractions: SwiGLU rows,
    // and plain rows at K = 8192 (at K = 4608, 64 blocks of nine waves for
    // the 350M-shape down projection measured slower than the f32 vector
    // GEMV: decode 3194 against 3102 tok/s).
    if (spw == 2 && !(single && (t.kind == XKind::Swiglu ||
                                 (t.kind == XKind::Plain && call.k == 8192))))
        return false;
    // Plain single rows at K = 1024 and 2048 are wide_row_kernel's (and the
    // ternary head's streaming rows kernel's).
    if (single && t.kind == XKind::Plain && spw == 1)
        return false;
    if (t.kind == XKind::Swiglu && !single)
        return false;
    const float *x = t.kind == XKind::Plain ? call.x : t.a;
    if (!x || !aligned(x))
        return false;
    if (t.kind == XKind::Swiglu && (!t.b || !aligned(t.b)))
        return false;
    if (t.kind == XKind::AddRms &&
        (!t.w || !aligned(t.w) || (t.b && !aligned(t.b)) || (t.side && !aligned(t.side))))
        return false;
    return true;
}

// Serves a one-row product (single, pair or SwiGLU pair; plain, add + RMS
// norm or SwiGLU activations) with wide_one_kernel; false leaves it to the
// other plans.  Measured in the LFM2 greedy decode (tok/s, fused step / op
// by op; 1.2B shape, then 350M) against the plans each use replaces: all of
// them 2302 / 1710, 3102 / 2030; the pairs on the register-prologue
// plans 2008 / 1571, 2730 / 2008; SwiGLU rows as a prologue kernel plus
// the K-split GEMV (op by op) 1620, 1814; the K = 8192 down projection on
// the f32 vector GEMV 2245 / 1710; the norm-fed singles (grouped q/k/v) on
// the vector GEMV's norm variant 2300 / 1711, 3104 / 2056 (the same).
template <Format F>
bool try_wide_one(hipStream_t stream, const PackedCall &call, uint32_t n_tiles)
{
    int p, spw;
    if constexpr (F == Format::Int8) {
        return false;
    } else {
        if (!wide_one_ok(call, p, spw))
            return false;
        const XKind kind = call.xform.kind;
        WideArgs args{};
        args.xform = call.xform;
        if (kind == XKind::Plain)
            args.xform.a = call.x;
        args.tiles[0] = call.a.tiles;
        args.tiles[1] = call.b.tiles;
        args.scales[0] = call.a.tiled_scales;
        args.scales[1] = call.b.tiled_scales;
        args.out[0] = call.out_a;
        args.out[1] = call.out_b;
        args.n = call.n;
        args.k = call.k;
        const bool half = call.a.tiled_half;
        switch (call.epilogue) {
        case Epilogue::Single:
            if (kind == XKind::AddRms)
                wide_one_go<F, 1, XKind::AddRms, Epilogue::Single>(stream, args, n_tiles, half, p);
            else if (kind == XKind::Swiglu)
                wide_one_go<F, 1, XKind::Swiglu, Epilogue::Single>(stream, args, n_tiles, half, p);
            else
                wide_one_go<F, 1, XKind::Plain, Epilogue::Single>(stream, args, n_tiles, half, p);
            break;
        case Epilogue::Pair:
            if (kind == XKind::AddRms)
                wide_one_go<F, 2, XKind::AddRms, Epilogue::Pair>(stream, args, n_tiles, half, p);
            else
                wide_one_go<F, 2, XKind::Plain, Epilogue::Pair>(stream, args, n_tiles, half, p);
            break;
        case Epilogue::SwigluPair:
            if (kind == XKind::AddRms)
                wide_one_go<F, 2, XKind::AddRms, Epilogue::SwigluPair>(stream, args, n_tiles, half,
                                                                        p);
            else
                wide_one_go<F, 2, XKind::Plain, Epilogue::SwigluPair>(stream, args, n_tiles, half,
                                                                       p);
            break;
        }
        return true;
    }
}

}  // namespace

// The convolution in-projection at one row (three row regions of one
// matrix: B, C, x) with the add + RMS norm, finished by the one-token
// convolution in the epilogue; ternary and NF4, hidden a multiple of 16.
// LFM2 greedy decode against the vector GEMV's convolution variant: 1.2B
// shape 2253 -> 2302 tok/s, 350M 2974 -> 3102.
bool head_fold_supported(Format f, uint32_t n, uint32_t k)
{
    const uint32_t n_tiles = pad_to(n, 64) / 16;
    return f != Format::Nf4 && n_tiles >= kHeadTiles &&
           (k == 1024 || (k == 2048 && f == Format::Int8));
}

bool wide_conv_supported(const PackedCall &call, const ConvStep &conv)
{
    int p, spw;
    const XForm &t = call.xform;
    auto aligned = [](const void *ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
    return call.format != Format::Int8 && call.m == 1 && t.kind == XKind::AddRms &&
           wide_one_shape(call.k, p, spw) && spw == 1 && conv.hidden % 16 == 0 &&
           call.n == 3 * conv.hidden && conv.width >= 1 && t.a && aligned(t.a) && t.w &&
           aligned(t.w) && (!t.b || aligned(t.b)) && (!t.side || aligned(t.side));
}

bool try_wide_conv(hipStream_t stream, const PackedCall &call, const ConvStep &conv)
{
    if (!wide_conv_supported(call, conv) || !call.a.tiles)
        return false;
    int p, spw;
    wide_one_shape(call.k, p, spw);
    WideArgs args{};
    args.xform = call.xform;
    args.tiles[0] = call.a.tiles;
    args.scales[0] = call.a.tiled_scales;
    args.n = call.n;
    args.k = call.k;
    args.stream_tiles = conv.hidden / 16;
    args.conv = conv;
    const uint32_t blocks = conv.hidden / 16;
    auto go = [&](auto f_tag, auto half_tag) {
        constexpr Format F = decltype(f_tag)::value;
        constexpr bool H = decltype(half_tag)::value;
        if (p == 4)
            launch_wide_one<F, H, 4, 1, 3, XKind::AddRms, Epilogue::Single>(stream, args, blocks);
        else
            launch_wide_one<F, H, 8, 1, 3, XKind::AddRms, Epilogue::Single>(stream, args, blocks);
    };
    auto by_half = [&](auto f_tag) {
        if (call.a.tiled_half)
            go(f_tag, std::true_type{});
        else
            go(f_tag, std::false_type{});
    };
    if (call.format == Format::Ternary)
        by_half(std::integral_constant<Format, Format::Ternary>{});
    else
        by_half(std::integral_constant<Format, Format::Nf4>{});
    return true;
}

namespace {

template <Format F>
void gemv_i8_format(hipStream_t stream, const PackedCall &call, void *scratch)
{
    const uint32_t k_pad = pad_to(call.k, Geo<F>::align);
    const uint32_t groups = k_pad / 128;
    const uint32_t n_tiles = call_tiles(call);
    // Ternary from kStreamMinTiles row tiles (two rows from
    // kStreamTwoRowMinTiles) to below the head size: the streaming kernels
    // before the one-tile-per-block plans.  Measured (us
    // per launch, A/B on one device), one / two / four / eight rows: 16384 x
    // 2048 5.6 / 9.1 / 9.3 / 14.8 -> 4.5 / 5.3 / 6.2 / 9.5, 32768 x 2048
    // 8.7 / 16.2 / 16.8 / 27.3 -> 5.3 / 6.0 / 6.6 / 9.5, 12288 x 2048 at
    // one / four rows 4.9 / 7.5 -> 4.4 / 6.1; two rows at K = 1024, 16384 /
    // 32768 rows 5.4 / 8.9 -> 3.9 / 4.3.
    if constexpr (F == Format::Ternary) {
        if (n_tiles < kHeadTiles && try_stream_ternary(stream, call, n_tiles))
            return;
    }
    if (try_wide_row<F>(stream, call, n_tiles))
        return;
    if (try_wide_one<F>(stream, call, n_tiles))
        return;
    if (try_vgemv(stream, call))
        return;
    if constexpr (F == Format::Ternary) {
        if (try_stream_ternary(stream, call, n_tiles))
            return;
    }
    const int nf = call.m <= 4 ? 1 : 2;
    Scratch sc = carve(scratch, k_pad);
    const int streams = call.epilogue == Epilogue::Single ? 1 : 2;
    const uint32_t ksteps = k_pad / 64;
    XForm xform = call.xform;
    if (xform.kind == XKind::Plain)
        xform.a = call.x;
    // The in-kernel prologue keeps the live fragment rows of all of K in
    // LDS; it is used while that (plus the reduction area) fits in 64 KB, so
    // blocks stay small enough for several to share a CU.  Every block
    // recomputes the prologue, so a large grid (the LM head) or many
    // activation rows are faster with the separate prologue kernel, and so
    // is a wave share above kFusedGroupsPerWave groups.
    auto tiles_of = [](Plan p) { return p.tiles_per_block == 4 ? 4 : 1; };  // T in {1, 4}
    auto fusable = [&](Plan p) {
        const int t = tiles_of(p);
        const size_t lds = fused_bytes(k_pad, call.m) +
                           size_t(p.waves) * streams * t * nf * 64 * sizeof(float);
        const uint32_t share = (groups + p.waves - 1) / p.waves;
        return !call.separate_prologue && call.m <= 2 && lds <= 64 * 1024 &&
               n_tiles / t <= kFusedMaxBlocks && share <= kFusedGroupsPerWave &&
               share <= held_groups(xform.kind) && fused_kind_served(call.epilogue, xform.kind);
    };
    // Segmented launches keep one tile per block.
    const int max_t = streams == 1 && !call.segments ? 4 : 1;
    const Plan narrow = plan_for(n_tiles, ksteps, Geo<F>::lb, max_t, false);
    const Plan wide = plan_for(n_tiles, ksteps, Geo<F>::lb, max_t, true);
    // The register prologue serves plain activations (up to eight rows for
    // single products, four for two-stream ones), and the add + RMS norm of
    // at most four rows when each wave's K range is at most kRegNormSteps
    // ksteps (it holds them all while the row's squares reduce), with 16-byte
    // aligned operands.  Ternary operands cost more arithmetic per group
    // (the field telescoping and the correction): past two groups per wave
    // the separate prologue kernel measured faster (65536 x 2048: 13.3
    // against 14.4 us).
    auto aligned = [](const void *ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
    auto reg_ok = [&](Plan p) {
        const uint32_t per_wave = ksteps / p.waves;
        if (call.separate_prologue || (F == Format::Ternary && per_wave / 2 > 2))
            return false;
        if (xform.kind == XKind::Plain && call.m > 4) {
            // Two fragments double each lane's prologue arithmetic, which
            // every block repeats for its K range: it stays ahead of the
            // separate kernel for INT8 up to 8 ksteps per wave (2048 x 8192
            // at 16: 12.7 -> 13.9 us) and for ternary up to kRegPairBlocks
            // blocks (8192 x 2048 at 512 blocks: 8.0 -> 10.7 us; 4608 x 1024
            // at 288: 6.3 -> 6.0 us).
            if (streams != 1 || (F == Format::Int8 && per_wave > 8) ||
                (F == Format::Ternary && n_tiles / tiles_of(p) > kRegPairBlocks))
                return false;
        }
        if (xform.kind == XKind::Plain)
            return aligned(xform.a);
        if (call.m > 4)
            return false;
        if (xform.kind == XKind::AddRms)
            return per_wave <= uint32_t(kRegNormSteps) && aligned(xform.a) && aligned(xform.b) &&
                   aligned(xform.w) && aligned(xform.side);
        return false;
    };
    // Preference: the register prologue (norm or plain), then the LDS one,
    // then the separate prologue kernel.  For plain activations the register
    // prologue measured 13-46 % faster than the LDS one wherever both apply
    // (4608 x 1024 at two rows: ternary 7.49 -> 4.01 us, INT8 5.52 -> 3.61);
    // for the add + norm, taking the LDS one wherever it applies made decode
    // slower (1.2B shape 1596 -> 1548 tok/s, 350M 2376 -> 2143).
    // The 8-wave plan takes the norm only with one tile per block: the 4-tile
    // norm kernel holds two waves per SIMD, too few for the LM head's 8-wave
    // blocks (1.2B-shape decode 1389 -> 1355 tok/s).
    Plan plan = narrow;
    int pro = -1;
    const bool reg_wide = reg_ok(wide) && tiles_of(wide) == 1;
    if (xform.kind == XKind::AddRms && (reg_ok(narrow) || reg_wide)) {
        plan = reg_ok(narrow) ? narrow : wide;
        pro = kRegPro + int(XKind::AddRms);
    } else if (xform.kind == XKind::Plain && (reg_ok(narrow) || (streams == 2 && reg_wide))) {
        // Two-stream products whose 4-wave share is past the ternary limit
        // take the 8-wave plan (8192 x 2048 pair at one row, against the LDS
        // prologue: 1.2B-shape op-by-op decode 1254 -> 1294 tok/s).
        plan = reg_ok(narrow) ? narrow : wide;
        pro = kRegPro;
    } else if (fusable(narrow) || fusable(wide)) {
        plan = fusable(narrow) ? narrow : wide;
        pro = int(xform.kind);
    }
    plan.tiles_per_block = tiles_of(plan);
    // The INT8 LM head at one or two rows takes one tile per block: 4096
    // blocks of 4 waves, 8 KB of weights per wave, against 1024 blocks with
    // 32 KB per wave in the 4-tile plan.  65536 x 2048 at B = 1: 25.1 ->
    // 23.2 us; B = 2: 25.3 -> 23.7 us.  From four rows on the 4-tile plan is
    // faster (B = 4: 24.9 against 25.8-26.5 us; B = 8 28.5 against 43-46).
    if (F == Format::Int8 && pro == kRegPro && streams == 1 && !call.segments && call.m <= 2 &&
        n_tiles >= kHeadTiles && plan.tiles_per_block == 4 && ksteps % (4 * Geo<F>::lb) == 0)
        plan = Plan{1, 4};
    if ((pro < 0 || pro == kRegPro) && streams == 1 && nf == 1)
        plan = deepen(plan, n_tiles, ksteps, Geo<F>::lb);
    // Small grids with the separate prologue split K over two blocks per
    // tile group (MfmaArgs::kparts); the prologue kernel zeroes the output
    // they add into, so the output must not overlap the activations.  Where
    // K does not divide over twice the waves, each part takes half of them
    // (the same K range per wave over twice the blocks).
    uint32_t kparts = 1;
    if (pro < 0 && streams == 1 && !call.segments && xform.kind == XKind::Plain &&
        n_tiles / plan.tiles_per_block <= kSplitMaxBlocks &&
        !overlaps(call.out_a, size_t(call.m) * call.n, xform.a, size_t(call.m) * call.k)) {
        if (ksteps % (2 * plan.waves * Geo<F>::lb) == 0) {
            kparts = 2;
        } else if (plan.waves % 2 == 0 && ksteps % (plan.waves * Geo<F>::lb) == 0) {
            plan.waves /= 2;
            kparts = 2;
        }
    }
    if (pro < 0)
        digits_kernel<F>
            <<<dim3((groups + kPrologueWaves - 1) / kPrologueWaves, 4 * nf), 64 * kPrologueWaves,
               0, stream>>>(xform, call.m, call.k, groups, nf, static_cast<int8_t *>(sc.afrag),
                            sc.xf, sc.corr, kparts > 1 ? call.out_a : nullptr,
                            kparts > 1 ? call.m * call.n : 0);
    MfmaArgs args{};
    args.xform = xform;
    args.k = call.k;
    args.afrag = sc.afrag;
    args.xf = sc.xf;
    args.corr = sc.corr;
    args.tiles[0] = call.a.tiles;
    args.tiles[1] = call.b.tiles;
    args.scales[0] = call.a.tiled_scales;
    args.scales[1] = call.b.tiled_scales;
    args.out[0] = call.out_a;
    args.out[1] = call.out_b;
    args.m = call.m;
    args.n = call.n;
    args.k_pad = k_pad;
    args.ksteps_per_wave = ksteps / (plan.waves * kparts);
    args.kparts = kparts;
    args.part_blocks = n_tiles / plan.tiles_per_block;
    set_segments(args, call);
    const unsigned blocks = n_tiles / plan.tiles_per_block * kparts;
    const bool half = call.a.tiled_half && (streams == 1 || call.b.tiled_half);
    if (streams == 1) {
        if (plan.tiles_per_block == 4)
            launch_i8_nf<F, 4, 1>(stream, args, call.epilogue, blocks, plan.waves, nf, half, pro);
        else
            launch_i8_nf<F, 1, 1>(stream, args, call.epilogue, blocks, plan.waves, nf, half, pro);
    } else {
        launch_i8_nf<F, 1, 2>(stream, args, call.epilogue, blocks, plan.waves, nf, half, pro);
    }
}

template <int G>
void launch_stream_nf4(hipStream_t stream, const StreamArgs &args, bool half)
{
    const unsigned blocks = (args.n_tiles + kStreamWaves - 1) / kStreamWaves;
    if (half)
        stream_nf4_kernel<G, true><<<blocks, 64 * kStreamWaves, 0, stream>>>(args);
    else
        stream_nf4_kernel<G, false><<<blocks, 64 * kStreamWaves, 0, stream>>>(args);
}

// As try_stream_ternary: K of 8 or 16 groups (one prologue group per wave),
// and grids of at least kStreamMinBlocks full 16-wave blocks.
// From 2048 row tiles (128 blocks) the streaming kernel serves what the wide
// kernels do not (two to eight rows).  Measured (us per launch, A/B on one
// device) against the K-split plans: 32768 x 2048 at B = 2 / 4 / 8 15.9 /
// 15.9 / 16.1 -> 14.8 / 15.2 / 14.8, 49152 x 2048 at B = 4 21.8 -> 16.6,
// 32768 x 1024 at B = 2 / 8 10.6 / 11.1 -> 9.5 / 9.6; at 1024 tiles slower
// (16384 x 2048 at B = 2 / 8 11.3 / 11.4 -> 14.1 / 13.8).
constexpr uint32_t kStreamNf4MinTiles = 2048;

bool try_stream_nf4(hipStream_t stream, const PackedCall &call, uint32_t n_tiles)
{
    const uint32_t groups = pad_to(call.k, 128) / 128;
    if (call.separate_prologue || call.xform.kind != XKind::Plain || call.segments ||
        call.epilogue != Epilogue::Single || call.m == 0 || call.m > 8 ||
        n_tiles < kStreamNf4MinTiles || (groups != 8 && groups != 16) ||
        reinterpret_cast<uintptr_t>(call.x) % 16 != 0)
        return false;
    StreamArgs args{};
    args.x = call.x;
    args.tiles = call.a.tiles;
    args.scales = call.a.tiled_scales;
    args.out = call.out_a;
    args.m = call.m;
    args.n = call.n;
    args.k = call.k;
    args.n_tiles = n_tiles;
    if (groups == 8)
        launch_stream_nf4<8>(stream, args, call.a.tiled_half);
    else
        launch_stream_nf4<16>(stream, args, call.a.tiled_half);
    return true;
}

void gemv_nf4(hipStream_t stream, const PackedCall &call, void *scratch)
{
    const uint32_t k_pad = pad_to(call.k, 128);
    const uint32_t groups = k_pad / 128;
    const uint32_t n_tiles = call_tiles(call);
    if (try_wide_row<Format::Nf4>(stream, call, n_tiles))
        return;
    if (try_wide_one<Format::Nf4>(stream, call, n_tiles))
        return;
    if (try_vgemv(stream, call))
        return;
    if (try_stream_nf4(stream, call, n_tiles))
        return;
    Scratch sc = carve(scratch, k_pad);
    const int streams = call.epilogue == Epilogue::Single ? 1 : 2;
    const uint32_t ksteps = k_pad / 32;
    XForm xform = call.xform;
    if (xform.kind == XKind::Plain)
        xform.a = call.x;
    // Same rule as the integer kernels (gemv_i8_format).
    auto fusable = [&](Plan p) {
        const size_t lds = fused_bytes_nf4(k_pad, call.m) +
                           size_t(p.waves) * streams * p.tiles_per_block * 2 * 64 * sizeof(float);
        const uint32_t share = (groups + p.waves - 1) / p.waves;
        return !call.separate_prologue && call.m <= 2 && lds <= 64 * 1024 &&
               n_tiles / p.tiles_per_block <= kFusedMaxBlocks && share <= kFusedGroupsPerWave &&
               share <= held_groups(xform.kind) && fused_kind_served(call.epilogue, xform.kind);
    };
    const int max_t = streams == 1 && !call.segments ? 2 : 1;
    const Plan narrow = plan_for(n_tiles, ksteps, 4, max_t, false);
    const Plan wide = plan_for(n_tiles, ksteps, 4, max_t, true);
    // Register prologue for plain activations (up to eight rows, 16-byte
    // aligned) over at most 256 k per wave.  NF4 forms twice the operand
    // values per k of the integer formats next to its table decode, and past
    // that share (the 65536 x 2048 head, K = 8192) or for the add + RMS norm
    // the separate or LDS prologue measured faster.  It is preferred to the
    // LDS prologue (1024 x 1024 at two rows: 5.01 -> 3.72 us) and to the
    // separate one at five to eight rows (1024 x 1024 at eight: 6.49 ->
    // 3.85 us; 8192 x 2048: 8.08 -> 6.87 us).
    Plan plan = narrow;
    int pro = -1;
    if (!call.separate_prologue && xform.kind == XKind::Plain && call.m <= 8 &&
        ksteps / narrow.waves <= 8 && reinterpret_cast<uintptr_t>(xform.a) % 16 == 0) {
        pro = kRegPro;
    } else if (fusable(narrow) || fusable(wide)) {
        plan = fusable(narrow) ? narrow : wide;
        pro = int(xform.kind);
    }
    if ((pro < 0 || pro == kRegPro) && streams == 1)
        plan = deepen(plan, n_tiles, ksteps, 4);
    // The two-part K split of gemv_i8_format.
    const uint32_t kparts = pro < 0 && streams == 1 && !call.segments &&
                                    xform.kind == XKind::Plain &&
                                    n_tiles / plan.tiles_per_block <= kSplitMaxBlocks &&
                                    ksteps % (2 * plan.waves * 4) == 0 &&
                                    !overlaps(call.out_a, size_t(call.m) * call.n, xform.a,
                                              size_t(call.m) * call.k)
                                ? 2
                                : 1;
    if (pro < 0)
        halves_kernel<<<dim3((groups + kPrologueWaves - 1) / kPrologueWaves, 8),
                        64 * kPrologueWaves, 0, stream>>>(
            xform, call.m, call.k, groups, static_cast<_Float16 *>(sc.afrag), sc.xf,
            kparts > 1 ? call.out_a : nullptr, kparts > 1 ? call.m * call.n : 0);
    MfmaArgs args{};
    args.xform = xform;
    args.k = call.k;
    args.afrag = sc.afrag;
    args.xf = sc.xf;
    args.tiles[0] = call.a.tiles;
    args.tiles[1] = call.b.tiles;
    args.scales[0] = call.a.tiled_scales;
    args.scales[1] = call.b.tiled_scales;
    args.out[0] = call.out_a;
    args.out[1] = call.out_b;
    args.m = call.m;
    args.n = call.n;
    args.k_pad = k_pad;
    args.ksteps_per_wave = ksteps / (plan.waves * kparts);
    args.kparts = kparts;
    args.part_blocks = n_tiles / plan.tiles_per_block;
    set_segments(args, call);
    const unsigned blocks = n_tiles / plan.tiles_per_block * kparts;
    const bool half = call.a.tiled_half && (streams == 1 || call.b.tiled_half);
    if (streams == 1) {
        if (plan.tiles_per_block == 2)
            launch_nf4_variant<2, 1>(stream, args, call.epilogue, blocks, plan.waves, half, pro);
        else
            launch_nf4_variant<1, 1>(stream, args, call.epilogue, blocks, plan.waves, half, pro);
    } else {
        launch_nf4_variant<1, 2>(stream, args, call.epilogue, blocks, plan.waves, half, pro);
    }
}

}  // namespace

bool gemv_mfma_supported(Format format)
{
    (void)format;
    return true;
}

size_t gemv_mfma_scratch_bytes(const PackedCall &call)
{
    const uint32_t k_pad = pad_to(call.k, 256);
    return size_t(k_pad) * 32 + size_t(8) * (k_pad / 128) * sizeof(float) +
           size_t(8) * (k_pad / 128) * 4 * sizeof(int);
}

bool gqa_merge_supported(const PackedCall &call)
{
    const uint32_t n_tiles = pad_to(call.n, 64) / 16;
    const XForm &t = call.xform;
    const uint64_t code_bytes = uint64_t(n_tiles) * 16 * call.k *
                                (call.format == Format::Int8 ? 8 : call.format == Format::Nf4 ? 4 : 2) / 8;
    return t.kind == XKind::GqaMerge && t.a && call.m == 1 && !call.separate_prologue &&
           !call.segments && call.epilogue == Epilogue::Single && n_tiles < kHeadTiles &&
           (call.k == 1024 || call.k == 2048) && code_bytes < (uint64_t(1) << 32) &&
           reinterpret_cast<uintptr_t>(t.a) % 16 == 0 && t.ranges > 0 &&
           t.ranges <= kGqaMergeMaxRanges && t.head_dim > 0 && t.head_dim % 4 == 0 &&
           call.k % t.head_dim == 0;
}

void launch_gemv_mfma(hipStream_t stream, const PackedCall &call, void *scratch)
{
    if (call.xform.kind == XKind::GqaMerge) {
        // Only the one-row wide kernel reads the merge transform; callers
        // check gqa_merge_supported first.
        const uint32_t n_tiles = pad_to(call.n, 64) / 16;
        switch (call.format) {
        case Format::Ternary: (void)try_wide_row<Format::Ternary>(stream, call, n_tiles); break;
        case Format::Int8: (void)try_wide_row<Format::Int8>(stream, call, n_tiles); break;
        case Format::Nf4: (void)try_wide_row<Format::Nf4>(stream, call, n_tiles); break;
        }
        return;
    }
    switch (call.format) {
    case Format::Ternary: gemv_i8_format<Format::Ternary>(stream, call, scratch); break;
    case Format::Int8: gemv_i8_format<Format::Int8>(stream, call, scratch); break;
    case Format::Nf4: gemv_nf4(stream, call, scratch); break;
    }
}

size_t repacked_bytes(Format format, uint32_t n, uint32_t k)
{
    const uint32_t n_tiles = pad_to(n, 64) / 16;
    return size_t(n_tiles) * 16 * pad_to(k, align_of(format)) / weights_per_byte(format);
}

size_t tiled_scales_bytes(Format format, uint32_t n, uint32_t k, bool half)
{
    const uint32_t n_tiles = pad_to(n, 64) / 16;
    const uint32_t k_pad = pad_to(k, align_of(format));
    return size_t(n_tiles) * (k_pad / 128) * 16 * (half ? 2 : 4);
}

void launch_repack(hipStream_t stream, Format format, const uint8_t *codes, uint8_t *tiles,
                   uint32_t n, uint32_t k)
{
    const uint32_t n_tiles = pad_to(n, 64) / 16;
    const uint32_t k_pad = pad_to(k, align_of(format));
    const size_t total = repacked_bytes(format, n, k) / 16;
    switch (format) {
    case Format::Ternary:
        repack_kernel<Format::Ternary><<<grid_for(total), 256, 0, stream>>>(codes, tiles, n, k,
                                                                             k_pad, n_tiles);
        break;
    case Format::Nf4:
        repack_kernel<Format::Nf4><<<grid_for(total), 256, 0, stream>>>(codes, tiles, n, k, k_pad,
                                                                         n_tiles);
        break;
    case Format::Int8:
        repack_kernel<Format::Int8><<<grid_for(total), 256, 0, stream>>>(codes, tiles, n, k,
                                                                          k_pad, n_tiles);
        break;
    }
}

void launch_tile_scales(hipStream_t stream, Format format, const float *scales, void *out,
                        uint32_t n, uint32_t k, bool half)
{
    const uint32_t n_tiles = pad_to(n, 64) / 16;
    const uint32_t k_pad = pad_to(k, align_of(format));
    const size_t total = size_t(n_tiles) * (k_pad / 128) * 16;
    if (half)
        tile_scales_kernel<true><<<grid_for(total), 256, 0, stream>>>(scales, out, n, k / 128,
                                                                      k_pad / 128, n_tiles);
    else
        tile_scales_kernel<false><<<grid_for(total), 256, 0, stream>>>(scales, out, n, k / 128,
                                                                       k_pad / 128, n_tiles);
}

}  // namespace mfh
