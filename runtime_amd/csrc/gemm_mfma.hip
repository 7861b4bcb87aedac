// Matrix-core prefill GEMM for packed ternary / NF4 / INT8 weights (m > 8).
//
// out[m, n] = sum_g scale[n, g] * sum_{k in g} x[m, k] * level(code[n, k]),
// the reference's group-then-scale order (kernels-simd/src/lib.rs:54,205).
//
// Exactness plan.
// - The activation prologue (split_kernel) scales every row by 2^-e so its
//   largest magnitude is below 1, and splits each value as x = hi + lo with
//   both halves binary16 (22 significant bits; values below 2^-14 of the
//   row's largest keep an absolute error under 2^-24 of it).
// - Weight levels are exact in binary16 for ternary (-1, 0, 1, 2) and INT8
//   (-127..127).  NF4 levels are split the same way as the activations.
// - v_mfma_f32_16x16x32_f16 forms the products exactly in f32 and
//   accumulates each 128-group separately.
// - The group epilogue adds group_sum * scale in f32 (one FMA), and the
//   store multiplies by the row's 2^e, a power of two, so the result equals
//   the reference's sum of scale * dot.  NF4 drops the lo * lo product,
//   which is below 2^-22 of each term.
// - Single-half mode (opt-in, mfh_set_gemm_activations): the activations
//   keep only the hi half, one MFMA per product (NF4: two), each activation
//   within 2^-12 of itself relative (2^-25 of the row's largest absolute
//   below 2^-14 of it); weights and the epilogue are unchanged.
//
// Operands.  B (the weights) is read straight from the decode GEMV's
// repacked tiles: 16 rows x K per tile, one 16-byte load per lane covering
// 64 (INT8), 128 (NF4) or 256 (ternary) k, already in the MFMA lane order.
// Each wave decodes its tiles to binary16 in registers (INT8 and ternary by
// placing the code under a binary16 exponent of 1024 and subtracting, NF4
// through a 256-entry LDS table of level halves), so weights never pass
// through LDS.  A, the activation halves, is staged through LDS, double
// buffered, one stage ahead in registers.  Within a 64-wide stage, MFMA
// half h takes k = 16q + 8h + 0..7 of lane block q (INT8, ternary: the
// tiles' byte order) or k = 32h + 8q + 0..7 (NF4: its 32-wide kstep).
//
// Tiling.  A 256-lane block (4 waves) computes a 128 (m) x 128 (n) output
// tile (64 x 128 where 128-row tiles would need a K split; its waves lie
// along n), split over S weight streams of 128 / S columns each.  The waves lie
// along n: each owns all 128 rows x 32 columns (8 x 2 MFMA tiles), so every
// weight tile is decoded by one wave of the block; exact ternary keeps 2 x 2
// waves of 64 x 64 (4 x 4 MFMA tiles), which reuse each activation fragment
// over four column tiles.  A wave holds a group accumulator and a running
// total per MFMA tile.  The 74 KB of LDS lets two blocks share a CU.
//
// Grid mapping.  Workgroups are dealt round-robin to the 8 XCDs.  Block b
// computes tile (b % 8) * (tiles / 8) + b / 8, so each XCD's L2 holds a
// contiguous run of tiles: neighbouring n-tiles of the same m rows.
#include <algorithm>
#include <type_traits>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace mfh {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves: 2 (m) x 2 (n)
constexpr int kBM = 128;       // rows per block tile
constexpr int kBN = 128;       // columns per block tile (all streams)
constexpr int kBK = 64;        // k per stage
// LDS row pitch in halves: kBK + 8 (144 bytes) puts the 16 rows read by one
// lane group on distinct banks.
constexpr int kRow = kBK + 8;

__constant__ float kLevels[16] = {
    -1.0f,        -0.6961928f,  -0.52507305f, -0.3949175f,
    -0.28444138f, -0.18477343f, -0.091050036f, 0.0f,
    0.0795803f,   0.1609302f,   0.2461123f,   0.33791524f,
    0.44070983f,  0.562617f,    0.72295684f,  1.0f,
};

__device__ __forceinline__ float silu_mul(float gate, float up)
{
    const float sigmoid = 1.0f / (1.0f + expf(-gate));
    return (gate * sigmoid) * up;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// One block per row: factor[m] = 2^e with every |x| of the row below 2^e
// (NaN for a row with a non-finite value), and the binary16 halves of
// x * 2^-e (the lo half only where `xl` is non-null).  K is a multiple of
// 128.
constexpr int kSplitThreads = 256;
constexpr uint32_t kSplitHeld = 8;  // float4 per lane: K <= 8192

__global__ __launch_bounds__(kSplitThreads) void split_kernel(const float *__restrict__ x,
                                                              uint32_t k,
                                                              _Float16 *__restrict__ xh,
                                                              _Float16 *__restrict__ xl,
                                                              float *__restrict__ factor)
{
    __shared__ float wave_mx[kSplitThreads / 64];
    const uint32_t row = blockIdx.x, tid = threadIdx.x;
    const float4 *src = reinterpret_cast<const float4 *>(x + size_t(row) * k);
    const uint32_t vecs = k / 4;
    // Rows of up to kSplitHeld vectors per lane stay in registers between the
    // maximum and the split (one read of the row instead of two).
    const bool held = vecs <= kSplitHeld * kSplitThreads;
    float4 keep[kSplitHeld];
    // A non-finite value makes the row's maximum +inf.
    float mx = 0.0f;
    if (held) {
#pragma unroll
        for (uint32_t u = 0; u < kSplitHeld; ++u) {
            const uint32_t i = tid + u * kSplitThreads;
            keep[u] = i < vecs ? src[i] : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (uint32_t u = 0; u < kSplitHeld; ++u)
            for (float c : {keep[u].x, keep[u].y, keep[u].z, keep[u].w})
                mx = fmaxf(mx, isfinite(c) ? fabsf(c) : __builtin_inff());
    } else {
        for (uint32_t i = tid; i < vecs; i += kSplitThreads) {
            const float4 v = src[i];
            for (float c : {v.x, v.y, v.z, v.w})
                mx = fmaxf(mx, isfinite(c) ? fabsf(c) : __builtin_inff());
        }
    }
    mx = wave_max(mx);
    if ((tid & 63) == 0)
        wave_mx[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wave_mx[0], wave_mx[1]), fmaxf(wave_mx[2], wave_mx[3]));
    const bool bad = !isfinite(mx);
    int e = 0;
    if (!bad && mx > 0.0f)
        frexpf(mx, &e);  // |x| < 2^e
    if (tid == 0)
        factor[row] = bad ? __builtin_nanf("") : ldexpf(1.0f, e);
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 *dh = reinterpret_cast<h4 *>(xh + size_t(row) * k);
    h4 *dl = reinterpret_cast<h4 *>(xl + size_t(row) * k);
    auto split = [&](uint32_t i, const float4 &v) {
        h4 hi, lo;
        int t = 0;
        for (float c : {v.x, v.y, v.z, v.w}) {
            const float sv = bad ? 0.0f : ldexpf(c, -e);
            hi[t] = _Float16(sv);
            lo[t] = _Float16(sv - float(hi[t]));
            ++t;
        }
        dh[i] = hi;
        if (xl)
            dl[i] = lo;
    };
    if (held) {
#pragma unroll
        for (uint32_t u = 0; u < kSplitHeld; ++u) {
            const uint32_t i = tid + u * kSplitThreads;
            if (i < vecs)
                split(i, keep[u]);
        }
    } else {
        for (uint32_t i = tid; i < vecs; i += kSplitThreads)
            split(i, src[i]);
    }
}

struct GemmArgs {
    const _Float16 *xh, *xl;
    const float *factor;       // [m]: 2^e of each row
    const uint8_t *wtiles[2];  // repacked codes per stream
    const void *scales[2];     // tiled scales per stream: [tile][groups_pad][16]
    float *out[2];
    float *partial;            // split-K: [chunk][stream][m][n] raw sums
    uint32_t m, n, k;
    uint32_t n_tiles;          // 16-row tiles of each repacked stream
    uint32_t tile_vecs;        // 16-byte lane loads per tile (of 64 lanes)
    uint32_t groups_pad;       // tiled scale groups per tile
    uint32_t tiles_n, tiles;   // output block tiles along n, and in all
    uint32_t chunks;           // K split into `chunks` runs of whole groups
};

// 64-wide stages covered by one 16-byte lane load of a tile.
template <Format F> struct Chunk {
    static constexpr int stages = F == Format::Int8 ? 1 : F == Format::Nf4 ? 2 : 4;
};

// INT8 bytes 8h..8h+7 of the lane's 16 (k = 16q + 8h + 0..7): binary16
// 1024 + (b ^ 0x80) is exact, and subtracting 1152 leaves the signed code.
__device__ __forceinline__ v8h decode_i8(const v4u &raw, int h)
{
    const v2h bias = {_Float16(-1152.0f), _Float16(-1152.0f)};
    v8h out;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const unsigned x = raw[2 * h + d] ^ 0x80808080u;
        // v_perm_b32 selector bytes 0-3 pick bytes of its second operand, 4-7
        // of its first: [x.b0, 0x64, x.b1, 0x64] and [x.b2, 0x64, x.b3, 0x64].
        const v2h a = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u)) +
                      bias;
        const v2h b = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u)) +
                      bias;
        out[4 * d] = a[0];
        out[4 * d + 1] = a[1];
        out[4 * d + 2] = b[0];
        out[4 * d + 3] = b[1];
    }
    return out;
}

// Ternary tile dword (16 codes, k = 16q + 4e + f at byte e, field f; field 3
// stored as (c + 2) mod 4), bytes 2h and 2h + 1: binary16 1024 + c minus
// 1025 is c - 1.
__device__ __forceinline__ v8h decode_ternary(unsigned w, int h)
{
    const v2h bias = {_Float16(-1025.0f), _Float16(-1025.0f)};
    w ^= 0x80808080u;                              // canonical codes
    const unsigned even = w & 0x33333333u;         // fields 0, 2 of each byte
    const unsigned odd = (w >> 2) & 0x33333333u;   // fields 1, 3
    v8h out;
#pragma unroll
    for (int e2 = 0; e2 < 2; ++e2) {
        const unsigned e = unsigned(2 * h + e2);
        // [even.b_e, even.b_e, odd.b_e, odd.b_e]: each 16-bit lane's low
        // byte carries (field f, field f + 2) of one parity.
        const unsigned d = __builtin_amdgcn_perm(odd, even, e | (e << 8) | ((4 + e) << 16) |
                                                                ((4 + e) << 24));
        const v2h a = __builtin_bit_cast(v2h, (d & 0x00030003u) | 0x64006400u) + bias;
        const v2h b = __builtin_bit_cast(v2h, ((d >> 4) & 0x00030003u) | 0x64006400u) + bias;
        out[4 * e2] = a[0];      // field 0
        out[4 * e2 + 1] = a[1];  // field 1
        out[4 * e2 + 2] = b[0];  // field 2
        out[4 * e2 + 3] = b[1];  // field 3
    }
    return out;
}

template <Format F, int S, Epilogue E, bool HALF, bool LO, int BM>
__global__ __launch_bounds__(kThreads, 2) void gemm_mfma_kernel(GemmArgs g)
{
    static_assert(BM == kBM || BM == kBM / 2, "128- or 64-row block tiles");
    constexpr int P = F == Format::Nf4 ? 2 : 1;  // weight level planes
    constexpr int PA = LO ? 2 : 1;               // activation planes (hi, lo)
    // Waves along n (M = 2048 x 8192 x 2048 against 2 x 2: NF4 exact 218 ->
    // 206 us, INT8 exact 172 -> 165, single-half 3-9 % faster; exact ternary
    // 158 -> 159-160, so it keeps 2 x 2 at 128 rows).
    constexpr int WN = LO && F == Format::Ternary && BM == kBM ? 2 : 4;
    constexpr int WM = 4 / WN;
    constexpr int TI = BM / 16 / WM;             // 16-row MFMA tiles per wave
    constexpr int TJ = kBN / 16 / WN;            // 16-column MFMA tiles per wave
    constexpr int TJS = TJ / S;                  // column tiles per stream per wave
    constexpr int BNS = kBN / S;                 // block columns per stream
    constexpr int SPC = Chunk<F>::stages;
    // Raised wave priority over each half-stage's MFMAs for exact ternary
    // (165 -> 157-160 us); with the waves along n every other variant ran
    // as fast or faster without it (INT8 exact 168.6 against 165.3 us, NF4
    // single-half 150.7 against 144.1).
    constexpr bool PRIO = LO && F == Format::Ternary;
    __shared__ _Float16 As[2][PA][BM][kRow];   // [stage][hi, lo][row][k]
    __shared__ uint2 lut[F == Format::Nf4 ? 256 : 1];

    if constexpr (F == Format::Nf4) {
        // Entry for one code byte: x = hi halves of (low nibble, high nibble),
        // y = lo halves, each a packed binary16 pair for consecutive k.
        const uint32_t e = threadIdx.x;
        const float l0 = kLevels[e & 15], l1 = kLevels[e >> 4];
        const _Float16 h0 = _Float16(l0), h1 = _Float16(l1);
        const _Float16 r0 = _Float16(l0 - float(h0)), r1 = _Float16(l1 - float(h1));
        lut[e] = uint2{unsigned(__builtin_bit_cast(unsigned short, h0)) |
                           (unsigned(__builtin_bit_cast(unsigned short, h1)) << 16),
                       unsigned(__builtin_bit_cast(unsigned short, r0)) |
                           (unsigned(__builtin_bit_cast(unsigned short, r1)) << 16)};
    }

    // XCD-aware tile order over (chunk, tile) blocks.
    const uint32_t blocks = g.tiles * g.chunks;
    uint32_t block = blockIdx.x;
    if (blocks % 8 == 0)
        block = (blockIdx.x % 8) * (blocks / 8) + blockIdx.x / 8;
    const uint32_t chunk = block / g.tiles, tile = block % g.tiles;
    const uint32_t m0 = (tile / g.tiles_n) * BM, n0 = (tile % g.tiles_n) * BNS;
    const int tid = threadIdx.x, lane = tid & 63;
    // Wave-uniform, so the tile addresses live in scalar registers.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int li = lane & 15, lq = lane >> 4;
    const uint32_t chunk_stages = g.k / kBK / g.chunks;
    const uint32_t s_begin = chunk * chunk_stages, s_end = s_begin + chunk_stages;

    // A staging: thread -> (row, k run of kBK / TPR) of both activation
    // halves.  Rows past m load row 0 (their outputs are never stored), so
    // every load is unconditional and nothing waits to clear a destination.
    constexpr int TPR = kThreads / BM;            // threads per staged row
    constexpr int AV = kBK / TPR / 8;             // 8-half vectors per thread
    const uint32_t a_row = tid / TPR, a_k = (tid % TPR) * (kBK / TPR);
    const bool a_live = m0 + a_row < g.m;
    const _Float16 *a_src[2] = {g.xh + size_t(a_live ? m0 + a_row : 0) * g.k + a_k,
                                g.xl + size_t(a_live ? m0 + a_row : 0) * g.k + a_k};
    struct ARaw {
        v8h v[PA][AV];
    };
    auto fetch_a = [&](uint32_t s, ARaw &r) {
#pragma unroll
        for (int p = 0; p < PA; ++p)
#pragma unroll
            for (int u = 0; u < AV; ++u)
                r.v[p][u] = *reinterpret_cast<const v8h *>(a_src[p] + s * kBK + 8 * u);
    };
    auto store_a = [&](int buf, const ARaw &r) {
#pragma unroll
        for (int p = 0; p < PA; ++p)
#pragma unroll
            for (int u = 0; u < AV; ++u)
                *reinterpret_cast<v8h *>(&As[buf][p][a_row][a_k + 8 * u]) = r.v[p][u];
    };

    // The wave's weight tiles: column tile jt is tile tt of stream jt / TJS.
    const v4u *wptr[TJ];
    const void *sptr[TJ];
    bool wlive[TJ];
#pragma unroll
    for (int jt = 0; jt < TJ; ++jt) {
        const int st = jt / TJS, tt = jt % TJS;
        const uint32_t t = n0 / 16 + wn * TJS + tt;
        wlive[jt] = t < g.n_tiles;
        wptr[jt] = reinterpret_cast<const v4u *>(g.wtiles[st]) +
                   size_t(wlive[jt] ? t : 0) * g.tile_vecs + lane;
        sptr[jt] = HALF ? static_cast<const void *>(static_cast<const __half *>(g.scales[st]) +
                                                    size_t(wlive[jt] ? t : 0) * g.groups_pad * 16 +
                                                    li)
                        : static_cast<const void *>(static_cast<const float *>(g.scales[st]) +
                                                    size_t(wlive[jt] ? t : 0) * g.groups_pad * 16 +
                                                    li);
    }
    v4u cur[TJ];
    // Tiles past n read tile 0 (their columns are never stored).
    auto load_chunk = [&](uint32_t c, v4u (&dst)[TJ]) {
#pragma unroll
        for (int jt = 0; jt < TJ; ++jt)
            dst[jt] = wptr[jt][size_t(c) * 64];
    };

    v4f acc[TI][TJ], total[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int jt = 0; jt < TJ; ++jt) {
            acc[i][jt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            total[i][jt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }

    // Each lane's weight scales of a group, kept in their stored form:
    // loaded when the group starts and used at its end, so the in-order load
    // counter never makes an early instruction wait for them.
    typename std::conditional<HALF, unsigned short, float>::type gsc_raw[TJ];
    auto load_group_constants = [&](uint32_t grp) {
#pragma unroll
        for (int jt = 0; jt < TJ; ++jt) {
            if constexpr (HALF)
                gsc_raw[jt] = static_cast<const unsigned short *>(sptr[jt])[size_t(grp) * 16];
            else
                gsc_raw[jt] = static_cast<const float *>(sptr[jt])[size_t(grp) * 16];
        }
    };

    ARaw next;
    fetch_a(s_begin, next);
    load_chunk(s_begin / SPC, cur);
    load_group_constants(s_begin / 2);
    store_a(0, next);
    __syncthreads();

    // One 64-wide stage; a group is two stages.  With the group unrolled the
    // first MFMA of each tile starts from zero instead of a cleared
    // accumulator; INT8, whose tile load refills every stage, keeps one stage
    // per iteration (unrolled it spills) and clears after the epilogue.
    constexpr bool UNROLL = F != Format::Int8;
    auto stage = [&](uint32_t s, auto first_tag) {
        const bool FIRST = first_tag;
        const int buf = (s - s_begin) & 1;
        // The last stage re-fetches itself and stores to the idle buffer:
        // with no conditional fetch, no path leaves a load pending at the
        // loop's back edge.
        fetch_a(s + 1 < s_end ? s + 1 : s, next);
        if (FIRST && s != s_begin)
            load_group_constants(s / 2);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            v8h bh[TJ], bl[TJ];
#pragma unroll
            for (int jt = 0; jt < TJ; ++jt) {
                if constexpr (F == Format::Int8) {
                    bh[jt] = decode_i8(cur[jt], h);
                } else if constexpr (F == Format::Ternary) {
                    bh[jt] = decode_ternary(cur[jt][s % 4], h);
                } else {
                    const unsigned word = cur[jt][2 * (s % 2) + h];
                    v4u hi, lo;
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        const uint2 e = lut[(word >> (8 * p)) & 255u];
                        hi[p] = e.x;
                        lo[p] = e.y;
                    }
                    bh[jt] = __builtin_bit_cast(v8h, hi);
                    bl[jt] = __builtin_bit_cast(v8h, lo);
                }
            }
            // The chunk's last decode: its registers take the next chunk,
            // in flight behind this half's MFMAs.
            if (h == 1 && (s + 1) % SPC == 0 && s + 1 < s_end)
                load_chunk((s + 1) / SPC, cur);
            const int koff = F == Format::Nf4 ? 32 * h + 8 * lq : 16 * lq + 8 * h;
            if constexpr (PRIO)
                __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const int row = wm * (BM / WM) + i * 16 + li;
                const v8h ah = *reinterpret_cast<const v8h *>(&As[buf][0][row][koff]);
                const v8h al = *reinterpret_cast<const v8h *>(&As[buf][PA - 1][row][koff]);
#pragma unroll
                for (int jt = 0; jt < TJ; ++jt) {
                    v4f c;
                    if (UNROLL && FIRST && h == 0)
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[jt], v4f{}, 0, 0, 0);
                    else
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[jt], acc[i][jt], 0, 0,
                                                                   0);
                    if constexpr (LO)
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[jt], c, 0, 0, 0);
                    if constexpr (P == 2)
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[jt], c, 0, 0, 0);
                    acc[i][jt] = c;
                }
            }
            if constexpr (PRIO)
                __builtin_amdgcn_s_setprio(0);
        }
        if (!FIRST) {
            // Group epilogue: total += group_sum * scale[n].
            float gsc[TJ];
#pragma unroll
            for (int jt = 0; jt < TJ; ++jt) {
                if constexpr (HALF)
                    gsc[jt] = __half2float(__ushort_as_half(gsc_raw[jt]));
                else
                    gsc[jt] = gsc_raw[jt];
            }
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int jt = 0; jt < TJ; ++jt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        total[i][jt][r] = fmaf(acc[i][jt][r], gsc[jt], total[i][jt][r]);
                        if (!UNROLL)
                            acc[i][jt][r] = 0.0f;
                    }
        }
        store_a(buf ^ 1, next);
        __syncthreads();
    };
    // Chunks are whole groups, so every run starts on a group's first stage.
    if constexpr (UNROLL) {
        for (uint32_t s = s_begin; s < s_end; s += 2) {
            stage(s, std::true_type{});
            stage(s + 1, std::false_type{});
        }
    } else {
        for (uint32_t s = s_begin; s < s_end; ++s)
            stage(s, (s - s_begin) % 2 == 0);
    }

    // The rows' 2^e (rows past m read row 0; they are never stored).
    float rowf[TI][4];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t mm = m0 + wm * (BM / WM) + i * 16 + lq * 4 + r;
            rowf[i][r] = g.factor[mm < g.m ? mm : 0];
        }
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t mm = m0 + wm * (BM / WM) + i * 16 + lq * 4 + r;
            if (mm >= g.m)
                continue;
#pragma unroll
            for (int tt = 0; tt < TJS; ++tt) {
                const uint32_t nn = n0 + (wn * TJS + tt) * 16 + li;
                if (nn >= g.n)
                    continue;
                const size_t o = size_t(mm) * g.n + nn;
                const float rf = rowf[i][r];
                if (g.chunks > 1) {
                    // Chunk sums; splitk_reduce_kernel finishes them.
                    const size_t plane = size_t(g.m) * g.n;
#pragma unroll
                    for (int st = 0; st < S; ++st)
                        g.partial[(size_t(chunk) * S + st) * plane + o] =
                            total[i][st * TJS + tt][r] * rf;
                    continue;
                }
                if constexpr (E == Epilogue::Single) {
                    g.out[0][o] = total[i][tt][r] * rf;
                } else if constexpr (E == Epilogue::Pair) {
                    g.out[0][o] = total[i][tt][r] * rf;
                    g.out[1][o] = total[i][(S - 1) * TJS + tt][r] * rf;
                } else {
                    g.out[0][o] = silu_mul(total[i][tt][r] * rf,
                                           total[i][(S - 1) * TJS + tt][r] * rf);
                }
            }
        }
}

// Split-K epilogue: chunk sums in chunk order, then the operation's epilogue.
template <int S, Epilogue E>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(float *__restrict__ out0,
                                                            float *__restrict__ out1,
                                                            const float *__restrict__ partial,
                                                            size_t plane, uint32_t chunks)
{
    const size_t stride = size_t(gridDim.x) * 256;
    for (size_t o = size_t(blockIdx.x) * 256 + threadIdx.x; o < plane; o += stride) {
        float v[S];
#pragma unroll
        for (int st = 0; st < S; ++st) {
            float sum = 0.0f;
            for (uint32_t c = 0; c < chunks; ++c)
                sum += partial[(size_t(c) * S + st) * plane + o];
            v[st] = sum;
        }
        if constexpr (E == Epilogue::Single) {
            out0[o] = v[0];
        } else if constexpr (E == Epilogue::Pair) {
            out0[o] = v[0];
            out1[o] = v[S - 1];
        } else {
            out0[o] = silu_mul(v[0], v[S - 1]);
        }
    }
}

template <Format F, int S, Epilogue E, int BM>
void launch_rows(hipStream_t stream, const GemmArgs &args, bool half, bool lo)
{
    const unsigned grid = args.tiles * args.chunks;
    if (half && lo)
        gemm_mfma_kernel<F, S, E, true, true, BM><<<grid, kThreads, 0, stream>>>(args);
    else if (lo)
        gemm_mfma_kernel<F, S, E, false, true, BM><<<grid, kThreads, 0, stream>>>(args);
    else if (half)
        gemm_mfma_kernel<F, S, E, true, false, BM><<<grid, kThreads, 0, stream>>>(args);
    else
        gemm_mfma_kernel<F, S, E, false, false, BM><<<grid, kThreads, 0, stream>>>(args);
}

template <Format F, int S, Epilogue E>
void launch_epilogue(hipStream_t stream, const GemmArgs &args, bool half, bool lo, uint32_t bm)
{
    if (bm == kBM)
        launch_rows<F, S, E, kBM>(stream, args, half, lo);
    else
        launch_rows<F, S, E, kBM / 2>(stream, args, half, lo);
    if (args.chunks > 1) {
        const size_t plane = size_t(args.m) * args.n;
        const unsigned rgrid = unsigned(std::min<size_t>((plane + 255) / 256, 65536));
        splitk_reduce_kernel<S, E><<<rgrid, 256, 0, stream>>>(args.out[0], args.out[1],
                                                              args.partial, plane, args.chunks);
    }
}

template <Format F>
void launch_format(hipStream_t stream, const PackedCall &call, const GemmArgs &args, bool half,
                   uint32_t bm)
{
    const bool lo = !call.single_half;
    switch (call.epilogue) {
    case Epilogue::Single:
        return launch_epilogue<F, 1, Epilogue::Single>(stream, args, half, lo, bm);
    case Epilogue::Pair:
        return launch_epilogue<F, 2, Epilogue::Pair>(stream, args, half, lo, bm);
    case Epilogue::SwigluPair:
        return launch_epilogue<F, 2, Epilogue::SwigluPair>(stream, args, half, lo, bm);
    }
}

// K chunks for a grid of `tiles` output tiles: the most chunks (any divisor
// of the group count, each at least two groups deep) that keep the grid
// within two blocks per CU.  A small-M product is a chain of its stages, so
// more, shorter chunks finish sooner: LFM2-350M-shape prefill (M = 128)
// 57-58k -> 68k tok/s against power-of-two chunks of at least four groups.
// One-group chunks (65k tok/s) and grids of up to four blocks per CU (M = 512
// x 8192 x 2048: 61 -> 72 us) measured slower.
uint32_t split_chunks(uint32_t tiles, uint32_t groups)
{
    uint32_t chunks = 1;
    for (uint32_t c = 2; c <= groups / 2; ++c)
        if (groups % c == 0 && tiles * c <= 512)
            chunks = c;
    return chunks;
}

uint32_t tiles_of(const PackedCall &call, uint32_t *tiles_n, uint32_t bm)
{
    const int S = call.epilogue == Epilogue::Single ? 1 : 2;
    *tiles_n = (call.n + kBN / S - 1) / (kBN / S);
    return *tiles_n * ((call.m + bm - 1) / bm);
}

// Rows per block tile: 64 where 128-row tiles would not fill the grid
// without a K split (fewer than kHalfRowsBelow tiles), so the product
// needs fewer K chunks (none at M = 512 x 8192) and their reduction --
// except for ternary and NF4 at long K past 512 rows, where the 128-row
// tiles and their split measured faster.  Measured (us per call, A/B on one device): M = 512 x
// 8192 x 2048 ternary 58.4 -> 50.0, INT8 61.3 -> 50.0-50.9, NF4 70-73 ->
// 62.6-63.5; M = 2048 x 2048 x 2048 ternary 63.5 -> 58.3-59.2, NF4 76.3 ->
// 69.6; M = 128 35.6 -> 30.1; M = 256 41.8 -> 39.0; M = 512 x 2048 x 8192
// 2-7 % faster; but M = 2048 x 2048 x 8192 ternary 156.1-156.6 with the
// split against 159.8-160.1, NF4 209.2-209.5 against 213.5-214.5, M = 1024
// ternary 95.8 against 98.7-100 (INT8 164.8-166.5 against 169.3-169.8: it
// keeps the 64-row tiles).
constexpr uint32_t kHalfRowsBelow = 512;
uint32_t block_rows(const PackedCall &call)
{
    uint32_t tiles_n;
    const bool split = tiles_of(call, &tiles_n, kBM) < kHalfRowsBelow;
    return split && (call.k <= 4096 || call.m <= 512 || call.format == Format::Int8) ? kBM / 2
                                                                                     : kBM;
}

}  // namespace

size_t gemm_mfma_scratch_bytes(const PackedCall &call)
{
    uint32_t tiles_n;
    const uint32_t chunks =
        split_chunks(tiles_of(call, &tiles_n, block_rows(call)), call.k / 128);
    const int S = call.epilogue == Epilogue::Single ? 1 : 2;
    const size_t partial = chunks > 1 ? size_t(chunks) * S * call.m * call.n * sizeof(float) : 0;
    return size_t(call.m) * call.k * 2 * sizeof(_Float16) + size_t(call.m) * sizeof(float) +
           partial;
}

void launch_gemm_mfma(hipStream_t stream, const PackedCall &call, void *scratch)
{
    const uint32_t groups = call.k / 128;
    char *p = static_cast<char *>(scratch);
    _Float16 *xh = reinterpret_cast<_Float16 *>(p);
    _Float16 *xl = xh + size_t(call.m) * call.k;
    float *factor = reinterpret_cast<float *>(xl + size_t(call.m) * call.k);
    split_kernel<<<call.m, kSplitThreads, 0, stream>>>(call.x, call.k, xh,
                                                       call.single_half ? nullptr : xl, factor);
    // The repacked tiles pad K to 256 (ternary) or 128; one 16-byte lane load
    // covers 64 (INT8), 128 (NF4) or 256 (ternary) k.
    const uint32_t align = call.format == Format::Ternary ? 256 : 128;
    const uint32_t k_pad = (call.k + align - 1) / align * align;
    const uint32_t chunk_k =
        call.format == Format::Int8 ? 64 : call.format == Format::Nf4 ? 128 : 256;
    GemmArgs args{};
    args.xh = xh;
    args.xl = xl;
    args.factor = factor;
    args.wtiles[0] = call.a.tiles;
    args.wtiles[1] = call.b.tiles;
    args.scales[0] = call.a.tiled_scales;
    args.scales[1] = call.b.tiled_scales;
    args.out[0] = call.out_a;
    args.out[1] = call.out_b;
    args.m = call.m;
    args.n = call.n;
    args.k = call.k;
    args.n_tiles = (call.n + 63) / 64 * 4;
    args.tile_vecs = k_pad / chunk_k * 64;
    args.groups_pad = k_pad / 128;
    const uint32_t bm = block_rows(call);
    args.tiles = tiles_of(call, &args.tiles_n, bm);
    args.chunks = split_chunks(args.tiles, groups);
    args.partial = factor + call.m;
    const int streams = call.epilogue == Epilogue::Single ? 1 : 2;
    const bool half = call.a.tiled_half && (streams == 1 || call.b.tiled_half);
    switch (call.format) {
    case Format::Ternary: launch_format<Format::Ternary>(stream, call, args, half, bm); break;
    case Format::Nf4: launch_format<Format::Nf4>(stream, call, args, half, bm); break;
    case Format::Int8: launch_format<Format::Int8>(stream, call, args, half, bm); break;
    }
}

}  // namespace mfh
