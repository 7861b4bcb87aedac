// Matrix-core prefill GEMM for packed ternary / NF4 / INT8 weights (m > 8).
//
// out[m, n] = sum_g scale[n, g] * sum_{k in g} x[m, k] * level(code[n, k]),
// the reference's group-then-scale order (kernels-simd/src/lib.rs:54,205).
//
// Exactness plan.
// - The activation prologue (split_kernel) scales every (row, 128-group) by
//   2^-e so its largest magnitude is below 1, and splits each value as
//   x = hi + lo with both halves binary16 (22 significant bits).
// - Weight levels are exact in binary16 for ternary (-1, 0, 1, 2) and INT8
//   (-127..127).  NF4 levels are split the same way as the activations.
// - v_mfma_f32_16x16x32_f16 forms the products exactly in f32 and
//   accumulates each 128-group separately.
// - The group epilogue adds group_sum * (2^e * scale) in f32.  2^e is a
//   power of two, so this equals the reference's scale * dot.  NF4 drops
//   the lo * lo product, which is below 2^-22 of each term.
//
// Tiling.  A 512-lane block computes a 128 (m) x 128 (n) output tile, split
// over S weight streams of 128 / S columns each.  Eight waves (4 x 2) own
// 32 x 64 (S = 1) or 32 x 32-per-stream (S = 2) pieces.  K advances in
// kBK-wide stages: the activation halves and the decoded weight levels are
// staged through LDS, double buffered.  The load of stage s + 1 runs from
// global memory while stage s feeds the MFMAs.
//
// Grid mapping.  Workgroups are dealt round-robin to the 8 XCDs.  Block b
// computes tile (b % 8) * (tiles / 8) + b / 8, so each XCD's L2 holds a
// contiguous run of tiles: neighbouring n-tiles of the same m rows.
#include <algorithm>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace mfh {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

#ifndef MFH_GEMM_KBK
#define MFH_GEMM_KBK 64
#endif
constexpr int kThreads = 512;     // 8 waves: 4 (m) x 2 (n)
constexpr int kBM = 128;          // rows per block tile
constexpr int kBN = 128;          // columns per block tile (all streams)
constexpr int kBK = MFH_GEMM_KBK; // k per stage (32 or 64: whole MFMA k-blocks)
// LDS row pitch in halves: kBK + 8 (80 or 144 bytes) puts the 16 rows read
// by one lane group on distinct banks.
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

// One wave per (128-group, row): factor[m, g] = 2^e (NaN for a group with a
// non-finite value) and the binary16 halves of x * 2^-e.
__global__ __launch_bounds__(64) void split_kernel(const float *__restrict__ x, uint32_t m,
                                                   uint32_t k, _Float16 *__restrict__ xh,
                                                   _Float16 *__restrict__ xl,
                                                   float *__restrict__ factor)
{
    const uint32_t g = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
    const uint32_t groups = k / 128;
    const float *src = x + size_t(row) * k + g * 128;
    float v[2];
    bool bad = false;
    float mx = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        v[h] = src[h * 64 + lane];
        if (!isfinite(v[h])) {
            bad = true;
            v[h] = 0.0f;
        }
        mx = fmaxf(mx, fabsf(v[h]));
    }
    bad = __any(bad);
    mx = wave_max(mx);
    int e = 0;
    if (mx > 0.0f)
        frexpf(mx, &e);  // |x| < 2^e
    if (lane == 0)
        factor[size_t(row) * groups + g] = bad ? __builtin_nanf("") : ldexpf(1.0f, e);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float s = ldexpf(v[h], -e);
        const _Float16 hi = _Float16(s);
        const size_t o = size_t(row) * k + g * 128 + h * 64 + lane;
        xh[o] = hi;
        xl[o] = _Float16(s - float(hi));
    }
}

struct GemmArgs {
    const _Float16 *xh, *xl;
    const float *factor;  // [m, k / 128]
    const uint8_t *codes[2];
    const float *scales[2];
    float *out[2];
    float *partial;       // split-K: [chunk][stream][m][n] raw sums
    uint32_t m, n, k;
    uint32_t tiles_n, tiles;
    uint32_t chunks;      // K split into `chunks` runs of whole groups
};

// Level planes of one weight stream: NF4 needs hi and lo.
template <Format F> struct Planes {
    static constexpr int value = F == Format::Nf4 ? 2 : 1;
};

// The 16 codes of one (n, 16-k) chunk as loaded: INT8 16 bytes, ternary 4,
// NF4 8.
template <Format F> struct Codes16;
template <> struct Codes16<Format::Int8> { typedef uint4 type; };
template <> struct Codes16<Format::Ternary> { typedef unsigned type; };
template <> struct Codes16<Format::Nf4> { typedef uint2 type; };

// Load one chunk, or the codes of level 0 for a row past n.
template <Format F>
__device__ __forceinline__ typename Codes16<F>::type load_codes16(const uint8_t *src, bool live)
{
    if constexpr (F == Format::Int8)
        return live ? *reinterpret_cast<const uint4 *>(src) : uint4{0, 0, 0, 0};
    else if constexpr (F == Format::Ternary)
        return live ? *reinterpret_cast<const unsigned *>(src) : 0x55555555u;
    else
        return live ? *reinterpret_cast<const uint2 *>(src) : uint2{0x77777777u, 0x77777777u};
}

// Decode a chunk to binary16 levels (NF4: hi and lo planes).
template <Format F>
__device__ __forceinline__ void decode16(const typename Codes16<F>::type &c,
                                         const _Float16 (*nf)[16], v8h (&hi)[2], v8h (&lo)[2])
{
    if constexpr (F == Format::Int8) {
        const unsigned words[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int i = 0; i < 16; ++i)
            hi[i / 8][i % 8] = _Float16(float(int8_t(words[i / 4] >> (8 * (i % 4)))));
    } else if constexpr (F == Format::Ternary) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            hi[i / 8][i % 8] = _Float16(float(int((c >> (2 * i)) & 3u) - 1));
    } else {
        const unsigned words[2] = {c.x, c.y};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const unsigned code = (words[i / 8] >> (4 * (i % 8))) & 15u;
            hi[i / 8][i % 8] = nf[0][code];
            lo[i / 8][i % 8] = nf[1][code];
        }
    }
}

template <Format F, int S, Epilogue E>
__global__ __launch_bounds__(kThreads) void gemm_mfma_kernel(GemmArgs g)
{
    constexpr int P = Planes<F>::value;
    constexpr int BNS = kBN / S;       // columns per stream
    constexpr int TI = kBM / 4 / 16;   // 16-row tiles per wave (4 wave rows)
    constexpr int TJ = BNS / 2 / 16;   // 16-column tiles per stream per wave (2 wave columns)
    constexpr int KB = kBK / 32;       // MFMA k-blocks per stage
    constexpr int SPG = 128 / kBK;     // stages per 128-group
    __shared__ _Float16 As[2][2][kBM][kRow];          // [stage][hi, lo][row][k]
    __shared__ _Float16 Bs[2][S][P][BNS][kRow];       // [stage][stream][plane][n][k]
    __shared__ _Float16 nf[2][16];

    if constexpr (F == Format::Nf4) {
        if (threadIdx.x < 16) {
            const float l = kLevels[threadIdx.x];
            const _Float16 h = _Float16(l);
            nf[0][threadIdx.x] = h;
            nf[1][threadIdx.x] = _Float16(l - float(h));
        }
        __syncthreads();
    }

    // XCD-aware tile order over (chunk, tile) blocks.
    const uint32_t blocks = g.tiles * g.chunks;
    uint32_t block = blockIdx.x;
    if (blocks % 8 == 0)
        block = (blockIdx.x % 8) * (blocks / 8) + blockIdx.x / 8;
    const uint32_t chunk = block / g.tiles, tile = block % g.tiles;
    const uint32_t m0 = (tile / g.tiles_n) * kBM, n0 = (tile % g.tiles_n) * BNS;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t groups = g.k / 128;
    const uint32_t chunk_stages = g.k / kBK / g.chunks;
    const uint32_t s_begin = chunk * chunk_stages, s_end = s_begin + chunk_stages;
    const size_t row_bytes = size_t(g.k) / weights_per_byte(F);

    // Global -> register staging, 16 consecutive k per thread and operand:
    // A = (row, k part) of both halves; B = (stream, n, k part).
    constexpr int APR = kBK / 16;  // A threads per row
    const uint32_t a_row = tid / APR, a_k = (tid % APR) * 16;
    const bool a_live = m0 + a_row < g.m;
    const uint32_t b_st = tid / (kThreads / S), b_local = tid % (kThreads / S);
    const uint32_t b_n = b_local / APR, b_k = (b_local % APR) * 16;
    const bool b_live = n0 + b_n < g.n;
    const uint8_t *b_src = g.codes[b_st] + size_t(b_live ? n0 + b_n : 0) * row_bytes;
    const _Float16 *a_hi = g.xh + size_t(a_live ? m0 + a_row : 0) * g.k;
    const _Float16 *a_lo = g.xl + size_t(a_live ? m0 + a_row : 0) * g.k;

    // One stage of this thread's operands as loaded from global memory:
    // the activation halves and the undecoded codes.  Two such sets are in
    // flight: stage s + 2 loads while stage s computes from LDS and stage
    // s + 1 waits in registers to be decoded into LDS.
    struct Raw {
        v8h a[2][2];
        typename Codes16<F>::type b;
    };
    auto fetch = [&](uint32_t s, Raw &r) {
        const uint32_t k0 = s * kBK + a_k;
        if (a_live) {
            const v8h *ph = reinterpret_cast<const v8h *>(a_hi + k0);
            const v8h *pl = reinterpret_cast<const v8h *>(a_lo + k0);
            r.a[0][0] = ph[0];
            r.a[0][1] = ph[1];
            r.a[1][0] = pl[0];
            r.a[1][1] = pl[1];
        } else {
            const v8h z = {};
            r.a[0][0] = r.a[0][1] = r.a[1][0] = r.a[1][1] = z;
        }
        r.b = load_codes16<F>(b_src + size_t(s * kBK + b_k) / weights_per_byte(F), b_live);
    };
    auto store = [&](int buf, const Raw &r) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            *reinterpret_cast<v8h *>(&As[buf][p][a_row][a_k]) = r.a[p][0];
            *reinterpret_cast<v8h *>(&As[buf][p][a_row][a_k + 8]) = r.a[p][1];
        }
        v8h b_hi[2], b_lo[2];
        decode16<F>(r.b, nf, b_hi, b_lo);
        *reinterpret_cast<v8h *>(&Bs[buf][b_st][0][b_n][b_k]) = b_hi[0];
        *reinterpret_cast<v8h *>(&Bs[buf][b_st][0][b_n][b_k + 8]) = b_hi[1];
        if constexpr (P == 2) {
            *reinterpret_cast<v8h *>(&Bs[buf][b_st][1][b_n][b_k]) = b_lo[0];
            *reinterpret_cast<v8h *>(&Bs[buf][b_st][1][b_n][b_k + 8]) = b_lo[1];
        }
    };

    v4f acc[S][TI][TJ], total[S][TI][TJ];
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                acc[st][i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
                total[st][i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            }

    const int li = lane & 15, lq = lane >> 4;
    const int row_base = wm * (kBM / 4), col_base = wn * (BNS / 2);
    // The group's constants, loaded when the group starts and applied when
    // it ends: 2^e per activation row and the weight scale per column.
    float gfx[TI][4], gsc[S][TJ];
    auto load_group_constants = [&](uint32_t grp) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t mm = m0 + row_base + i * 16 + lq * 4 + r;
                gfx[i][r] = mm < g.m ? g.factor[size_t(mm) * groups + grp] : 0.0f;
            }
#pragma unroll
        for (int st = 0; st < S; ++st)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const uint32_t nn = n0 + col_base + j * 16 + li;
                gsc[st][j] = nn < g.n ? g.scales[st][size_t(nn) * groups + grp] : 0.0f;
            }
    };

    // One stage: `next` holds stage s + 1 (loaded a stage ago), `freed`
    // held stage s (already in LDS) and receives stage s + 2.
    auto step = [&](uint32_t s, Raw &next, Raw &freed) {
        const int buf = (s - s_begin) & 1;
        if (s + 2 < s_end)
            fetch(s + 2, freed);
        if (s % SPG == 0)
            load_group_constants(s / SPG);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            v8h ah[TI], al[TI];
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const int row = row_base + i * 16 + li;
                ah[i] = *reinterpret_cast<const v8h *>(&As[buf][0][row][kb * 32 + lq * 8]);
                al[i] = *reinterpret_cast<const v8h *>(&As[buf][1][row][kb * 32 + lq * 8]);
            }
#pragma unroll
            for (int st = 0; st < S; ++st)
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    const int nrow = col_base + j * 16 + li;
                    const v8h bh =
                        *reinterpret_cast<const v8h *>(&Bs[buf][st][0][nrow][kb * 32 + lq * 8]);
                    v8h bl;
                    if constexpr (P == 2)
                        bl = *reinterpret_cast<const v8h *>(
                            &Bs[buf][st][1][nrow][kb * 32 + lq * 8]);
#pragma unroll
                    for (int i = 0; i < TI; ++i) {
                        v4f c = acc[st][i][j];
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bh, c, 0, 0, 0);
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bh, c, 0, 0, 0);
                        if constexpr (P == 2)
                            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bl, c, 0, 0, 0);
                        acc[st][i][j] = c;
                    }
                }
        }
        if (s % SPG == SPG - 1) {
            // Group epilogue: total += group_sum * (2^e[m] * scale[n]).
#pragma unroll
            for (int st = 0; st < S; ++st)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
#pragma unroll
                    for (int i = 0; i < TI; ++i) {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            total[st][i][j][r] += acc[st][i][j][r] * (gfx[i][r] * gsc[st][j]);
                        acc[st][i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
                    }
        }
        if (s + 1 < s_end)
            store(buf ^ 1, next);
        __syncthreads();
    };

    Raw r0, r1;
    fetch(s_begin, r0);
    if (s_begin + 1 < s_end)
        fetch(s_begin + 1, r1);
    store(0, r0);
    __syncthreads();
    for (uint32_t s = s_begin; s < s_end; s += 2) {
        step(s, r1, r0);
        if (s + 1 < s_end)
            step(s + 1, r0, r1);
    }

#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t mm = m0 + row_base + i * 16 + lq * 4 + r;
            if (mm >= g.m)
                continue;
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const uint32_t nn = n0 + col_base + j * 16 + li;
                if (nn >= g.n)
                    continue;
                const size_t o = size_t(mm) * g.n + nn;
                if (g.chunks > 1) {
                    // Raw sums per chunk; splitk_reduce_kernel finishes them.
                    const size_t plane = size_t(g.m) * g.n;
#pragma unroll
                    for (int st = 0; st < S; ++st)
                        g.partial[(size_t(chunk) * S + st) * plane + o] = total[st][i][j][r];
                    continue;
                }
                if constexpr (E == Epilogue::Single) {
                    g.out[0][o] = total[0][i][j][r];
                } else if constexpr (E == Epilogue::Pair) {
                    g.out[0][o] = total[0][i][j][r];
                    g.out[1][o] = total[S - 1][i][j][r];
                } else {
                    g.out[0][o] = silu_mul(total[0][i][j][r], total[S - 1][i][j][r]);
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

template <Format F>
void launch_format(hipStream_t stream, const PackedCall &call, const GemmArgs &args)
{
    const unsigned grid = args.tiles * args.chunks;
    const size_t plane = size_t(args.m) * args.n;
    const unsigned rgrid = unsigned(std::min<size_t>((plane + 255) / 256, 65536));
    switch (call.epilogue) {
    case Epilogue::Single:
        gemm_mfma_kernel<F, 1, Epilogue::Single><<<grid, kThreads, 0, stream>>>(args);
        if (args.chunks > 1)
            splitk_reduce_kernel<1, Epilogue::Single><<<rgrid, 256, 0, stream>>>(
                args.out[0], args.out[1], args.partial, plane, args.chunks);
        break;
    case Epilogue::Pair:
        gemm_mfma_kernel<F, 2, Epilogue::Pair><<<grid, kThreads, 0, stream>>>(args);
        if (args.chunks > 1)
            splitk_reduce_kernel<2, Epilogue::Pair><<<rgrid, 256, 0, stream>>>(
                args.out[0], args.out[1], args.partial, plane, args.chunks);
        break;
    case Epilogue::SwigluPair:
        gemm_mfma_kernel<F, 2, Epilogue::SwigluPair><<<grid, kThreads, 0, stream>>>(args);
        if (args.chunks > 1)
            splitk_reduce_kernel<2, Epilogue::SwigluPair><<<rgrid, 256, 0, stream>>>(
                args.out[0], args.out[1], args.partial, plane, args.chunks);
        break;
    }
}

// K chunks for a grid of `tiles` output tiles: enough to give every CU a
// block, in whole groups, each chunk at least 4 groups deep.
uint32_t split_chunks(uint32_t tiles, uint32_t groups)
{
    uint32_t chunks = 1;
    while (tiles * chunks * 2 <= 256 && groups % (chunks * 2) == 0 && groups / (chunks * 2) >= 4)
        chunks *= 2;
    return chunks;
}

}  // namespace

namespace {

uint32_t tiles_of(const PackedCall &call, uint32_t *tiles_n)
{
    const int S = call.epilogue == Epilogue::Single ? 1 : 2;
    *tiles_n = (call.n + kBN / S - 1) / (kBN / S);
    return *tiles_n * ((call.m + kBM - 1) / kBM);
}

}  // namespace

size_t gemm_mfma_scratch_bytes(const PackedCall &call)
{
    uint32_t tiles_n;
    const uint32_t chunks = split_chunks(tiles_of(call, &tiles_n), call.k / 128);
    const int S = call.epilogue == Epilogue::Single ? 1 : 2;
    const size_t partial = chunks > 1 ? size_t(chunks) * S * call.m * call.n * sizeof(float) : 0;
    return size_t(call.m) * call.k * 2 * sizeof(_Float16) +
           size_t(call.m) * (call.k / 128) * sizeof(float) + partial;
}

void launch_gemm_mfma(hipStream_t stream, const PackedCall &call, void *scratch)
{
    const uint32_t groups = call.k / 128;
    char *p = static_cast<char *>(scratch);
    _Float16 *xh = reinterpret_cast<_Float16 *>(p);
    _Float16 *xl = xh + size_t(call.m) * call.k;
    float *factor = reinterpret_cast<float *>(xl + size_t(call.m) * call.k);
    split_kernel<<<dim3(groups, call.m), 64, 0, stream>>>(call.x, call.m, call.k, xh, xl, factor);
    GemmArgs args{};
    args.xh = xh;
    args.xl = xl;
    args.factor = factor;
    args.codes[0] = call.a.codes;
    args.codes[1] = call.b.codes;
    args.scales[0] = call.a.scales;
    args.scales[1] = call.b.scales;
    args.out[0] = call.out_a;
    args.out[1] = call.out_b;
    args.m = call.m;
    args.n = call.n;
    args.k = call.k;
    args.tiles = tiles_of(call, &args.tiles_n);
    args.chunks = split_chunks(args.tiles, groups);
    args.partial = factor + size_t(call.m) * groups;
    switch (call.format) {
    case Format::Ternary: launch_format<Format::Ternary>(stream, call, args); break;
    case Format::Nf4: launch_format<Format::Nf4>(stream, call, args); break;
    case Format::Int8: launch_format<Format::Int8>(stream, call, args); break;
    }
}

}  // namespace mfh
