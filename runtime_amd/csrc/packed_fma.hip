// FP32-FMA packed kernels: decode GEMV (m <= 8), LDS-tiled prefill GEMM,
// row gather, SwiGLU staging and fill.
//
// Weight decode follows crates/kernels-simd/src/lib.rs:31-208:
//   ternary  w = ((byte[j/4] >> 2*(j%4)) & 3) - 1     (32 B per 128 weights)
//   nf4      w = NF4[nibble], low nibble first         (64 B per 128 weights)
//   int8     w = (i8) byte                             (128 B per 128 weights)
// Every kernel reduces one 128-weight group, then applies that group's scale,
// the reference's group-then-scale order (lib.rs:54,168,205).  Only the
// order of additions inside a group differs from the CPU.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace mfh {
namespace {

__constant__ float kNf4Levels[16] = {
    -1.0f,        -0.6961928f,  -0.52507305f, -0.3949175f,
    -0.28444138f, -0.18477343f, -0.091050036f, 0.0f,
    0.0795803f,   0.1609302f,   0.2461123f,   0.33791524f,
    0.44070983f,  0.562617f,    0.72295684f,  1.0f,
};

template <Format F>
struct ChunkBytes;  // code bytes holding 16 consecutive weights of one row
template <> struct ChunkBytes<Format::Ternary> { static constexpr int value = 4; };
template <> struct ChunkBytes<Format::Nf4> { static constexpr int value = 8; };
template <> struct ChunkBytes<Format::Int8> { static constexpr int value = 16; };

// Raw code words of one 16-weight chunk.
struct Words {
    uint32_t w[4];
};

template <Format F>
__device__ __forceinline__ Words load_chunk(const uint8_t *p)
{
    Words out{};
    if constexpr (F == Format::Ternary) {
        out.w[0] = *reinterpret_cast<const uint32_t *>(p);
    } else if constexpr (F == Format::Nf4) {
        uint2 v = *reinterpret_cast<const uint2 *>(p);
        out.w[0] = v.x;
        out.w[1] = v.y;
    } else {
        uint4 v = *reinterpret_cast<const uint4 *>(p);
        out.w[0] = v.x;
        out.w[1] = v.y;
        out.w[2] = v.z;
        out.w[3] = v.w;
    }
    return out;
}

// Unscaled levels of the 16 weights in a chunk.
template <Format F>
__device__ __forceinline__ void decode_chunk(const Words &c, float w[16], const float *lut)
{
    if constexpr (F == Format::Ternary) {
#pragma unroll
        for (int j = 0; j < 16; ++j)
            w[j] = float((c.w[0] >> (2 * j)) & 3u) - 1.0f;
    } else if constexpr (F == Format::Nf4) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            w[j] = lut[(c.w[0] >> (4 * j)) & 15u];
            w[8 + j] = lut[(c.w[1] >> (4 * j)) & 15u];
        }
    } else {
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                w[4 * d + j] = float(int8_t((c.w[d] >> (8 * j)) & 0xFFu));
    }
}

__device__ __forceinline__ float load_scale(const PackedStream &s, size_t index)
{
    if (s.scales16)
        return __half2float(reinterpret_cast<const __half *>(s.scales16)[index]);
    return s.scales[index];
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        v += __shfl_xor(v, offset, 64);
    return v;
}

__device__ __forceinline__ float silu_mul(float gate, float up)
{
    // (g * (1 / (1 + exp(-g)))) * u, backend-cpu/src/packed.rs:361-362.
    float sigmoid = 1.0f / (1.0f + expf(-gate));
    return (gate * sigmoid) * up;
}

// ---------------------------------------------------------------------------
// Decode GEMV: one wave owns kRows weight rows and strides the whole K range
// with 16 weights per lane per step, so the wave's code loads are contiguous
// row segments and each activation chunk in registers serves kRows rows.
// ---------------------------------------------------------------------------
constexpr int kGemvRows = 4;
constexpr int kGemvWaves = 4;

template <Format F, int BM, Epilogue E>
__global__ __launch_bounds__(256) void gemv_fma_kernel(PackedCall call)
{
    constexpr int S = (E == Epilogue::Single) ? 1 : 2;
    constexpr int CB = ChunkBytes<F>::value;
    __shared__ float lut[16];
    if (threadIdx.x < 16)
        lut[threadIdx.x] = kNf4Levels[threadIdx.x];
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t row0 = (blockIdx.x * kGemvWaves + wave) * kGemvRows;
    const uint32_t n = call.n, k = call.k, m = call.m;
    const uint32_t chunks = k / 16;
    const size_t row_bytes = size_t(k) / weights_per_byte(F);
    const uint32_t groups = k / 128;

    float acc[S][kGemvRows][BM];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r)
#pragma unroll
            for (int b = 0; b < BM; ++b)
                acc[s][r][b] = 0.0f;

    for (uint32_t c = lane; c < chunks; c += 64) {
        Words words[S][kGemvRows];
        float scale[S][kGemvRows];
#pragma unroll
        for (int r = 0; r < kGemvRows; ++r) {
            uint32_t row = row0 + r;
            if (row < n) {
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const PackedStream &st = s ? call.b : call.a;
                    words[s][r] = load_chunk<F>(st.codes + row * row_bytes + size_t(c) * CB);
                    scale[s][r] = load_scale(st, size_t(row) * groups + c / 8);
                }
            } else {
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    words[s][r] = Words{};
                    scale[s][r] = 0.0f;
                }
            }
        }
        float xv[BM][16];
#pragma unroll
        for (int b = 0; b < BM; ++b) {
            if (uint32_t(b) < m) {
                const float4 *xp =
                    reinterpret_cast<const float4 *>(call.x + size_t(b) * k + size_t(c) * 16);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float4 v = xp[q];
                    xv[b][4 * q + 0] = v.x;
                    xv[b][4 * q + 1] = v.y;
                    xv[b][4 * q + 2] = v.z;
                    xv[b][4 * q + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    xv[b][j] = 0.0f;
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int r = 0; r < kGemvRows; ++r) {
                float w[16];
                decode_chunk<F>(words[s][r], w, lut);
#pragma unroll
                for (int b = 0; b < BM; ++b) {
                    float partial = 0.0f;
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        partial += w[j] * xv[b][j];
                    acc[s][r][b] += scale[s][r] * partial;
                }
            }
    }

#pragma unroll
    for (int r = 0; r < kGemvRows; ++r) {
        uint32_t row = row0 + r;
#pragma unroll
        for (int b = 0; b < BM; ++b) {
            float va = wave_sum(acc[0][r][b]);
            float vb = (S == 2) ? wave_sum(acc[S - 1][r][b]) : 0.0f;
            if (lane == 0 && row < n && uint32_t(b) < m) {
                size_t o = size_t(b) * n + row;
                if constexpr (E == Epilogue::Single) {
                    call.out_a[o] = va;
                } else if constexpr (E == Epilogue::Pair) {
                    call.out_a[o] = va;
                    call.out_b[o] = vb;
                } else {
                    call.out_a[o] = silu_mul(va, vb);
                }
            }
        }
    }
}

template <Format F, Epilogue E>
void gemv_fma_dispatch(hipStream_t stream, const PackedCall &call)
{
    dim3 grid((call.n + kGemvRows * kGemvWaves - 1) / (kGemvRows * kGemvWaves));
    if (call.m <= 1)
        gemv_fma_kernel<F, 1, E><<<grid, 256, 0, stream>>>(call);
    else if (call.m <= 2)
        gemv_fma_kernel<F, 2, E><<<grid, 256, 0, stream>>>(call);
    else if (call.m <= 4)
        gemv_fma_kernel<F, 4, E><<<grid, 256, 0, stream>>>(call);
    else
        gemv_fma_kernel<F, 8, E><<<grid, 256, 0, stream>>>(call);
}

template <Format F>
void gemv_fma_epilogue(hipStream_t stream, const PackedCall &call)
{
    switch (call.epilogue) {
    case Epilogue::Single: gemv_fma_dispatch<F, Epilogue::Single>(stream, call); break;
    case Epilogue::Pair: gemv_fma_dispatch<F, Epilogue::Pair>(stream, call); break;
    case Epilogue::SwigluPair: gemv_fma_dispatch<F, Epilogue::SwigluPair>(stream, call); break;
    }
}

// ---------------------------------------------------------------------------
// Prefill GEMM: a 64x64 output tile per 256-thread block.  Each 128-weight
// group is staged as two 64-wide K slices: activations and decoded
// (unscaled) weight levels go to LDS as f32, every thread accumulates a 4x4
// micro-tile for the group, then applies the group scale.
// ---------------------------------------------------------------------------
constexpr int kTile = 64;
constexpr int kSlice = 64;

template <Format F, Epilogue E>
__global__ __launch_bounds__(256) void gemm_fma_kernel(PackedCall call)
{
    constexpr int S = (E == Epilogue::Single) ? 1 : 2;
    __shared__ float xs[kSlice][kTile + 4];
    __shared__ float ws[S][kSlice][kTile + 4];
    __shared__ float lut[16];
    if (threadIdx.x < 16)
        lut[threadIdx.x] = kNf4Levels[threadIdx.x];

    const uint32_t n = call.n, k = call.k, m = call.m;
    const uint32_t n0 = blockIdx.x * kTile, m0 = blockIdx.y * kTile;
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const size_t row_bytes = size_t(k) / weights_per_byte(F);
    const uint32_t groups = k / 128;

    float total[S][4][4];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                total[s][i][j] = 0.0f;

    for (uint32_t g = 0; g < groups; ++g) {
        float part[S][4][4];
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    part[s][i][j] = 0.0f;
        for (int half = 0; half < 2; ++half) {
            const uint32_t k0 = g * 128 + half * kSlice;
            __syncthreads();
            // Activations: 64 rows x 64 k, 16 floats per thread, stored
            // k-major so the micro-tile reads are float4 along m.
            {
                const int mm = tid >> 2;
                const int kq = (tid & 3) * 16;
                float v[16];
                if (m0 + mm < m) {
                    const float4 *xp = reinterpret_cast<const float4 *>(
                        call.x + size_t(m0 + mm) * k + k0 + kq);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        float4 t = xp[q];
                        v[4 * q] = t.x;
                        v[4 * q + 1] = t.y;
                        v[4 * q + 2] = t.z;
                        v[4 * q + 3] = t.w;
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        v[j] = 0.0f;
                }
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    xs[kq + j][mm] = v[j];
            }
            // Weights: 64 rows x 64 k decoded to unscaled levels.
            {
                const int nn = tid >> 2;
                const int kq = (tid & 3) * 16;
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const PackedStream &st = s ? call.b : call.a;
                    float w[16];
                    if (n0 + nn < n) {
                        Words words = load_chunk<F>(st.codes + size_t(n0 + nn) * row_bytes +
                                                    size_t(k0 + kq) / weights_per_byte(F));
                        decode_chunk<F>(words, w, lut);
                    } else {
#pragma unroll
                        for (int j = 0; j < 16; ++j)
                            w[j] = 0.0f;
                    }
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        ws[s][kq + j][nn] = w[j];
                }
            }
            __syncthreads();
#pragma unroll 8
            for (int kk = 0; kk < kSlice; ++kk) {
                float4 a = *reinterpret_cast<const float4 *>(&xs[kk][ty * 4]);
                float av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    float4 bw = *reinterpret_cast<const float4 *>(&ws[s][kk][tx * 4]);
                    float bv[4] = {bw.x, bw.y, bw.z, bw.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            part[s][i][j] += av[i] * bv[j];
                }
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const PackedStream &st = s ? call.b : call.a;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t col = n0 + tx * 4 + j;
                float sc = col < n ? load_scale(st, size_t(col) * groups + g) : 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    total[s][i][j] += sc * part[s][i][j];
            }
        }
    }

#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t row = m0 + ty * 4 + i;
        if (row >= m)
            continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t col = n0 + tx * 4 + j;
            if (col >= n)
                continue;
            size_t o = size_t(row) * n + col;
            if constexpr (E == Epilogue::Single) {
                call.out_a[o] = total[0][i][j];
            } else if constexpr (E == Epilogue::Pair) {
                call.out_a[o] = total[0][i][j];
                call.out_b[o] = total[S - 1][i][j];
            } else {
                call.out_a[o] = silu_mul(total[0][i][j], total[S - 1][i][j]);
            }
        }
    }
}

template <Format F>
void gemm_fma_epilogue(hipStream_t stream, const PackedCall &call)
{
    dim3 grid((call.n + kTile - 1) / kTile, (call.m + kTile - 1) / kTile);
    switch (call.epilogue) {
    case Epilogue::Single:
        gemm_fma_kernel<F, Epilogue::Single><<<grid, 256, 0, stream>>>(call);
        break;
    case Epilogue::Pair:
        gemm_fma_kernel<F, Epilogue::Pair><<<grid, 256, 0, stream>>>(call);
        break;
    case Epilogue::SwigluPair:
        gemm_fma_kernel<F, Epilogue::SwigluPair><<<grid, 256, 0, stream>>>(call);
        break;
    }
}

// ---------------------------------------------------------------------------
// Row gather (backend-cpu/src/packed.rs:11-91; device-id poisoning as the
// deferred backends do it, backend-wgpu/src/shaders/packed_gather.wgsl).
// ---------------------------------------------------------------------------
template <Format F>
__global__ __launch_bounds__(256) void gather_kernel(float *out, const uint8_t *codes,
                                                     const float *scales, const float *ids,
                                                     uint32_t count, uint32_t rows, uint32_t k)
{
    const size_t total = size_t(count) * k;
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += size_t(gridDim.x) * 256) {
        const uint32_t r = uint32_t(i / k);
        const uint32_t index = uint32_t(i - size_t(r) * k);
        const float f = ids[r];
        // Finite, non-negative, integral and < 2^24 (dense.rs:35-49); NaN
        // fails every comparison.
        const bool valid = f >= 0.0f && f < 16777216.0f && floorf(f) == f;
        const uint32_t src = valid ? uint32_t(f) : 0xFFFFFFFFu;
        if (src >= rows) {
            out[i] = __builtin_nanf("");
            continue;
        }
        const uint32_t group = index / 128, within = index % 128;
        float w;
        if constexpr (F == Format::Ternary) {
            uint32_t byte = codes[size_t(src) * (k / 4) + group * 32 + within / 4];
            w = float((byte >> (2 * (within % 4))) & 3u) - 1.0f;
        } else if constexpr (F == Format::Nf4) {
            uint32_t byte = codes[size_t(src) * (k / 2) + group * 64 + within / 2];
            w = kNf4Levels[(within & 1) ? (byte >> 4) : (byte & 15u)];
        } else {
            w = float(int8_t(codes[size_t(src) * k + index]));
        }
        out[i] = w * scales[size_t(src) * (k / 128) + group];
    }
}

__global__ __launch_bounds__(256) void fill_kernel(float *dst, size_t count, float value)
{
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < count;
         i += size_t(gridDim.x) * 256)
        dst[i] = value;
}

__global__ __launch_bounds__(256) void swiglu_kernel(float *out, const float *gate,
                                                     const float *up, size_t count)
{
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < count;
         i += size_t(gridDim.x) * 256)
        out[i] = silu_mul(gate[i], up[i]);
}

unsigned grid_for(size_t count)
{
    size_t blocks = (count + 255) / 256;
    return unsigned(blocks < 65536 ? (blocks ? blocks : 1) : 65536);
}

}  // namespace

void launch_gemv_fma(hipStream_t stream, const PackedCall &call)
{
    switch (call.format) {
    case Format::Ternary: gemv_fma_epilogue<Format::Ternary>(stream, call); break;
    case Format::Nf4: gemv_fma_epilogue<Format::Nf4>(stream, call); break;
    case Format::Int8: gemv_fma_epilogue<Format::Int8>(stream, call); break;
    }
}

void launch_gemm_fma(hipStream_t stream, const PackedCall &call)
{
    switch (call.format) {
    case Format::Ternary: gemm_fma_epilogue<Format::Ternary>(stream, call); break;
    case Format::Nf4: gemm_fma_epilogue<Format::Nf4>(stream, call); break;
    case Format::Int8: gemm_fma_epilogue<Format::Int8>(stream, call); break;
    }
}

void launch_packed_gather(hipStream_t stream, Format format, float *out, const uint8_t *codes,
                          const float *scales, const float *ids, uint32_t count, uint32_t rows,
                          uint32_t k)
{
    unsigned grid = grid_for(size_t(count) * k);
    switch (format) {
    case Format::Ternary:
        gather_kernel<Format::Ternary><<<grid, 256, 0, stream>>>(out, codes, scales, ids, count,
                                                                 rows, k);
        break;
    case Format::Nf4:
        gather_kernel<Format::Nf4><<<grid, 256, 0, stream>>>(out, codes, scales, ids, count, rows,
                                                             k);
        break;
    case Format::Int8:
        gather_kernel<Format::Int8><<<grid, 256, 0, stream>>>(out, codes, scales, ids, count,
                                                              rows, k);
        break;
    }
}

// f16_to_f32 of the loader (executor-core/src/loader.rs:408-421), in integer
// steps so that no floating-point mode (denormal flushing) can change a bit:
// a subnormal m * 2^-24 is normalised by its leading bit.
__global__ void f16_to_f32_kernel(float *out, const uint16_t *bits, size_t count)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        const uint32_t h = bits[i];
        const uint32_t sign = (h & 0x8000u) << 16;
        const uint32_t exponent = (h >> 10) & 0x1Fu;
        uint32_t mantissa = h & 0x3FFu;
        uint32_t w;
        if (exponent == 0) {
            if (mantissa == 0) {
                w = 0;
            } else {
                // value = mantissa * 2^-24 = 1.f * 2^(lead - 24)
                const int lead = 31 - __clz(mantissa);
                mantissa = (mantissa << (23 - lead)) & 0x7FFFFFu;
                w = (uint32_t(lead - 24 + 127) << 23) | mantissa;
            }
        } else if (exponent == 31) {
            w = 0x7F800000u | (mantissa << 13);
        } else {
            w = ((exponent + 112) << 23) | (mantissa << 13);
        }
        out[i] = __uint_as_float(w | sign);
    }
}

void launch_f16_to_f32(hipStream_t stream, float *out, const uint16_t *bits, size_t count)
{
    if (count)
        f16_to_f32_kernel<<<grid_for(count), 256, 0, stream>>>(out, bits, count);
}

void launch_fill_f32(hipStream_t stream, float *dst, size_t count, float value)
{
    if (count)
        fill_kernel<<<grid_for(count), 256, 0, stream>>>(dst, count, value);
}

void launch_swiglu(hipStream_t stream, float *out, const float *gate, const float *up,
                   size_t count)
{
    if (count)
        swiglu_kernel<<<grid_for(count), 256, 0, stream>>>(out, gate, up, count);
}

}  // namespace mfh
