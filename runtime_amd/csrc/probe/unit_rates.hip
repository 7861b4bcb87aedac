// Unit rates of the device the decode GEMV kernels lean on besides HBM: LDS
// reads at the NF4 level table's access pattern (and at other widths), the
// same reads mixed with f16 MFMAs as the NF4 kstep issues them, and the
// f16 / int8 MFMA rates.  They bound what the table lookups and matrix
// products of a head can cost next to its streaming read.
//
// Not part of the InferenceOps boundary: a measurement tool in the probe
// library (libminifield_probe.so), with no counterpart in the reference.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kLdsWords = 16384;  // 64 KB table
constexpr int kLdsIters = 4096;   // reads per lane
constexpr int kMfmaIters = 2048;  // per accumulator

// MODE 0: ds_read_b64 at code * 256 + 8 * (lane % 32), the NF4 table's
// conflict-free pattern (32 copies of each 8-byte entry); 1: ds_read_b32 at
// code * 256 + 4 * (lane % 32); 2: ds_read_b128 at code * 256 + 16 * lane
// % 256; 3: MODE 0 with one f16 MFMA per two reads, its B operand the two
// entries (the NF4 kstep: 4 reads, 2 MFMAs).  Each lane keeps eight fixed
// codes (0..127) and adds a loop-varying base in {0, 8192, 16384, 24576}:
// every access lies below 32512 + 24576 + 256 bytes, inside the table.
// Eight reads are in flight before an empty asm consumes them, so nothing
// but the reads (and MODE 3's MFMAs) is timed.
template <int MODE>
__global__ __launch_bounds__(1024) void lds_rate_kernel(unsigned *sink, unsigned seed)
{
    __shared__ unsigned table[kLdsWords];
    for (unsigned i = threadIdx.x; i < kLdsWords; i += blockDim.x)
        table[i] = i * 2654435761u;
    __syncthreads();
    const unsigned lane = threadIdx.x & 63;
    unsigned addr[8];
    unsigned h = seed * 977u + threadIdx.x * 131u;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        h = h * 1664525u + 1013904223u;
        const unsigned code = (h >> 16) & 127;
        addr[u] = MODE == 2 ? code * 256 + 16 * lane % 256
                  : MODE == 1 ? code * 256 + 4 * (lane % 32)
                              : code * 256 + 8 * (lane % 32);
    }
    v8h a;
    for (int i = 0; i < 8; ++i)
        a[i] = _Float16(1.0f + threadIdx.x * 0.001f + i);
    v4f c{};
    const char *cells = reinterpret_cast<const char *>(table);
    for (int it = 0; it < kLdsIters / 8; ++it) {
        const unsigned base =
            __builtin_amdgcn_readfirstlane((unsigned(it) * 2654435761u) >> 7) & 24576u;
        if constexpr (MODE == 0) {
            uint2 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = *reinterpret_cast<const uint2 *>(cells + addr[u] + base);
            asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]),
                         "v"(v[6]), "v"(v[7]));
        } else if constexpr (MODE == 1) {
            unsigned v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = *reinterpret_cast<const unsigned *>(cells + addr[u] + base);
            asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]),
                         "v"(v[6]), "v"(v[7]));
        } else if constexpr (MODE == 2) {
            v4u v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = *reinterpret_cast<const v4u *>(cells + addr[u] + base);
            asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]),
                         "v"(v[6]), "v"(v[7]));
        } else {
            uint2 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = *reinterpret_cast<const uint2 *>(cells + addr[u] + base);
#pragma unroll
            for (int u = 0; u < 8; u += 2) {
                const v4u bw = v4u{v[u].x, v[u].y, v[u + 1].x, v[u + 1].y};
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(v8h, bw), c, 0, 0,
                                                           0);
            }
        }
    }
    // Stored only for a value the fill never produces, so nothing is dropped.
    if (c.x == -1.0f)
        sink[blockIdx.x] = 1;
}

// Four independent accumulators per wave, 256-lane blocks.
__global__ __launch_bounds__(256) void mfma_f16_kernel(float *sink, float seed)
{
    v8h a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = _Float16(seed + threadIdx.x * 0.001f + i);
        b[i] = _Float16(seed - i * 0.01f);
    }
    v4f c0{}, c1{}, c2{}, c3{};
    for (int it = 0; it < kMfmaIters; ++it) {
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c3, 0, 0, 0);
    }
    const v4f s = c0 + c1 + c2 + c3;
    if (s.x == -1.0f)
        sink[blockIdx.x] = s.y;
}

__global__ __launch_bounds__(256) void mfma_i8_kernel(int *sink, int seed)
{
    v4i a{seed, seed + 1, int(threadIdx.x), 3}, b{1, 2, 3, seed};
    v4i c0{}, c1{}, c2{}, c3{};
    for (int it = 0; it < kMfmaIters; ++it) {
        c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c3, 0, 0, 0);
    }
    const v4i s = c0 + c1 + c2 + c3;
    if (s.x == -1)
        sink[blockIdx.x] = s.y;
}

// Milliseconds per launch of `launch` over 10 launches after one untimed.
template <typename L>
float time_ms(L launch, hipStream_t s, hipEvent_t e0, hipEvent_t e1, bool &ok)
{
    launch();
    ok = ok && hipEventRecord(e0, s) == hipSuccess;
    for (int r = 0; r < 10; ++r)
        launch();
    float ms = 0.0f;
    ok = ok && hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
         hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
    return ms / 10;
}

}  // namespace

extern "C" {

// out[0..3]: LDS read rate in bytes per ns per CU of MODE 0..3 of
// lds_rate_kernel (two 64 KB blocks of 16 waves per CU); out[4], out[5]:
// ns per f16 16x16x32 / int8 16x16x64 MFMA per SIMD (8 waves per SIMD, four
// independent accumulators each).  Returns 0, or -1 on a HIP error.
int mfp_unit_rates(double *out)
{
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
        return -1;
    const unsigned lds_blocks = unsigned(cus) * 2, mfma_blocks = unsigned(cus) * 8;
    void *sink = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    bool ok = hipMalloc(&sink, size_t(mfma_blocks) * sizeof(float)) == hipSuccess &&
              hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess &&
              hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess;
    unsigned *usink = static_cast<unsigned *>(sink);
    const double lds_lanes = double(lds_blocks) * 1024 * kLdsIters;
    if (ok) {
        const float ms0 = time_ms([&] { lds_rate_kernel<0><<<lds_blocks, 1024, 0, s>>>(usink, 1); },
                                  s, e0, e1, ok);
        const float ms1 = time_ms([&] { lds_rate_kernel<1><<<lds_blocks, 1024, 0, s>>>(usink, 1); },
                                  s, e0, e1, ok);
        const float ms2 = time_ms([&] { lds_rate_kernel<2><<<lds_blocks, 1024, 0, s>>>(usink, 1); },
                                  s, e0, e1, ok);
        const float ms3 = time_ms([&] { lds_rate_kernel<3><<<lds_blocks, 1024, 0, s>>>(usink, 1); },
                                  s, e0, e1, ok);
        const float msf = time_ms(
            [&] { mfma_f16_kernel<<<mfma_blocks, 256, 0, s>>>(static_cast<float *>(sink), 1.0f); },
            s, e0, e1, ok);
        const float msi = time_ms(
            [&] { mfma_i8_kernel<<<mfma_blocks, 256, 0, s>>>(static_cast<int *>(sink), 1); }, s,
            e0, e1, ok);
        // bytes / (ms * 1e6 ns) / CUs
        out[0] = lds_lanes * 8 / (double(ms0) * 1e6) / cus;
        out[1] = lds_lanes * 4 / (double(ms1) * 1e6) / cus;
        out[2] = lds_lanes * 16 / (double(ms2) * 1e6) / cus;
        out[3] = lds_lanes * 8 / (double(ms3) * 1e6) / cus;
        // MFMAs per SIMD: blocks * 4 waves * 4 accumulators * iterations / (CUs * 4)
        const double per_simd = double(mfma_blocks) * 4 * 4 * kMfmaIters / (double(cus) * 4);
        out[4] = double(msf) * 1e6 / per_simd;
        out[5] = double(msi) * 1e6 / per_simd;
    }
    ok = ok && hipStreamSynchronize(s) == hipSuccess && hipGetLastError() == hipSuccess;
    if (sink)
        (void)hipFree(sink);
    if (e0)
        (void)hipEventDestroy(e0);
    if (e1)
        (void)hipEventDestroy(e1);
    if (s)
        (void)hipStreamDestroy(s);
    return ok ? 0 : -1;
}

}  // extern "C"
