// Streaming-read ceiling: the rate a plain read of N bytes reaches on this
// device when each launch misses the Infinity Cache, measured the way the
// decode GEMV heads are (back-to-back launches rotating over copies that
// total at least 1 GiB, HIP events around the timed launches).  It is the
// control the heads' roofline fractions are read against: no packed kernel
// can stream its bytes faster than a kernel that only reads them.
//
// Not part of the InferenceOps boundary: a measurement tool in a library of
// its own (libminifield_probe.so), with no counterpart in the reference.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <vector>

namespace {

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// Each wave reads LOADS consecutive KB (one 16-byte non-temporal load per
// lane per KB, all issued before any is consumed) and folds them so the
// loads cannot be dropped; the result is stored only if it matches a value
// the fill never produces.
template <int LOADS>
__global__ __launch_bounds__(1024) void read_kernel(const v4u *__restrict__ src, size_t chunks,
                                                    unsigned *sink)
{
    const size_t lane = threadIdx.x & 63;
    const size_t wave = (size_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    v4u v[LOADS];
#pragma unroll
    for (int l = 0; l < LOADS; ++l) {
        size_t c = wave * LOADS + l;
        c = c < chunks ? c : chunks - 1;
        v[l] = __builtin_nontemporal_load(&src[c * 64 + lane]);
    }
    v4u acc = {0, 0, 0, 0};
#pragma unroll
    for (int l = 0; l < LOADS; ++l)
        acc ^= v[l];
    const unsigned r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (r == 0x12345678u)
        sink[0] = r;
}

template <int LOADS>
void launch(const v4u *src, size_t chunks, int waves_per_block, unsigned *sink, hipStream_t s)
{
    const size_t waves = (chunks + LOADS - 1) / LOADS;
    const unsigned blocks = unsigned((waves + waves_per_block - 1) / waves_per_block);
    read_kernel<LOADS><<<blocks, 64 * waves_per_block, 0, s>>>(src, chunks, sink);
}

void launch_any(int kb_per_wave, const v4u *src, size_t chunks, int wpb, unsigned *sink,
                hipStream_t s)
{
    switch (kb_per_wave) {
    case 1: launch<1>(src, chunks, wpb, sink, s); break;
    case 2: launch<2>(src, chunks, wpb, sink, s); break;
    case 4: launch<4>(src, chunks, wpb, sink, s); break;
    case 8: launch<8>(src, chunks, wpb, sink, s); break;
    default: launch<16>(src, chunks, wpb, sink, s); break;
    }
}

// One wave reads the core-clock cycle counter (s_memtime) and the
// constant-rate counter (s_memrealtime) around `spins` further cycle-counter
// reads: the shader clock the device is running at when it executes.
__global__ void clock_kernel(unsigned long long *out, int spins)
{
    const unsigned long long c0 = __builtin_readcyclecounter();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    unsigned long long c = c0;
    for (int i = 0; i < spins; ++i)
        c = __builtin_readcyclecounter();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        out[0] = c - c0;
        out[1] = r1 - r0;
    }
}

}  // namespace

extern "C" {

// The shader clock (MHz) of the current device, measured by one wave queued
// on `stream` (a hipStream_t, so it runs right after the work queued before
// it); waits for the stream.  Returns 0, or -1 on a HIP error.
int mfp_shader_clock(void *stream, double *mhz)
{
    static unsigned long long *counters = nullptr;
    static int wall_khz = 0;
    if (!counters && (hipMalloc(&counters, 16) != hipSuccess ||
                      hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, 0) !=
                          hipSuccess || wall_khz <= 0))
        return -1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    clock_kernel<<<1, 64, 0, s>>>(counters, 20000);
    unsigned long long host[2] = {0, 0};
    if (hipGetLastError() != hipSuccess ||
        hipMemcpyAsync(host, counters, 16, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess || host[1] == 0)
        return -1;
    *mhz = double(host[0]) * (wall_khz / 1e3) / double(host[1]);
    return 0;
}

// Average microseconds per launch of a plain read of `bytes` (a multiple of
// 1024) over `launches` back-to-back launches rotating over copies totalling
// at least 1 GiB, for each (KB per wave, waves per block) pair given:
// kb_per_wave in {1, 2, 4, 8, 16}, waves_per_block in {4, 8, 16}.  Returns 0,
// or -1 on a HIP error or invalid argument (the device memory is freed).
int mfp_read_ceiling(size_t bytes, const int *kb_per_wave, const int *waves_per_block,
                     int configs, int launches, double *us_out)
{
    if (bytes < 1024 || bytes % 1024 || configs <= 0 || launches <= 0)
        return -1;
    for (int c = 0; c < configs; ++c)
        if (waves_per_block[c] != 4 && waves_per_block[c] != 8 && waves_per_block[c] != 16)
            return -1;
    const size_t copies = std::max<size_t>(1, ((size_t(1) << 30) + bytes - 1) / bytes);
    std::vector<v4u *> bufs(copies, nullptr);
    unsigned *sink = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int status = -1;
    bool ok = hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess &&
              hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess &&
              hipMalloc(&sink, 64) == hipSuccess;
    for (size_t i = 0; ok && i < copies; ++i)
        ok = hipMalloc(&bufs[i], bytes) == hipSuccess &&
             hipMemsetAsync(bufs[i], 0x5A, bytes, s) == hipSuccess;
    const size_t chunks = bytes / 1024;
    for (int c = 0; ok && c < configs; ++c) {
        for (size_t i = 0; i < copies; ++i)
            launch_any(kb_per_wave[c], bufs[i], chunks, waves_per_block[c], sink, s);
        ok = hipEventRecord(e0, s) == hipSuccess;
        for (int r = 0; ok && r < launches; ++r)
            launch_any(kb_per_wave[c], bufs[r % copies], chunks, waves_per_block[c], sink, s);
        float ms = 0.0f;
        ok = ok && hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
             hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
        us_out[c] = double(ms) * 1e3 / launches;
    }
    if (ok && hipStreamSynchronize(s) == hipSuccess && hipGetLastError() == hipSuccess)
        status = 0;
    for (v4u *b : bufs)
        if (b)
            (void)hipFree(b);
    if (sink)
        (void)hipFree(sink);
    if (e0)
        (void)hipEventDestroy(e0);
    if (e1)
        (void)hipEventDestroy(e1);
    if (s)
        (void)hipStreamDestroy(s);
    return status;
}

}  // extern "C"
