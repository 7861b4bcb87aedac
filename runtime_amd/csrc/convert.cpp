// Host-side converters: seeded synthetic inputs and the group-128 quantizer.
//
// mfc_quantize restates tools/converters/src/minifield_converters/
// quantization.py:115-160 operation by operation:
//   scale  = f16(absmax)            (ternary, nf4)  - f32 max, RNE to binary16
//   scale  = f16(absmax / 127f)     (int8)          - f32 divide first
//   safe   = scale > 0 ? scale : 1, widened to f64
//   n      = f32(f64(w) / safe)                      - f64 divide, RNE to f32
//   ternary/int8: r = sign(n) * floor(|n| + 0.5f)   - all in f32
//   ternary: q = clip(r + 1, 0, 2), zero-scale groups -> 1
//   int8:    q = u8(i8(clip(r, -127, 127))), zero-scale groups -> 0
//   nf4:     q = first argmin_l |n - NF4[l]| (f32 distances, strict <),
//            zero-scale groups -> 7
// then pack_codes (:52-71): first weight in the least-significant bits.
#include "../../include/minifield_convert.h"

#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#pragma clang fp contract(off)

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

// NF4 codebook as f32, quantization.py:22-42 (identical bits to
// crates/kernels-simd/src/lib.rs:113-130).
constexpr float kNf4[16] = {
    -1.0f,        -0.6961928009986877f,  -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f,  0.7229568362236023f,  1.0f,
};

inline uint64_t mix(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint32_t f32_bits(float v)
{
    uint32_t b;
    std::memcpy(&b, &v, 4);
    return b;
}

template <typename F>
void parallel_rows(size_t rows, unsigned threads, F &&body)
{
    if (threads <= 1 || rows < 2 * threads) {
        body(size_t(0), rows);
        return;
    }
    std::vector<std::thread> pool;
    size_t chunk = (rows + threads - 1) / threads;
    for (unsigned t = 0; t < threads; ++t) {
        size_t begin = t * chunk, end = std::min(rows, begin + chunk);
        if (begin >= end)
            break;
        pool.emplace_back([&body, begin, end] { body(begin, end); });
    }
    for (auto &th : pool)
        th.join();
}

int bits_of(mfc_format format)
{
    return format == MFC_TERNARY ? 2 : format == MFC_NF4 ? 4 : 8;
}

}  // namespace

extern "C" float mfc_f16_to_f32(uint16_t bits)
{
    uint32_t sign = uint32_t(bits & 0x8000u) << 16;
    uint32_t exponent = (bits >> 10) & 0x1Fu;
    uint32_t mantissa = bits & 0x3FFu;
    uint32_t out;
    if (exponent == 0) {
        float value = float(mantissa) * 5.9604644775390625e-08f;  // exact: m * 2^-24
        out = f32_bits(value);
    } else if (exponent == 31) {
        out = 0x7F800000u | (mantissa << 13);
    } else {
        out = ((exponent + 112u) << 23) | (mantissa << 13);
    }
    out |= sign;
    float value;
    std::memcpy(&value, &out, 4);
    return value;
}

extern "C" uint16_t mfc_f32_to_f16(float value)
{
    uint32_t x = f32_bits(value);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u)  // inf / nan
        return uint16_t(sign | (absx > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (absx >= 0x477FF000u)  // >= 65520 rounds to infinity
        return uint16_t(sign | 0x7C00u);
    if (absx < 0x38800000u) {  // below 2^-14: binary16 subnormal or zero
        uint32_t e = absx >> 23;
        if (e < 102)
            return uint16_t(sign);
        uint32_t m = (absx & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126 - e;  // units of 2^-24
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u)))
            ++q;
        return uint16_t(sign | q);
    }
    uint32_t h = (absx - 0x38000000u) >> 13;  // rebias 127 -> 15, drop 13 bits
    uint32_t rem = absx & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
        ++h;  // a carry into the exponent is the correct rounding
    return uint16_t(sign | h);
}

extern "C" void mfc_f16_to_f32_array(const uint16_t *in, float *out, size_t count)
{
    for (size_t i = 0; i < count; ++i)
        out[i] = mfc_f16_to_f32(in[i]);
}

extern "C" int mfc_quantize(const float *weights, size_t rows, size_t k, mfc_format format,
                            uint8_t *codes, uint16_t *scales_f16, unsigned threads)
{
    if (rows == 0 || k == 0 || k % 128 != 0)
        return 1;
    if (format != MFC_TERNARY && format != MFC_NF4 && format != MFC_INT8)
        return 1;
    for (size_t i = 0; i < rows * k; ++i)
        if (!std::isfinite(weights[i]))
            return 1;
    const size_t groups = k / 128;
    const int bits = bits_of(format);
    const size_t per_byte = 8 / bits;
    const size_t code_width = k / per_byte;
    // Scales first, so an overflowing group rejects the whole matrix before
    // any code is written (the reference raises before packing).
    for (size_t g = 0; g < rows * groups; ++g) {
        const float *w = weights + g * 128;
        float maximum = 0.0f;
        for (int j = 0; j < 128; ++j) {
            float a = std::fabs(w[j]);
            if (a > maximum)
                maximum = a;
        }
        float scaled = format == MFC_INT8 ? maximum / 127.0f : maximum;
        uint16_t s = mfc_f32_to_f16(scaled);
        if ((s & 0x7C00u) == 0x7C00u)
            return 1;
        scales_f16[g] = s;
    }
    parallel_rows(rows, threads, [&](size_t begin, size_t end) {
        uint8_t q[128];
        for (size_t r = begin; r < end; ++r) {
            uint8_t *row_codes = codes + r * code_width;
            std::memset(row_codes, 0, code_width);
            for (size_t g = 0; g < groups; ++g) {
                const float *w = weights + r * k + g * 128;
                uint16_t s16 = scales_f16[r * groups + g];
                float scale = mfc_f16_to_f32(s16);
                bool zero = !(scale > 0.0f);
                double safe = zero ? 1.0 : double(scale);
                for (int j = 0; j < 128; ++j) {
                    float n = float(double(w[j]) / safe);
                    if (format == MFC_NF4) {
                        float best = INFINITY;
                        uint8_t code = 0;
                        for (int l = 0; l < 16; ++l) {
                            float d = std::fabs(n - kNf4[l]);
                            if (d < best) {
                                best = d;
                                code = uint8_t(l);
                            }
                        }
                        q[j] = zero ? 7 : code;
                    } else {
                        float sign = n > 0.0f ? 1.0f : (n < 0.0f ? -1.0f : 0.0f);
                        float rounded = sign * std::floor(std::fabs(n) + 0.5f);
                        if (format == MFC_TERNARY) {
                            float c = rounded + 1.0f;
                            c = c < 0.0f ? 0.0f : (c > 2.0f ? 2.0f : c);
                            q[j] = zero ? 1 : uint8_t(c);
                        } else {
                            float c = rounded < -127.0f ? -127.0f
                                      : (rounded > 127.0f ? 127.0f : rounded);
                            q[j] = zero ? 0 : uint8_t(int8_t(c));
                        }
                    }
                }
                // pack_codes: weight index i of the row lands in byte i/per_byte
                // at bit offset (i % per_byte) * bits.
                for (int j = 0; j < 128; ++j) {
                    size_t i = g * 128 + size_t(j);
                    row_codes[i / per_byte] |= uint8_t(q[j] << ((i % per_byte) * bits));
                }
            }
        }
    });
    return 0;
}

extern "C" int mfc_dequantize(const uint8_t *codes, const uint16_t *scales_f16, size_t rows,
                              size_t k, mfc_format format, float *out)
{
    if (rows == 0 || k == 0 || k % 128 != 0)
        return 1;
    const int bits = bits_of(format);
    const size_t per_byte = 8 / bits;
    const size_t code_width = k / per_byte;
    const unsigned mask = (1u << bits) - 1u;
    for (size_t r = 0; r < rows; ++r)
        for (size_t i = 0; i < k; ++i) {
            unsigned q = (codes[r * code_width + i / per_byte] >> ((i % per_byte) * bits)) & mask;
            float level;
            if (format == MFC_TERNARY) {
                if (q == 3)
                    return 1;
                level = float(q) - 1.0f;
            } else if (format == MFC_INT8) {
                if (q == 0x80)
                    return 1;
                level = float(int8_t(uint8_t(q)));
            } else {
                level = kNf4[q];
            }
            out[r * k + i] = level * mfc_f16_to_f32(scales_f16[r * (k / 128) + i / 128]);
        }
    return 0;
}

extern "C" void mfc_fill_normal(float *out, size_t count, uint64_t seed, double mean,
                                double sigma, unsigned threads)
{
    const size_t pairs = (count + 1) / 2;
    parallel_rows(pairs, threads, [&](size_t begin, size_t end) {
        const double two_pi = 6.283185307179586476925286766559;
        for (size_t p = begin; p < end; ++p) {
            uint64_t a = mix(seed + (2 * p + 1) * kGolden);
            uint64_t b = mix(seed + (2 * p + 2) * kGolden);
            double u1 = double((a >> 11) + 1) * 0x1.0p-53;
            double u2 = double(b >> 11) * 0x1.0p-53;
            double r = std::sqrt(-2.0 * std::log(u1));
            double theta = two_pi * u2;
            out[2 * p] = float(mean + sigma * (r * std::cos(theta)));
            if (2 * p + 1 < count)
                out[2 * p + 1] = float(mean + sigma * (r * std::sin(theta)));
        }
    });
}

extern "C" void mfc_fill_token_ids(uint32_t *out, size_t count, uint64_t seed, uint32_t vocab)
{
    for (size_t i = 0; i < count; ++i) {
        uint64_t z = mix(seed + (i + 1) * kGolden) >> 32;
        out[i] = uint32_t((z * uint64_t(vocab)) >> 32);
    }
}
