/*
 * minifield_convert.h - host-side converters shipped with the backend:
 * the offline group-128 quantizer and the seeded synthetic-input generator
 * used to build benchmark workloads.
 *
 * mfc_quantize restates tools/converters/src/minifield_converters/
 * quantization.py:115-160 (`quantize`) and :52-71 (`pack_codes`) bit for
 * bit; mfc_dequantize restates :96-112 (`dequantize`).  No GPU is involved.
 */
#ifndef MINIFIELD_CONVERT_H
#define MINIFIELD_CONVERT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Packed stream formats, crates/kernels-simd/src/lib.rs:87-96. */
typedef enum mfc_format {
    MFC_TERNARY = 0, /* minifield.ternary.v1: 2-bit codes, w = (q - 1) * s */
    MFC_NF4 = 1,     /* minifield.nf4.v1: 4-bit codes, w = NF4[q] * s      */
    MFC_INT8 = 2     /* minifield.int8.v1: signed bytes, w = i8(q) * s      */
} mfc_format;

/* Quantize dense f32 weights [rows, k] (k % 128 == 0) into packed codes
 * [rows, k * bits / 8] and IEEE binary16 scales [rows, k / 128].
 * Returns 0, or 1 (ConversionError) for non-finite weights, k % 128 != 0,
 * empty shapes or an absmax that overflows binary16.  `threads` <= 1 runs
 * single-threaded; the output does not depend on it. */
int mfc_quantize(const float *weights, size_t rows, size_t k, mfc_format format,
                 uint8_t *codes, uint16_t *scales_f16, unsigned threads);

/* Decode packed codes + binary16 scales to f32 [rows, k]
 * (quantization.py:96-112).  Returns 1 for reserved codes. */
int mfc_dequantize(const uint8_t *codes, const uint16_t *scales_f16, size_t rows, size_t k,
                   mfc_format format, float *out);

/* binary16 -> binary32 (exact) and binary32 -> binary16 (round to nearest
 * even, overflow to infinity), the conversions numpy applies. */
float mfc_f16_to_f32(uint16_t bits);
uint16_t mfc_f32_to_f16(float value);
/* Convert a binary16 array to f32 (the loader's scale decode,
 * crates/executor-core/src/loader.rs:408-421). */
void mfc_f16_to_f32_array(const uint16_t *in, float *out, size_t count);

/* Seeded N(mean, sigma) f32 samples: counter-based splitmix64, Box-Muller in
 * f64, cast to f32.  Element 2p and 2p+1 come from counters 2p+1 and 2p+2:
 *   u1 = ((mix(seed + (2p+1)*G) >> 11) + 1) * 2^-53,
 *   u2 = (mix(seed + (2p+2)*G) >> 11) * 2^-53,
 *   r = sqrt(-2 ln u1), out[2p] = mean + sigma*r*cos(2 pi u2),
 *   out[2p+1] = mean + sigma*r*sin(2 pi u2),
 * where G = 0x9E3779B97F4A7C15 and mix is the splitmix64 finaliser. */
void mfc_fill_normal(float *out, size_t count, uint64_t seed, double mean, double sigma,
                     unsigned threads);
/* Seeded uniform token ids in [0, vocab): id_i = ((mix(seed + (i+1)*G) >> 32)
 * * vocab) >> 32. */
void mfc_fill_token_ids(uint32_t *out, size_t count, uint64_t seed, uint32_t vocab);

#ifdef __cplusplus
}
#endif

#endif /* MINIFIELD_CONVERT_H */
