/*
 * le_quant.h -- host-side (CPU) helpers that produce GGUF blocks and seeded test inputs.
 *
 * The reference has no quantizer (it only dequantizes GGUF files, src/quant.rs:1-2), so these are
 * this project's own, written from the block layouts. They produce the weights of the parity
 * tests and the benchmark; they are not on the device path.
 */
#ifndef LE_QUANT_H
#define LE_QUANT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element k of the sequence is a standard normal deviate built from splitmix64 outputs:
 * state_k = seed + k * 0x9E3779B97F4A7C15, u_k = mix(state_k); pair j = (2j, 2j+1) takes
 * u1 = ((u_2j >> 11) + 1) * 2^-53, u2 = (u_2j+1 >> 11) * 2^-53 and Box-Muller in double:
 * r = sqrt(-2 ln u1), value 2j = r cos(2 pi u2), value 2j+1 = r sin(2 pi u2).
 * dst[i] = (float)(mean + std * z_{offset + i}). Threaded; deterministic for any thread count. */
void le_fill_normal(float *dst, size_t n, uint64_t seed, uint64_t offset, double mean, double std, int nthreads);

/* Quantize rows x cols fp32 values (row-major) into GGUF blocks of type ty; dst holds
 * rows * row_bytes(ty, cols) bytes. Returns 0 or a negative le_status code. */
int le_quantize_rows(int ty, const float *src, void *dst, size_t rows, size_t cols, int nthreads);

/* IEEE round-to-nearest-even float -> half conversion used by the quantizers. */
uint16_t le_f32_to_f16(float f);

#ifdef __cplusplus
}
#endif
#endif
