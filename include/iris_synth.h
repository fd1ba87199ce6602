/*
 * iris_synth.h - seeded synthetic tensors for random-init models and inputs.
 *
 * No counterpart in the reference: the reference loads trained weights. The
 * benchmark and the parity tests need random-init weights of the real
 * architectures, identical on every machine, so values are a pure function of
 * (seed, element index):
 *   r  = splitmix64(seed * 0x9E3779B97F4A7C15 + index)
 *   u  = sum of the four 16-bit fields of r         (Irwin-Hall, n = 4)
 *   z  = (u - 131070) * (1 / 37837.2273)           (mean 0, variance 1)
 *   f32 value = fmaf(z, std, mean); bf16 value = RNE(f32 value)
 * Every step is integer arithmetic or one correctly rounded IEEE operation, so
 * any conforming C compiler produces the same bits.
 */
#ifndef IRIS_SYNTH_H
#define IRIS_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float iris_synth_value(uint64_t seed, uint64_t index, float mean, float std);
/* Fills dst[0..n) with values for indices [first, first+n). Multithreaded. */
void iris_synth_fill_f32(float *dst, size_t n, uint64_t seed, uint64_t first, float mean, float std);
void iris_synth_fill_bf16(uint16_t *dst, size_t n, uint64_t seed, uint64_t first, float mean, float std);
/* Stable per-tensor seed: FNV-1a of the tensor name mixed with a model seed. */
uint64_t iris_synth_seed(uint64_t model_seed, const char *name);
/* Mean and std of a random-init VAE tensor by name (norm scales ~1, biases
 * small, conv weights 1 / sqrt(fan_in)). */
void iris_synth_vae_stats(const char *name, int fan_in, float *mean, float *std);

#ifdef __cplusplus
}
#endif
#endif
