/*
 * iris_synth.c - seeded synthetic tensors (definition of the values in iris_synth.h).
 */
#include "../../include/iris_synth.h"
#include "iris_st.h"

#include <math.h>
#include <string.h>

static inline uint64_t splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

float iris_synth_value(uint64_t seed, uint64_t index, float mean, float std) {
    uint64_t r = splitmix64(seed * 0x9E3779B97F4A7C15ULL + index);
    int32_t u = (int32_t)(r & 0xffff) + (int32_t)((r >> 16) & 0xffff) +
                (int32_t)((r >> 32) & 0xffff) + (int32_t)(r >> 48);
    float z = (float)(u - 131070) * (1.0f / 37837.2273f);
    return fmaf(z, std, mean);
}

void iris_synth_fill_f32(float *dst, size_t n, uint64_t seed, uint64_t first, float mean, float std) {
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; i++) dst[i] = iris_synth_value(seed, first + i, mean, std);
}

void iris_synth_fill_bf16(uint16_t *dst, size_t n, uint64_t seed, uint64_t first, float mean, float std) {
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; i++) dst[i] = iris_f32_to_bf16(iris_synth_value(seed, first + i, mean, std));
}

uint64_t iris_synth_seed(uint64_t model_seed, const char *name) {
    uint64_t h = 0xcbf29ce484222325ULL;
    for (const unsigned char *p = (const unsigned char *)name; *p; p++) {
        h ^= *p;
        h *= 0x100000001b3ULL;
    }
    return splitmix64(h ^ splitmix64(model_seed));
}

/* Mean and standard deviation of a random-init VAE tensor, from its name:
 * norm scales ~1, biases and batch-norm means small, batch-norm variances
 * ~1, convolution weights 1 / sqrt(fan_in) (half that for decoder.conv_out,
 * which keeps most output pixels inside [-1, 1]). */
void iris_synth_vae_stats(const char *name, int fan_in, float *mean, float *std) {
    size_t n = strlen(name);
#define ENDS(s) (n >= sizeof(s) - 1 && strcmp(name + n - (sizeof(s) - 1), s) == 0)
    if (ENDS("running_var")) { *mean = 1.0f; *std = 0.1f; }
    else if (ENDS("running_mean")) { *mean = 0.0f; *std = 0.1f; }
    else if (ENDS(".bias")) { *mean = 0.0f; *std = 0.05f; }
    else if (strstr(name, "norm") && ENDS(".weight")) { *mean = 1.0f; *std = 0.1f; }
    else {
        *mean = 0.0f;
        *std = (strcmp(name, "decoder.conv_out.weight") == 0 ? 0.5f : 1.0f) / sqrtf((float)(fan_in > 0 ? fan_in : 1));
    }
#undef ENDS
}
