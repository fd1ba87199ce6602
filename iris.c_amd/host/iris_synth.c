/*
 * iris_synth.c - seeded synthetic tensors (definition of the values in iris_synth.h).
 */
#include "../../include/iris_synth.h"
#include "iris_st.h"

#include <math.h>

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
