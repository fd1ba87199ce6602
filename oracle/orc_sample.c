/*
 * orc_sample.c - schedules and seeded noise of the reference sampler
 * (iris_sample.c, iris_kernels.c RNG). TEST INFRASTRUCTURE ONLY.
 */
#include "orc_internal.h"

#include <math.h>
#include <stdlib.h>

/* compute_empirical_mu, iris_sample.c:144-158 */
static float empirical_mu(int seq, int n) {
    const float a1 = 8.73809524e-05f, b1 = 1.89833333f;
    const float a2 = 0.00016927f, b2 = 0.45666666f;
    if (seq > 4300) return a2 * seq + b2;
    float m200 = a2 * seq + b2, m10 = a1 * seq + b1;
    float a = (m200 - m10) / 190.0f;
    float b = m200 - 200.0f * a;
    return a * n + b;
}

/* iris_official_schedule + generalized_time_snr_shift, iris_sample.c:160-182 */
float *orc_official_schedule(int n, int seq) {
    float *s = (float *)malloc((size_t)(n + 1) * sizeof(float));
    float mu = empirical_mu(seq, n);
    for (int i = 0; i <= n; i++) {
        float t = 1.0f - (float)i / (float)n;
        if (t <= 0.0f) s[i] = 0.0f;
        else if (t >= 1.0f) s[i] = 1.0f;
        else s[i] = expf(mu) / (expf(mu) + powf(1.0f / t - 1.0f, 1.0f));
    }
    return s;
}

/* iris_zimage_schedule, iris_sample.c:216-244 (shift passed explicitly) */
float *orc_zimage_schedule(int n, float shift) {
    float *s = (float *)malloc((size_t)(n + 1) * sizeof(float));
    const float smax = 1.0f, tmin = 1.0f / 1000.0f;
    const float smin = shift * tmin / (1.0f + (shift - 1.0f) * tmin);
    for (int i = 0; i < n; i++) {
        float u = (n > 1) ? (float)i / (float)(n - 1) : 0.0f;
        float raw = smax + (smin - smax) * u;
        s[i] = shift * raw / (1.0f + (shift - 1.0f) * raw);
    }
    s[n] = 0.0f;
    return s;
}

/* xoshiro256** seeded by SplitMix64 + Box-Muller, iris_kernels.c:50-107 */
static uint64_t rs[4];
static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
static uint64_t xoshiro(void) {
    uint64_t r = rotl(rs[1] * 5, 7) * 9, t = rs[1] << 17;
    rs[2] ^= rs[0]; rs[3] ^= rs[1]; rs[1] ^= rs[2]; rs[0] ^= rs[3];
    rs[2] ^= t; rs[3] = rotl(rs[3], 45);
    return r;
}
static void seed_rng(uint64_t seed) {
    for (int i = 0; i < 4; i++) {
        seed += 0x9e3779b97f4a7c15ULL;
        uint64_t z = seed;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
        rs[i] = z ^ (z >> 31);
    }
}
static float uni(void) { return (float)((xoshiro() >> 11) * (1.0 / 9007199254740992.0)); }
static float normal(void) {
    float u1 = uni(), u2 = uni();
    while (u1 == 0.0f) u1 = uni();
    return sqrtf(-2.0f * logf(u1)) * cosf(2.0f * 3.14159265358979323846f * u2);
}

/* iris_init_noise, iris_sample.c:1146-1188 (112x112 field, nearest subsample) */
float *orc_init_noise(int batch, int ch, int h, int w, int64_t seed) {
    size_t n = (size_t)batch * ch * h * w;
    float *out = (float *)malloc(n * sizeof(float));
    if (seed >= 0) seed_rng((uint64_t)seed);
    const int M = 112;
    if (h >= M && w >= M) {
        for (size_t i = 0; i < n; i++) out[i] = normal();
        return out;
    }
    size_t mn = (size_t)batch * ch * M * M;
    float *mx = (float *)malloc(mn * sizeof(float));
    for (size_t i = 0; i < mn; i++) mx[i] = normal();
    for (int b = 0; b < batch; b++)
        for (int c = 0; c < ch; c++)
            for (int y = 0; y < h; y++)
                for (int x = 0; x < w; x++) {
                    int sy = y * M / h, sx = x * M / w;
                    out[(((size_t)b * ch + c) * h + y) * w + x] = mx[(((size_t)b * ch + c) * M + sy) * M + sx];
                }
    free(mx);
    return out;
}
