/*
 * iris_schedule.c - timestep schedules with the reference build's bits.
 *
 * The reference compiles iris_sample.c:61-244 with -O3 -march=native
 * -ffast-math (its Makefile:5). gcc then vectorizes every schedule loop and
 * rewrites its arithmetic:
 *   - a loop over `count` elements runs 8-wide blocks while count >= 8, one
 *     4-wide block when at least 4 elements remain, and scalar code for the
 *     rest; the vector lanes and the scalar tail do not compute alike;
 *   - in the vector lanes a division a / b becomes a * rcp_nr(b), where
 *     rcp_nr(b) = (r + r) - r * (r * b) refines the hardware reciprocal
 *     estimate r = rcpps(b) by one Newton step; the scalar tail divides;
 *   - expf / powf of the vector lanes are glibc libmvec's 8-wide AVX2
 *     (_ZGVdN8v_expf, _ZGVdN8vv_powf) and 4-wide SSE (_ZGVbN4v_expf,
 *     _ZGVbN4vv_powf) entry points, the scalar tail calls libm;
 *   - i / n becomes i * (1 / n), a - b * c and a + b * c become fused
 *     multiply-adds, and sums are reassociated.
 * This file performs those same operations in the same order, with the same
 * instructions (AVX2 + FMA intrinsics, the libmvec entry points), so on a
 * given host every schedule equals the reference build's on that host bit for
 * bit. The last bit of rcpps is specific to the CPU model, and so is the
 * reference build's schedule; the lane classes follow the element count, not
 * the CPU. The file is compiled with -ffp-contract=off so that only the fused
 * operations written here are fused.
 *
 * The vector lanes need AVX2 and FMA, as the reference's -march=native build
 * does on the hosts whose bits it reproduces. On a CPU without them every
 * element takes the scalar formula (the build's scalar tail), checked once
 * per process with __builtin_cpu_supports; the values then equal the
 * reference formulas evaluated in plain IEEE float (the reference build's
 * scalar tail), not its vector lanes.
 */
#include "../../include/iris_sample.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>

__m256 _ZGVdN8v_expf(__m256);
__m128 _ZGVbN4v_expf(__m128);
__m256 _ZGVdN8vv_powf(__m256, __m256);
__m128 _ZGVbN4vv_powf(__m128, __m128);

#define VEC __attribute__((target("avx2,fma")))

/* the vector lanes run only where the CPU has AVX2 and FMA
 * (IRIS_SCHEDULE_SCALAR=1 in the environment takes the scalar formulas
 * everywhere, as on a CPU without them) */
static int vec_ok(void) {
    static int ok = -1;
    if (ok < 0) {
        const char *e = getenv("IRIS_SCHEDULE_SCALAR");
        __builtin_cpu_init();
        ok = !(e && atoi(e) > 0) && __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    }
    return ok;
}

/* elements handled 8-wide, then 4-wide, before the scalar tail */
static void lane_plan(int count, int *n8, int *n4) {
    *n8 = count >= 8 ? count & ~7 : 0;
    *n4 = count - *n8 >= 4 ? 4 : 0;
}

VEC static inline __m256 rcp_nr8(__m256 b) {
    const __m256 r = _mm256_rcp_ps(b);
    return _mm256_sub_ps(_mm256_add_ps(r, r), _mm256_mul_ps(r, _mm256_mul_ps(r, b)));
}

VEC static inline __m128 rcp_nr4(__m128 b) {
    const __m128 r = _mm_rcp_ps(b);
    return _mm_sub_ps(_mm_add_ps(r, r), _mm_mul_ps(r, _mm_mul_ps(r, b)));
}

VEC static inline __m256 iota8(int i0) {
    return _mm256_cvtepi32_ps(_mm256_setr_epi32(i0, i0 + 1, i0 + 2, i0 + 3, i0 + 4, i0 + 5, i0 + 6, i0 + 7));
}

VEC static inline __m128 iota4(int i0) { return _mm_cvtepi32_ps(_mm_setr_epi32(i0, i0 + 1, i0 + 2, i0 + 3)); }

static float *alloc_sched(int num_steps) {
    if (num_steps < 0) return NULL;
    return (float *)malloc((size_t)(num_steps + 1) * sizeof(float));
}

/* iris_linear_schedule (:61-68): 1 - i * (1 / n), fused, in every lane class */
float *iris_linear_schedule(int num_steps) {
    float *s = alloc_sched(num_steps);
    if (!s) return NULL;
    const float inv = 1.0f / (float)num_steps;
    for (int i = 0; i <= num_steps; i++) s[i] = fmaf(-(float)i, inv, 1.0f);
    return s;
}

/* iris_power_schedule (:75-84): 1 - powf(i * (1 / n), alpha) */
VEC static int power_lanes(float *s, int num_steps, float inv, float alpha) {
    int n8, n4, i = 0;
    lane_plan(num_steps + 1, &n8, &n4);
    for (; i < n8; i += 8)
        _mm256_storeu_ps(s + i, _mm256_sub_ps(_mm256_set1_ps(1.0f),
                                              _ZGVdN8vv_powf(_mm256_mul_ps(iota8(i), _mm256_set1_ps(inv)),
                                                             _mm256_set1_ps(alpha))));
    if (n4) {
        _mm_storeu_ps(s + i, _mm_sub_ps(_mm_set1_ps(1.0f), _ZGVbN4vv_powf(_mm_mul_ps(iota4(i), _mm_set1_ps(inv)),
                                                                          _mm_set1_ps(alpha))));
        i += 4;
    }
    return i;
}

float *iris_power_schedule(int num_steps, float alpha) {
    float *s = alloc_sched(num_steps);
    if (!s) return NULL;
    const float inv = 1.0f / (float)num_steps;
    int i = vec_ok() ? power_lanes(s, num_steps, inv, alpha) : 0;
    for (; i <= num_steps; i++) s[i] = 1.0f - powf((float)i * inv, alpha);
    return s;
}

/* iris_sigmoid_schedule (:90-107): 1 - 1 / (1 + expf(-((t - 0.5) * 10 + shift)))
 * with t = i * (1 / n); the exponent's argument is one fused
 * -((t - 0.5) * 10) - shift, itself from t - 0.5 = fma(i, 1/n, -0.5) */
VEC static int sigmoid_lanes(float *s, int num_steps, float inv, float shift) {
    int n8, n4, i = 0;
    lane_plan(num_steps + 1, &n8, &n4);
    for (; i < n8; i += 8) {
        const __m256 tm = _mm256_fmadd_ps(iota8(i), _mm256_set1_ps(inv), _mm256_set1_ps(-0.5f));
        const __m256 arg = _mm256_fnmsub_ps(tm, _mm256_set1_ps(10.0f), _mm256_set1_ps(shift));
        const __m256 d = _mm256_add_ps(_ZGVdN8v_expf(arg), _mm256_set1_ps(1.0f));
        _mm256_storeu_ps(s + i, _mm256_sub_ps(_mm256_set1_ps(1.0f), rcp_nr8(d)));
    }
    if (n4) {
        const __m128 tm = _mm_fmadd_ps(iota4(i), _mm_set1_ps(inv), _mm_set1_ps(-0.5f));
        const __m128 arg = _mm_fnmsub_ps(tm, _mm_set1_ps(10.0f), _mm_set1_ps(shift));
        const __m128 d = _mm_add_ps(_ZGVbN4v_expf(arg), _mm_set1_ps(1.0f));
        _mm_storeu_ps(s + i, _mm_sub_ps(_mm_set1_ps(1.0f), rcp_nr4(d)));
        i += 4;
    }
    return i;
}

float *iris_sigmoid_schedule(int num_steps, float shift) {
    float *s = alloc_sched(num_steps);
    if (!s) return NULL;
    const float inv = 1.0f / (float)num_steps;
    int i = vec_ok() ? sigmoid_lanes(s, num_steps, inv, shift) : 0;
    for (; i <= num_steps; i++) {
        const float tm = fmaf((float)i, inv, -0.5f);
        const float e = expf(-fmaf(tm, 10.0f, shift));
        s[i] = 1.0f - 1.0f / (e + 1.0f);
    }
    s[0] = 1.0f;
    s[num_steps] = 0.0f;
    return s;
}

/* iris_resolution_schedule (:113-136): 1 - powf(i * (1 / n), 1 + shift / 2)
 * for i >= 1 (the loop from i = 1 is the vectorized one), s[0] = 1 */
VEC static int resolution_lanes(float *s, int num_steps, float inv, float ex) {
    int n8, n4, k = 0;
    lane_plan(num_steps, &n8, &n4);
    for (; k < n8; k += 8)
        _mm256_storeu_ps(s + 1 + k, _mm256_sub_ps(_mm256_set1_ps(1.0f),
                                                  _ZGVdN8vv_powf(_mm256_mul_ps(iota8(1 + k), _mm256_set1_ps(inv)),
                                                                 _mm256_set1_ps(ex))));
    if (n4) {
        _mm_storeu_ps(s + 1 + k, _mm_sub_ps(_mm_set1_ps(1.0f),
                                            _ZGVbN4vv_powf(_mm_mul_ps(iota4(1 + k), _mm_set1_ps(inv)),
                                                           _mm_set1_ps(ex))));
        k += 4;
    }
    return k;
}

float *iris_resolution_schedule(int num_steps, int height, int width) {
    float *s = alloc_sched(num_steps);
    if (!s) return NULL;
    const int pixels = height * width;
    const float ex = pixels >= 1024 * 1024 ? 1.5f : pixels >= 512 * 512 ? 1.25f : 1.0f;
    s[0] = 1.0f;
    if (num_steps == 0) return s;
    const float inv = 1.0f / (float)num_steps;
    int k = vec_ok() ? resolution_lanes(s, num_steps, inv, ex) : 0;
    for (; k < num_steps; k++) s[1 + k] = 1.0f - powf((float)(1 + k) * inv, ex);
    return s;
}

/* compute_empirical_mu (:144-158): m200 = a2 seq + b2 and, up to 4300 tokens,
 * a = ((m200 - a1 seq) - b1) * (1 / 190), mu = (m200 + n a) - 200 a, each
 * line fused the way the reference build evaluates it */
static float empirical_mu(int seq, int n) {
    const float a1 = 8.73809524e-05f, b1 = 1.89833333f, a2 = 0.00016927f, b2 = 0.45666666f;
    const float fs = (float)seq;
    const float m200 = fmaf(a2, fs, b2);
    if (seq > 4300) return m200;
    const float a = (fmaf(-fs, a1, m200) - b1) * (1.0f / 190.0f);
    return fmaf(-a, 200.0f, fmaf((float)n, a, m200));
}

/* iris_official_schedule (:160-182): for t = 1 - i * (1 / n) strictly inside
 * (0, 1), e^mu / (e^mu + (1 / t - 1)); t >= 1 gives 1 and t <= 0 gives 0.
 * 8-wide lanes: e * rcp_nr(rcp_nr(t) + (e - 1)); 4-wide lanes:
 * e * rcp_nr((rcp_nr(t) - 1) + e); scalar: e / ((1 / t - 1) + e). */
VEC static int official_lanes(float *s, int num_steps, float inv, float mu) {
    int n8, n4, i = 0;
    lane_plan(num_steps + 1, &n8, &n4);
    float u[8], v[8];
    if (n8) {
        const __m256 e = _ZGVdN8v_expf(_mm256_set1_ps(mu));
        const __m256 em1 = _mm256_add_ps(e, _mm256_set1_ps(-1.0f));
        for (; i < n8; i += 8) {
            const __m256 uu = _mm256_mul_ps(iota8(i), _mm256_set1_ps(inv));
            const __m256 r1 = rcp_nr8(_mm256_sub_ps(_mm256_set1_ps(1.0f), uu));
            _mm256_storeu_ps(v, _mm256_mul_ps(e, rcp_nr8(_mm256_add_ps(r1, em1))));
            _mm256_storeu_ps(u, uu);
            for (int j = 0; j < 8; j++) s[i + j] = u[j] >= 1.0f ? 0.0f : u[j] <= 0.0f ? 1.0f : v[j];
        }
    }
    if (n4) {
        const __m128 e = _ZGVbN4v_expf(_mm_set1_ps(mu));
        const __m128 uu = _mm_mul_ps(iota4(i), _mm_set1_ps(inv));
        const __m128 r1 = rcp_nr4(_mm_sub_ps(_mm_set1_ps(1.0f), uu));
        _mm_storeu_ps(v, _mm_mul_ps(e, rcp_nr4(_mm_add_ps(_mm_add_ps(r1, _mm_set1_ps(-1.0f)), e))));
        _mm_storeu_ps(u, uu);
        for (int j = 0; j < 4; j++) s[i + j] = u[j] >= 1.0f ? 0.0f : u[j] <= 0.0f ? 1.0f : v[j];
        i += 4;
    }
    return i;
}

float *iris_official_schedule(int num_steps, int image_seq_len) {
    float *s = alloc_sched(num_steps);
    if (!s) return NULL;
    const float mu = empirical_mu(image_seq_len, num_steps);
    const float inv = 1.0f / (float)num_steps;
    int i = vec_ok() ? official_lanes(s, num_steps, inv, mu) : 0;
    for (; i <= num_steps; i++) {
        const float uu = (float)i * inv;
        if (uu >= 1.0f) s[i] = 0.0f;
        else if (uu <= 0.0f) s[i] = 1.0f;
        else {
            const float e = expf(mu);
            s[i] = e / ((1.0f / (1.0f - uu) - 1.0f) + e);
        }
    }
    return s;
}

/* iris_zimage_schedule (:216-244): n sigmas raw = 1 + i * ((smin - 1) / (n - 1))
 * (fused), shifted as shift raw / (1 + (shift - 1) raw) with the denominator
 * fused, then a terminal 0; smin = shift / 1000 / (1 + (shift - 1) / 1000).
 * The shift is 3, or IRIS_ZIMAGE_SHIFT when that parses to a positive value. */
VEC static int zimage_lanes(float *s, int num_steps, float c, float shift, float sm1) {
    int n8, n4, i = 0;
    lane_plan(num_steps, &n8, &n4);
    for (; i < n8; i += 8) {
        const __m256 raw = _mm256_fmadd_ps(iota8(i), _mm256_set1_ps(c), _mm256_set1_ps(1.0f));
        const __m256 num = _mm256_mul_ps(raw, _mm256_set1_ps(shift));
        const __m256 den = _mm256_fmadd_ps(raw, _mm256_set1_ps(sm1), _mm256_set1_ps(1.0f));
        _mm256_storeu_ps(s + i, _mm256_mul_ps(num, rcp_nr8(den)));
    }
    if (n4) {
        const __m128 raw = _mm_fmadd_ps(iota4(i), _mm_set1_ps(c), _mm_set1_ps(1.0f));
        const __m128 num = _mm_mul_ps(raw, _mm_set1_ps(shift));
        const __m128 den = _mm_fmadd_ps(raw, _mm_set1_ps(sm1), _mm_set1_ps(1.0f));
        _mm_storeu_ps(s + i, _mm_mul_ps(num, rcp_nr4(den)));
        i += 4;
    }
    return i;
}

float *iris_zimage_schedule(int num_steps, int image_seq_len) {
    (void)image_seq_len;
    float *s = alloc_sched(num_steps);
    if (!s) return NULL;
    float shift = 3.0f;
    const char *env = getenv("IRIS_ZIMAGE_SHIFT");
    if (env) {
        const float v = (float)atof(env);
        if (v > 0.0f) shift = v;
    }
    const float sm1 = shift - 1.0f;
    const float smin = (shift * (1.0f / 1000.0f)) / fmaf(sm1, 1.0f / 1000.0f, 1.0f);
    if (num_steps >= 1) {
        if (num_steps == 1) {
            s[0] = 1.0f;
        } else {
            const float c = (smin - 1.0f) * (1.0f / (float)(num_steps - 1));
            int i = vec_ok() ? zimage_lanes(s, num_steps, c, shift, sm1) : 0;
            for (; i < num_steps; i++) {
                const float raw = fmaf((float)i, c, 1.0f);
                s[i] = (raw * shift) / fmaf(raw, sm1, 1.0f);
            }
        }
    }
    s[num_steps] = 0.0f;
    return s;
}
