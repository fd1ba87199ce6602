/*
 * iris_schedule.c - timestep schedules with the reference build's bits.
 *
 * The reference compiles iris_sample.c:61-244 with -O3 -march=native
 * -ffast-math (its Makefile:5). gcc then vectorizes every schedule loop and
 * rewrites its arithmetic:
 *   - a loop over `count` elements runs a main loop of wide blocks, one
 *     narrower epilogue block when enough elements remain, and scalar code
 *     for the rest; the lane classes do not compute alike. The widths follow
 *     the host's vector ISA:
 *       AVX2 + FMA: 8-wide blocks while count >= 8, one 4-wide block when at
 *         least 4 elements remain, at most 3 scalar;
 *       AVX-512 (F + VL): 16-wide blocks while count >= 16, one 8-wide block
 *         when at least 8 remain, at most 7 scalar;
 *   - in the vector lanes a division a / b becomes a * rcp_nr(b), where
 *     rcp_nr(b) = (r + r) - r * (r * b) refines the hardware reciprocal
 *     estimate r by one Newton step: rcpps for 4- and 8-wide blocks, vrcp14ps
 *     for 16-wide ones; the scalar tail divides;
 *   - expf / powf of the vector lanes are glibc libmvec's entry points of
 *     the block's width (_ZGVeN16v_expf / _ZGVeN16vv_powf, _ZGVdN8v_expf /
 *     _ZGVdN8vv_powf, _ZGVbN4v_expf / _ZGVbN4vv_powf), the scalar tail calls
 *     libm;
 *   - i / n becomes i * (1 / n), a - b * c and a + b * c become fused
 *     multiply-adds, and sums are reassociated (the main loop and the
 *     epilogue block of iris_official_schedule associate one sum
 *     differently).
 * This file performs those same operations in the same order, with the same
 * instructions (AVX2 / AVX-512 + FMA intrinsics, the libmvec entry points),
 * so on a given host every schedule equals the reference build's on that
 * host bit for bit. The last bit of the reciprocal estimates is specific to
 * the CPU model, and so is the reference build's schedule; the lane classes
 * follow the element count and the ISA, not the CPU model. The file is
 * compiled with -ffp-contract=off so that only the fused operations written
 * here are fused.
 *
 * The lane plan is chosen per call from the CPU (__builtin_cpu_supports):
 * AVX-512 where the CPU has AVX-512F and VL, else AVX2 where it has AVX2 and
 * FMA, else every element takes the scalar formula (the build's scalar
 * tail: the reference formulas in plain IEEE float). The environment can
 * only narrow that choice: IRIS_SCHEDULE_ISA=avx2 or =scalar (the plan of a
 * reference build made on such a host), IRIS_SCHEDULE_SCALAR=1 as scalar.
 */
#include "../../include/iris_sample.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

__m512 _ZGVeN16v_expf(__m512);
__m256 _ZGVdN8v_expf(__m256);
__m128 _ZGVbN4v_expf(__m128);
__m512 _ZGVeN16vv_powf(__m512, __m512);
__m256 _ZGVdN8vv_powf(__m256, __m256);
__m128 _ZGVbN4vv_powf(__m128, __m128);

#define VEC __attribute__((target("avx2,fma")))
#define VEC512 __attribute__((target("avx512f,avx512vl,avx2,fma")))

enum { PLAN_SCALAR = 0, PLAN_AVX2 = 2, PLAN_AVX512 = 3 };

/* the widest lane plan the CPU runs, narrowed by the environment */
static int lane_isa(void) {
    __builtin_cpu_init();
    int best = PLAN_SCALAR;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) {
        best = PLAN_AVX2;
        if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512vl")) best = PLAN_AVX512;
    }
    const char *sc = getenv("IRIS_SCHEDULE_SCALAR");
    if (sc && atoi(sc) > 0) return PLAN_SCALAR;
    const char *want = getenv("IRIS_SCHEDULE_ISA");
    if (want) {
        const int w = !strcmp(want, "scalar") ? PLAN_SCALAR : !strcmp(want, "avx2") ? PLAN_AVX2 : best;
        if (w < best) best = w;
    }
    return best;
}

/* elements of the main loop (width w) and of the epilogue block (w / 2) */
static void lane_plan(int count, int w, int *nmain, int *nepi) {
    *nmain = count >= w ? count - count % w : 0;
    *nepi = count - *nmain >= w / 2 ? w / 2 : 0;
}

VEC512 static inline __m512 rcp_nr16(__m512 b) {
    const __m512 r = _mm512_rcp14_ps(b);
    return _mm512_sub_ps(_mm512_add_ps(r, r), _mm512_mul_ps(r, _mm512_mul_ps(r, b)));
}

VEC static inline __m256 rcp_nr8(__m256 b) {
    const __m256 r = _mm256_rcp_ps(b);
    return _mm256_sub_ps(_mm256_add_ps(r, r), _mm256_mul_ps(r, _mm256_mul_ps(r, b)));
}

VEC static inline __m128 rcp_nr4(__m128 b) {
    const __m128 r = _mm_rcp_ps(b);
    return _mm_sub_ps(_mm_add_ps(r, r), _mm_mul_ps(r, _mm_mul_ps(r, b)));
}

VEC512 static inline __m512 iota16(int i0) {
    return _mm512_cvtepi32_ps(_mm512_add_epi32(_mm512_set1_epi32(i0),
                                               _mm512_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15)));
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
/* Runs the lane plan over count elements from element `first`: blocks of
 * the main width through `wide`, the epilogue block through `narrow`, both
 * given the block's first element index; returns the elements done. */
#define RUN_LANES(isa, count, first, W16, W8, E8, W4)                            \
    ({                                                                           \
        int nm_, ne_, k_ = 0;                                                    \
        if ((isa) == PLAN_AVX512) {                                              \
            lane_plan((count), 16, &nm_, &ne_);                                  \
            for (; k_ < nm_; k_ += 16) W16((first) + k_);                        \
            if (ne_) { E8((first) + k_); k_ += 8; }                              \
        } else if ((isa) == PLAN_AVX2) {                                         \
            lane_plan((count), 8, &nm_, &ne_);                                   \
            for (; k_ < nm_; k_ += 8) W8((first) + k_);                          \
            if (ne_) { W4((first) + k_); k_ += 4; }                              \
        }                                                                        \
        k_;                                                                      \
    })

float *iris_linear_schedule(int num_steps) {
    float *s = alloc_sched(num_steps);
    if (!s) return NULL;
    const float inv = 1.0f / (float)num_steps;
    for (int i = 0; i <= num_steps; i++) s[i] = fmaf(-(float)i, inv, 1.0f);
    return s;
}

/* iris_power_schedule (:75-84): 1 - powf(i * (1 / n), alpha), in every
 * lane class (the epilogue block computes like the main loop) */
VEC512 static void power16(float *s, int i, float inv, float alpha) {
    _mm512_storeu_ps(s + i, _mm512_sub_ps(_mm512_set1_ps(1.0f), _ZGVeN16vv_powf(_mm512_mul_ps(iota16(i), _mm512_set1_ps(inv)),
                                                                                 _mm512_set1_ps(alpha))));
}

VEC static void power8(float *s, int i, float inv, float alpha) {
    _mm256_storeu_ps(s + i, _mm256_sub_ps(_mm256_set1_ps(1.0f), _ZGVdN8vv_powf(_mm256_mul_ps(iota8(i), _mm256_set1_ps(inv)),
                                                                                _mm256_set1_ps(alpha))));
}

VEC static void power4(float *s, int i, float inv, float alpha) {
    _mm_storeu_ps(s + i, _mm_sub_ps(_mm_set1_ps(1.0f), _ZGVbN4vv_powf(_mm_mul_ps(iota4(i), _mm_set1_ps(inv)),
                                                                      _mm_set1_ps(alpha))));
}

float *iris_power_schedule(int num_steps, float alpha) {
    float *s = alloc_sched(num_steps);
    if (!s) return NULL;
    const float inv = 1.0f / (float)num_steps;
#define P16(i) power16(s, i, inv, alpha)
#define P8(i) power8(s, i, inv, alpha)
#define P4(i) power4(s, i, inv, alpha)
    int i = RUN_LANES(lane_isa(), num_steps + 1, 0, P16, P8, P8, P4);
#undef P16
#undef P8
#undef P4
    for (; i <= num_steps; i++) s[i] = 1.0f - powf((float)i * inv, alpha);
    return s;
}

/* iris_sigmoid_schedule (:90-107): 1 - 1 / (1 + expf(-((t - 0.5) * 10 + shift)))
 * with t = i * (1 / n); the exponent's argument is one fused
 * -((t - 0.5) * 10) - shift, itself from t - 0.5 = fma(i, 1/n, -0.5) */
VEC512 static void sigmoid16(float *s, int i, float inv, float shift) {
    const __m512 tm = _mm512_fmadd_ps(iota16(i), _mm512_set1_ps(inv), _mm512_set1_ps(-0.5f));
    const __m512 arg = _mm512_fnmsub_ps(tm, _mm512_set1_ps(10.0f), _mm512_set1_ps(shift));
    const __m512 d = _mm512_add_ps(_ZGVeN16v_expf(arg), _mm512_set1_ps(1.0f));
    _mm512_storeu_ps(s + i, _mm512_sub_ps(_mm512_set1_ps(1.0f), rcp_nr16(d)));
}

VEC static void sigmoid8(float *s, int i, float inv, float shift) {
    const __m256 tm = _mm256_fmadd_ps(iota8(i), _mm256_set1_ps(inv), _mm256_set1_ps(-0.5f));
    const __m256 arg = _mm256_fnmsub_ps(tm, _mm256_set1_ps(10.0f), _mm256_set1_ps(shift));
    const __m256 d = _mm256_add_ps(_ZGVdN8v_expf(arg), _mm256_set1_ps(1.0f));
    _mm256_storeu_ps(s + i, _mm256_sub_ps(_mm256_set1_ps(1.0f), rcp_nr8(d)));
}

VEC static void sigmoid4(float *s, int i, float inv, float shift) {
    const __m128 tm = _mm_fmadd_ps(iota4(i), _mm_set1_ps(inv), _mm_set1_ps(-0.5f));
    const __m128 arg = _mm_fnmsub_ps(tm, _mm_set1_ps(10.0f), _mm_set1_ps(shift));
    const __m128 d = _mm_add_ps(_ZGVbN4v_expf(arg), _mm_set1_ps(1.0f));
    _mm_storeu_ps(s + i, _mm_sub_ps(_mm_set1_ps(1.0f), rcp_nr4(d)));
}

float *iris_sigmoid_schedule(int num_steps, float shift) {
    float *s = alloc_sched(num_steps);
    if (!s) return NULL;
    const float inv = 1.0f / (float)num_steps;
#define G16(i) sigmoid16(s, i, inv, shift)
#define G8(i) sigmoid8(s, i, inv, shift)
#define G4(i) sigmoid4(s, i, inv, shift)
    int i = RUN_LANES(lane_isa(), num_steps + 1, 0, G16, G8, G8, G4);
#undef G16
#undef G8
#undef G4
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
/* (the blocks are power16 / power8 / power4 with alpha = the exponent) */

float *iris_resolution_schedule(int num_steps, int height, int width) {
    float *s = alloc_sched(num_steps);
    if (!s) return NULL;
    const int pixels = height * width;
    const float ex = pixels >= 1024 * 1024 ? 1.5f : pixels >= 512 * 512 ? 1.25f : 1.0f;
    s[0] = 1.0f;
    if (num_steps == 0) return s;
    const float inv = 1.0f / (float)num_steps;
#define R16(i) power16(s, i, inv, ex)
#define R8(i) power8(s, i, inv, ex)
#define R4(i) power4(s, i, inv, ex)
    int k = RUN_LANES(lane_isa(), num_steps, 1, R16, R8, R8, R4);
#undef R16
#undef R8
#undef R4
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
 * Main-loop blocks: e * rcp_nr(rcp_nr(t) + (e - 1)); the epilogue block:
 * e * rcp_nr((rcp_nr(t) - 1) + e); scalar: e / ((1 / t - 1) + e). e is the
 * libmvec expf of the block's width. */
static void official_pick(float *s, int i, int w, const float *u, const float *v) {
    for (int j = 0; j < w; j++) s[i + j] = u[j] >= 1.0f ? 0.0f : u[j] <= 0.0f ? 1.0f : v[j];
}

VEC512 static void official16(float *s, int i, float inv, float mu) {
    float u[16], v[16];
    const __m512 e = _ZGVeN16v_expf(_mm512_set1_ps(mu));
    const __m512 em1 = _mm512_add_ps(e, _mm512_set1_ps(-1.0f));
    const __m512 uu = _mm512_mul_ps(iota16(i), _mm512_set1_ps(inv));
    const __m512 r1 = rcp_nr16(_mm512_sub_ps(_mm512_set1_ps(1.0f), uu));
    _mm512_storeu_ps(v, _mm512_mul_ps(e, rcp_nr16(_mm512_add_ps(r1, em1))));
    _mm512_storeu_ps(u, uu);
    official_pick(s, i, 16, u, v);
}

VEC static void official8(float *s, int i, float inv, float mu) {
    float u[8], v[8];
    const __m256 e = _ZGVdN8v_expf(_mm256_set1_ps(mu));
    const __m256 em1 = _mm256_add_ps(e, _mm256_set1_ps(-1.0f));
    const __m256 uu = _mm256_mul_ps(iota8(i), _mm256_set1_ps(inv));
    const __m256 r1 = rcp_nr8(_mm256_sub_ps(_mm256_set1_ps(1.0f), uu));
    _mm256_storeu_ps(v, _mm256_mul_ps(e, rcp_nr8(_mm256_add_ps(r1, em1))));
    _mm256_storeu_ps(u, uu);
    official_pick(s, i, 8, u, v);
}

VEC static void official8_epi(float *s, int i, float inv, float mu) {
    float u[8], v[8];
    const __m256 e = _ZGVdN8v_expf(_mm256_set1_ps(mu));
    const __m256 uu = _mm256_mul_ps(iota8(i), _mm256_set1_ps(inv));
    const __m256 r1 = rcp_nr8(_mm256_sub_ps(_mm256_set1_ps(1.0f), uu));
    _mm256_storeu_ps(v, _mm256_mul_ps(e, rcp_nr8(_mm256_add_ps(_mm256_add_ps(r1, _mm256_set1_ps(-1.0f)), e))));
    _mm256_storeu_ps(u, uu);
    official_pick(s, i, 8, u, v);
}

VEC static void official4_epi(float *s, int i, float inv, float mu) {
    float u[4], v[4];
    const __m128 e = _ZGVbN4v_expf(_mm_set1_ps(mu));
    const __m128 uu = _mm_mul_ps(iota4(i), _mm_set1_ps(inv));
    const __m128 r1 = rcp_nr4(_mm_sub_ps(_mm_set1_ps(1.0f), uu));
    _mm_storeu_ps(v, _mm_mul_ps(e, rcp_nr4(_mm_add_ps(_mm_add_ps(r1, _mm_set1_ps(-1.0f)), e))));
    _mm_storeu_ps(u, uu);
    official_pick(s, i, 4, u, v);
}

float *iris_official_schedule(int num_steps, int image_seq_len) {
    float *s = alloc_sched(num_steps);
    if (!s) return NULL;
    const float mu = empirical_mu(image_seq_len, num_steps);
    const float inv = 1.0f / (float)num_steps;
#define O16(i) official16(s, i, inv, mu)
#define O8(i) official8(s, i, inv, mu)
#define O8E(i) official8_epi(s, i, inv, mu)
#define O4E(i) official4_epi(s, i, inv, mu)
    int i = RUN_LANES(lane_isa(), num_steps + 1, 0, O16, O8, O8E, O4E);
#undef O16
#undef O8
#undef O8E
#undef O4E
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
VEC512 static void zimage16(float *s, int i, float c, float shift, float sm1) {
    const __m512 raw = _mm512_fmadd_ps(iota16(i), _mm512_set1_ps(c), _mm512_set1_ps(1.0f));
    const __m512 num = _mm512_mul_ps(raw, _mm512_set1_ps(shift));
    const __m512 den = _mm512_fmadd_ps(raw, _mm512_set1_ps(sm1), _mm512_set1_ps(1.0f));
    _mm512_storeu_ps(s + i, _mm512_mul_ps(num, rcp_nr16(den)));
}

VEC static void zimage8(float *s, int i, float c, float shift, float sm1) {
    const __m256 raw = _mm256_fmadd_ps(iota8(i), _mm256_set1_ps(c), _mm256_set1_ps(1.0f));
    const __m256 num = _mm256_mul_ps(raw, _mm256_set1_ps(shift));
    const __m256 den = _mm256_fmadd_ps(raw, _mm256_set1_ps(sm1), _mm256_set1_ps(1.0f));
    _mm256_storeu_ps(s + i, _mm256_mul_ps(num, rcp_nr8(den)));
}

VEC static void zimage4(float *s, int i, float c, float shift, float sm1) {
    const __m128 raw = _mm_fmadd_ps(iota4(i), _mm_set1_ps(c), _mm_set1_ps(1.0f));
    const __m128 num = _mm_mul_ps(raw, _mm_set1_ps(shift));
    const __m128 den = _mm_fmadd_ps(raw, _mm_set1_ps(sm1), _mm_set1_ps(1.0f));
    _mm_storeu_ps(s + i, _mm_mul_ps(num, rcp_nr4(den)));
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
#define Z16(i) zimage16(s, i, c, shift, sm1)
#define Z8(i) zimage8(s, i, c, shift, sm1)
#define Z4(i) zimage4(s, i, c, shift, sm1)
            int i = RUN_LANES(lane_isa(), num_steps, 0, Z16, Z8, Z8, Z4);
#undef Z16
#undef Z8
#undef Z4
            for (; i < num_steps; i++) {
                const float raw = fmaf((float)i, c, 1.0f);
                s[i] = (raw * shift) / fmaf(raw, sm1, 1.0f);
            }
        }
    }
    s[num_steps] = 0.0f;
    return s;
}
