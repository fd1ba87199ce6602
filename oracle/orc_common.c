/*
 * orc_common.c - BLAS binding and scalar kernels of the oracle.
 * TEST INFRASTRUCTURE ONLY (see iris_oracle.h).
 */
#include "orc_internal.h"

#include <dlfcn.h>
#include <immintrin.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef void (*sgemm_fn_t)(int order, int ta, int tb, int M, int N, int K, float alpha,
                           const float *A, int lda, const float *B, int ldb, float beta,
                           float *C, int ldc);
static sgemm_fn_t g_sgemm = NULL;
static char g_info[256] = "builtin loops";

int orc_set_blas(const char *so_path, const char *prefix, int threads) {
    void *h = dlopen(so_path, RTLD_NOW | RTLD_LOCAL);
    if (!h) { fprintf(stderr, "orc_set_blas: %s\n", dlerror()); return -1; }
    char sym[128];
    snprintf(sym, sizeof(sym), "%scblas_sgemm", prefix);
    g_sgemm = (sgemm_fn_t)dlsym(h, sym);
    if (!g_sgemm) return -1;
    snprintf(sym, sizeof(sym), "%sopenblas_set_num_threads", prefix);
    void (*set_threads)(int) = (void (*)(int))dlsym(h, sym);
    if (set_threads && threads > 0) set_threads(threads);
    snprintf(sym, sizeof(sym), "%sopenblas_get_config", prefix);
    const char *(*get_config)(void) = (const char *(*)(void))dlsym(h, sym);
    snprintf(sym, sizeof(sym), "%sopenblas_get_corename", prefix);
    const char *(*get_core)(void) = (const char *(*)(void))dlsym(h, sym);
    snprintf(g_info, sizeof(g_info), "%s | %s | threads=%d",
             get_config ? get_config() : "OpenBLAS", get_core ? get_core() : "?", threads);
    return 0;
}

const char *orc_blas_info(void) { return g_info; }

/* CBLAS enum values (RowMajor=101, NoTrans=111, Trans=112). */
enum { ROWMAJOR = 101, NOTRANS = 111, TRANS = 112 };

/* C[M,N] = alpha * A[M,K] * B^T (B is [N,K]) + beta*C */
void orc_sgemm_nt(int M, int N, int K, float alpha, const float *A, int lda,
                  const float *B, int ldb, float beta, float *C, int ldc) {
    if (g_sgemm) {
        g_sgemm(ROWMAJOR, NOTRANS, TRANS, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
        return;
    }
#pragma omp parallel for schedule(static) if ((long)M * N * K > (1L << 22))
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) {
            const float *a = A + (size_t)m * lda, *b = B + (size_t)n * ldb;
            float s = 0.0f;
            for (int k = 0; k < K; k++) s += a[k] * b[k];
            float *c = C + (size_t)m * ldc + n;
            *c = alpha * s + (beta != 0.0f ? beta * *c : 0.0f);
        }
    }
}

/* C[M,N] = alpha * A[M,K] * B[K,N] + beta*C */
void orc_sgemm_nn(int M, int N, int K, float alpha, const float *A, int lda,
                  const float *B, int ldb, float beta, float *C, int ldc) {
    if (g_sgemm) {
        g_sgemm(ROWMAJOR, NOTRANS, NOTRANS, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
        return;
    }
#pragma omp parallel for schedule(static) if ((long)M * N * K > (1L << 22))
    for (int m = 0; m < M; m++) {
        float *c = C + (size_t)m * ldc;
        for (int n = 0; n < N; n++) c[n] = beta != 0.0f ? beta * c[n] : 0.0f;
        for (int k = 0; k < K; k++) {
            float a = alpha * A[(size_t)m * lda + k];
            const float *b = B + (size_t)k * ldb;
            for (int n = 0; n < N; n++) c[n] += a * b[n];
        }
    }
}

/* fast_expf: range reduction + degree-5 polynomial, iris_kernels.h:21-35. */
float orc_fast_expf(float x) {
    if (x < -87.3f) return 0.0f;
    if (x > 88.7f) return 1e38f;
    float n = floorf(x * 1.4426950408889634f + 0.5f);
    float r = x - n * 0.6931471805599453f;
    float p = 1.0f + r * (1.0f + r * (0.5f + r * (0.16666667f + r * (0.04166667f + r * 0.00833333f))));
    union { float f; int32_t i; } v;
    v.f = p;
    v.i += (int32_t)((uint32_t)(int32_t)n << 23);
    return v.f;
}

/* iris_linear (BLAS branch), iris_kernels.c:220-290: y = x W^T (+ b). */
void orc_linear(float *y, const float *x, const float *W, const float *b,
                int seq, int in_dim, int out_dim) {
    orc_sgemm_nt(seq, out_dim, in_dim, 1.0f, x, in_dim, W, in_dim, 0.0f, y, out_dim);
    if (b)
        for (int s = 0; s < seq; s++)
            for (int o = 0; o < out_dim; o++) y[(size_t)s * out_dim + o] += b[o];
}

/* iris_silu, iris_kernels.c:610-621 (fast_expf). */
void orc_silu(float *x, int n) {
    for (int i = 0; i < n; i++) x[i] = x[i] / (1.0f + orc_fast_expf(-x[i]));
}

/* iris_silu_mul, iris_kernels.c:626-638. */
void orc_silu_mul(float *gate, const float *up, size_t n) {
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; i++) {
        float v = gate[i];
        gate[i] = (v / (1.0f + orc_fast_expf(-v))) * up[i];
    }
}

/* iris_softmax_cpu, iris_kernels.c:641-664. */
void orc_softmax(float *x, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        float *row = x + (size_t)r * cols;
        float mx = row[0];
        for (int c = 1; c < cols; c++) if (row[c] > mx) mx = row[c];
        float sum = 0.0f;
        for (int c = 0; c < cols; c++) { row[c] = orc_fast_expf(row[c] - mx); sum += row[c]; }
        float inv = 1.0f / sum;
        for (int c = 0; c < cols; c++) row[c] *= inv;
    }
}

/* iris_rms_norm, iris_kernels.c:511-540. */
void orc_rms_norm(float *out, const float *x, const float *w, int rows, int dim, float eps) {
    for (int s = 0; s < rows; s++) {
        const float *xr = x + (size_t)s * dim;
        float *o = out + (size_t)s * dim;
        float ss = 0.0f;
        for (int i = 0; i < dim; i++) ss += xr[i] * xr[i];
        float inv = 1.0f / sqrtf(ss / dim + eps);
        for (int i = 0; i < dim; i++) o[i] = xr[i] * inv * w[i];
    }
}

void orc_free(void *p) { free(p); }

/* The reference is built with -O3 -march=native -ffast-math (Makefile:5). Under
 * those flags gcc evaluates `1.0f / powf(theta, e)` in its RoPE table builders
 * (iris_transformer_flux.c:903-906, iris_transformer_zimage.c:603) as glibc
 * libmvec's vector powf(theta, -e); cosf/sinf and the timestep-frequency expf
 * (iris_transformer_flux.c:1354, iris_transformer_zimage.c:550) stay scalar.
 * These wrappers call the same libmvec entry point explicitly, so the tables do
 * not depend on this file's flags. */
__m128 _ZGVbN4vv_powf(__m128, __m128);
__m128 _ZGVbN4v_expf(__m128);

void orc_vpowf(float *out, const float *x, const float *y, int n) {
    for (int i = 0; i < n; i += 4) {
        float xa[4] = {1, 1, 1, 1}, ya[4] = {0, 0, 0, 0}, o[4];
        for (int j = 0; j < 4 && i + j < n; j++) { xa[j] = x[i + j]; ya[j] = y[i + j]; }
        _mm_storeu_ps(o, _ZGVbN4vv_powf(_mm_loadu_ps(xa), _mm_loadu_ps(ya)));
        for (int j = 0; j < 4 && i + j < n; j++) out[i + j] = o[j];
    }
}

void orc_vexpf(float *out, const float *x, int n) {
    for (int i = 0; i < n; i += 4) {
        float xa[4] = {0, 0, 0, 0}, o[4];
        for (int j = 0; j < 4 && i + j < n; j++) xa[j] = x[i + j];
        _mm_storeu_ps(o, _ZGVbN4v_expf(_mm_loadu_ps(xa)));
        for (int j = 0; j < 4 && i + j < n; j++) out[i + j] = o[j];
    }
}

/* RoPE base frequencies theta^(-2d/axis_dim), d < half (see above). */
void orc_rope_bases(float *base, int half, int axis_dim, float theta) {
    float x[64], y[64];
    for (int d = 0; d < half; d++) { x[d] = theta; y[d] = -((float)(2 * d) / (float)axis_dim); }
    orc_vpowf(base, x, y, half);
}

/* ---- tensor loading helpers ---- */

float *orc_load_f32(const iris_st_set_t *s, const char *name) {
    const iris_st_file_t *f;
    const iris_st_tensor_t *t = iris_st_set_find(s, name, &f);
    if (!t) { fprintf(stderr, "oracle: required tensor %s not found\n", name); return NULL; }
    float *d = (float *)malloc((size_t)iris_st_numel(t) * sizeof(float));
    if (!d || iris_st_read_f32(f, t, d)) { free(d); return NULL; }
    return d;
}

/* Synthetic tensor: bf16 values of the seeded generator widened to f32, exactly
 * what a bf16 safetensors file written from the same generator would load as. */
float *orc_synth_f32(uint64_t seed, const char *name, size_t n, float mean, float std) {
    float *d = (float *)malloc(n * sizeof(float));
    if (!d) return NULL;
    uint64_t ts = iris_synth_seed(seed, name);
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; i++)
        d[i] = iris_bf16_to_f32(iris_f32_to_bf16(iris_synth_value(ts, i, mean, std)));
    return d;
}
