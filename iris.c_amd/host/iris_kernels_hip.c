/*
 * iris_kernels_hip.c - the host-pointer math API of iris_kernels.h on the GPU.
 *
 * The reference routes each of these calls to the GPU only above a size
 * threshold and otherwise computes on the CPU (iris_kernels.c:28-29,
 * :150-161, :224-253, :301-318, :513-520). Here every call runs on the GPU:
 * operands are copied into a growable device staging area, the kernels of
 * csrc/kernels_api.hip (and the MFMA GEMM of csrc/gemm.hip) run on the
 * library's stream, and the result comes back with a synchronous copy.
 *
 * f32 products. A and B are split into bf16 hi/lo parts; one GEMM over three
 * K segments ([Ahi|Ahi|Alo] against [Bhi|Blo|Bhi]) accumulates
 * Ahi.Bhi + Ahi.Blo + Alo.Bhi in f32. The dropped Alo.Blo term and the bf16
 * rounding of lo bound the error near 2^-16 of |A||B| per product, so results
 * track cblas_sgemm (iris_kernels.c:220-336) to about 1e-5 relative.
 * bf16 weights (iris_linear_nobias_bf16, :292-336) are exact in bf16, so two
 * segments suffice there: [xhi|xlo] against [W|W].
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/iris_hip.h"
#include "../../include/iris_kernels.h"

/* ---- globals of the API (iris_kernels.c:33-44); iris_cancel_requested lives
 *      with the samplers ---- */
iris_substep_callback_t iris_substep_callback = NULL;
iris_step_callback_t iris_step_callback = NULL;
iris_phase_callback_t iris_phase_callback = NULL;
iris_step_image_callback_t iris_step_image_callback = NULL;
void *iris_step_image_vae = NULL;
iris_text_progress_callback_t iris_text_progress_callback = NULL;
iris_vae_progress_callback_t iris_vae_progress_callback = NULL;
int iris_verbose = 0;

/* ---- device staging: a few growable slots, reused call to call. Each call
 *      ends with a synchronous device-to-host copy, so a slot is idle
 *      whenever a later call regrows it. ---- */
enum { SLOT_A, SLOT_B, SLOT_C, SLOT_D, SLOT_SA, SLOT_SB, N_SLOTS };
static void *g_slot[N_SLOTS];
static size_t g_slot_bytes[N_SLOTS];

static void *slot(int s, size_t bytes) {
    if (bytes == 0) bytes = 256;
    if (g_slot_bytes[s] >= bytes) return g_slot[s];
    if (g_slot[s]) iris_hip_free(g_slot[s]);
    size_t want = bytes + bytes / 4;
    want = (want + 4095) & ~(size_t)4095;
    g_slot[s] = iris_hip_malloc(want);
    g_slot_bytes[s] = g_slot[s] ? want : 0;
    return g_slot[s];
}

static int fail(const char *what, float *out, size_t n) {
    fprintf(stderr, "iris_kernels (HIP): %s failed: %s\n", what, iris_hip_last_error());
    if (out && n) memset(out, 0, n * sizeof(float));
    return -1;
}

/* host f32 array -> slot */
static float *up(int s, const float *src, size_t n) {
    float *d = (float *)slot(s, n * sizeof(float));
    if (!d || iris_hip_memcpy_h2d(d, src, n * sizeof(float))) return NULL;
    return d;
}

static int down(float *dst, const float *d, size_t n) { return iris_hip_memcpy_d2h(dst, d, n * sizeof(float)); }

static int pad64(int k) { return (k + 63) / 64 * 64; }

/* ---- elementwise ---- */
static void ew(int op, const char *name, float *out, const float *a, const float *b, float s, int n) {
    if (n <= 0) return;
    const size_t N = (size_t)n;
    float *da = up(SLOT_A, a, N);
    float *db = b ? up(SLOT_B, b, N) : NULL;
    if (!da || (b && !db) || iris_hip_elementwise(op, da, da, db, s, N) || down(out, da, N)) fail(name, out, N);
}

void iris_add(float *out, const float *a, const float *b, int n) { ew(0, "iris_add", out, a, b, 0.0f, n); }
void iris_add_inplace(float *a, const float *b, int n) { ew(0, "iris_add_inplace", a, a, b, 0.0f, n); }
void iris_mul_inplace(float *a, const float *b, int n) { ew(1, "iris_mul_inplace", a, a, b, 0.0f, n); }
void iris_axpy(float *a, float scale, const float *b, int n) { ew(2, "iris_axpy", a, a, b, scale, n); }
void iris_silu(float *x, int n) { ew(3, "iris_silu", x, x, NULL, 0.0f, n); }
void iris_silu_mul(float *gate, const float *up_, int n) { ew(4, "iris_silu_mul", gate, gate, up_, 0.0f, n); }

void iris_copy(float *dst, const float *src, int n) {
    if (n <= 0) return;
    float *d = up(SLOT_A, src, (size_t)n);
    if (!d || down(dst, d, (size_t)n)) fail("iris_copy", dst, (size_t)n);
}

/* ---- products ---- */

/* C[M,N] = A[M,K] . B^T with A, B already split on the device into
 * [rows][nseg * Kp]; bias per column or NULL. */
static int gemm_split(float *dC, const uint16_t *dA, const uint16_t *dB, const float *dbias, int M, int N, int Kp,
                      int nseg) {
    iris_gemm_problem_t p;
    memset(&p, 0, sizeof p);
    p.A = dA;
    p.W = dB;
    p.out = dC;
    p.vec = dbias;
    p.M = M;
    p.N = N;
    p.K = nseg * Kp;
    p.lda = p.ldw = nseg * Kp;
    p.ldo = N;
    p.epi = IRIS_EPI_F32;
    return iris_hip_gemm(&p, 1);
}

/* transB 0: B is [K][N]; 1: B is [N][K] */
static void matmul_any(const char *name, float *C, const float *A, const float *B, const float *bias, int M, int K,
                       int N, int transB) {
    if (M <= 0 || N <= 0) return;
    const size_t MN = (size_t)M * N;
    if (K <= 0) {
        /* empty sum: C = bias (or 0), still produced on the device */
        float *dC = (float *)slot(SLOT_C, MN * sizeof(float));
        if (!dC || iris_hip_memset(dC, 0, MN * sizeof(float))) { fail(name, C, MN); return; }
        if (bias) {
            float *db = up(SLOT_D, bias, (size_t)N);
            if (!db || iris_hip_fill_rows(dC, db, 0, M, N)) { fail(name, C, MN); return; }
        }
        if (down(C, dC, MN)) fail(name, C, MN);
        return;
    }
    const int Kp = pad64(K);
    float *dA = up(SLOT_A, A, (size_t)M * K);
    float *dB = up(SLOT_B, B, (size_t)N * K);
    float *dbias = bias ? up(SLOT_D, bias, (size_t)N) : NULL;
    uint16_t *sA = (uint16_t *)slot(SLOT_SA, (size_t)M * 3 * Kp * 2);
    uint16_t *sB = (uint16_t *)slot(SLOT_SB, (size_t)N * 3 * Kp * 2);
    float *dC = (float *)slot(SLOT_C, MN * sizeof(float));
    if (!dA || !dB || (bias && !dbias) || !sA || !sB || !dC) { fail(name, C, MN); return; }
    if (iris_hip_split_rows(sA, dA, M, K, K, Kp, 3, 4)) { fail(name, C, MN); return; }
    if (transB ? iris_hip_split_rows(sB, dB, N, K, K, Kp, 3, 2) : iris_hip_split_transpose(sB, dB, K, N, Kp, 3, 2)) {
        fail(name, C, MN);
        return;
    }
    if (gemm_split(dC, sA, sB, dbias, M, N, Kp, 3) || down(C, dC, MN)) fail(name, C, MN);
}

void iris_matmul(float *C, const float *A, const float *B, int M, int K, int N) {
    matmul_any("iris_matmul", C, A, B, NULL, M, K, N, 0);
}
void iris_matmul_t(float *C, const float *A, const float *B, int M, int K, int N) {
    matmul_any("iris_matmul_t", C, A, B, NULL, M, K, N, 1);
}
void iris_linear(float *y, const float *x, const float *W, const float *b, int seq_len, int in_dim, int out_dim) {
    matmul_any("iris_linear", y, x, W, b, seq_len, in_dim, out_dim, 1);
}
void iris_linear_nobias(float *y, const float *x, const float *W, int seq_len, int in_dim, int out_dim) {
    matmul_any("iris_linear_nobias", y, x, W, NULL, seq_len, in_dim, out_dim, 1);
}

void iris_linear_nobias_bf16(float *y, const float *x, const uint16_t *W_bf16, int seq_len, int in_dim,
                             int out_dim) {
    const int M = seq_len, K = in_dim, N = out_dim;
    if (M <= 0 || N <= 0) return;
    const size_t MN = (size_t)M * N;
    if (K <= 0) {
        float *dC = (float *)slot(SLOT_C, MN * sizeof(float));
        if (!dC || iris_hip_memset(dC, 0, MN * sizeof(float)) || down(y, dC, MN)) fail("iris_linear_nobias_bf16", y, MN);
        return;
    }
    const int Kp = pad64(K);
    float *dx = up(SLOT_A, x, (size_t)M * K);
    uint16_t *dW = (uint16_t *)slot(SLOT_B, (size_t)N * K * 2);
    uint16_t *sA = (uint16_t *)slot(SLOT_SA, (size_t)M * 2 * Kp * 2);
    uint16_t *sB = (uint16_t *)slot(SLOT_SB, (size_t)N * 2 * Kp * 2);
    float *dC = (float *)slot(SLOT_C, MN * sizeof(float));
    if (!dx || !dW || !sA || !sB || !dC || iris_hip_memcpy_h2d(dW, W_bf16, (size_t)N * K * 2) ||
        iris_hip_split_rows(sA, dx, M, K, K, Kp, 2, 2) || iris_hip_pad_bf16(sB, dW, N, K, Kp, 2) ||
        gemm_split(dC, sA, sB, NULL, M, N, Kp, 2) || down(y, dC, MN))
        fail("iris_linear_nobias_bf16", y, MN);
}

/* ---- convolution: per image, out[oc][pix] = W[oc][K] . im2col[pix][K]^T,
 *      with the pixel range cut into chunks that bound the im2col buffer ---- */
void iris_conv2d(float *out, const float *in, const float *weight, const float *bias, int batch, int in_ch,
                 int out_ch, int H, int W, int kH, int kW, int stride, int padding) {
    if (stride <= 0 || kH <= 0 || kW <= 0 || in_ch <= 0 || padding < 0) {
        fprintf(stderr, "iris_kernels (HIP): iris_conv2d: invalid geometry (in_ch %d, kernel %dx%d, stride %d, "
                        "padding %d)\n", in_ch, kH, kW, stride, padding);
        return;
    }
    const int oH = (H + 2 * padding - kH) / stride + 1, oW = (W + 2 * padding - kW) / stride + 1;
    if (batch <= 0 || out_ch <= 0 || oH <= 0 || oW <= 0) return;
    const int npix = oH * oW, K = in_ch * kH * kW, Kp = pad64(K);
    const size_t out_n = (size_t)batch * out_ch * npix, in_n = (size_t)batch * in_ch * H * W;
    float *din = up(SLOT_A, in, in_n);
    float *dw = up(SLOT_B, weight, (size_t)out_ch * K);
    float *dbias = bias ? up(SLOT_D, bias, (size_t)out_ch) : NULL;
    float *dout = (float *)slot(SLOT_C, out_n * sizeof(float));
    uint16_t *sW = (uint16_t *)slot(SLOT_SA, (size_t)out_ch * 3 * Kp * 2);
    /* about 256 MB of im2col per chunk, a multiple of 256 pixels */
    size_t chunk = ((size_t)256 << 20) / ((size_t)3 * Kp * 2);
    chunk = chunk < 256 ? 256 : chunk / 256 * 256;
    if (chunk > (size_t)npix) chunk = (size_t)npix;
    uint16_t *sI = (uint16_t *)slot(SLOT_SB, chunk * 3 * Kp * 2);
    if (!din || !dw || (bias && !dbias) || !dout || !sW || !sI ||
        iris_hip_split_rows(sW, dw, out_ch, K, K, Kp, 3, 4)) {
        fail("iris_conv2d", out, out_n);
        return;
    }
    for (int b = 0; b < batch; b++) {
        const float *img = din + (size_t)b * in_ch * H * W;
        float *o = dout + (size_t)b * out_ch * npix;
        for (int p0 = 0; p0 < npix; p0 += (int)chunk) {
            const int np = npix - p0 < (int)chunk ? npix - p0 : (int)chunk;
            iris_gemm_problem_t p;
            memset(&p, 0, sizeof p);
            p.A = sW;
            p.W = sI;
            p.out = o + p0;
            p.M = out_ch;
            p.N = np;
            p.K = 3 * Kp;
            p.lda = p.ldw = 3 * Kp;
            p.ldo = npix;
            p.epi = IRIS_EPI_F32;
            if (iris_hip_im2col_split(sI, img, in_ch, H, W, kH, kW, stride, padding, oW, p0, np, Kp, 3, 2) ||
                iris_hip_gemm(&p, 1)) {
                fail("iris_conv2d", out, out_n);
                return;
            }
        }
        if (dbias && iris_hip_add_row_bias(o, dbias, out_ch, npix, npix)) {
            fail("iris_conv2d", out, out_n);
            return;
        }
    }
    if (down(out, dout, out_n)) fail("iris_conv2d", out, out_n);
}

/* ---- normalisation ---- */
void iris_rms_norm(float *out, const float *x, const float *weight, int seq_len, int hidden, float eps) {
    if (seq_len <= 0 || hidden <= 0) return;
    const size_t n = (size_t)seq_len * hidden;
    float *dx = up(SLOT_A, x, n), *dw = up(SLOT_B, weight, (size_t)hidden);
    if (!dx || !dw || iris_hip_rms_rows(dx, dx, dw, seq_len, hidden, eps) || down(out, dx, n))
        fail("iris_rms_norm", out, n);
}

void iris_group_norm(float *out, const float *x, const float *gamma, const float *beta, int batch, int channels,
                     int H, int W, int num_groups, float eps) {
    if (batch <= 0 || channels <= 0 || H <= 0 || W <= 0) return;
    const size_t n = (size_t)batch * channels * H * W;
    float *dx = up(SLOT_A, x, n), *dg = up(SLOT_B, gamma, (size_t)channels), *db = up(SLOT_D, beta, (size_t)channels);
    float *dout = (float *)slot(SLOT_C, n * sizeof(float));
    if (!dx || !dg || !db || !dout ||
        iris_hip_group_norm(dout, dx, dg, db, batch, channels, H * W, num_groups, eps) || down(out, dout, n))
        fail("iris_group_norm", out, n);
}

void iris_batch_norm(float *out, const float *x, const float *running_mean, const float *running_var,
                     const float *gamma, const float *beta, int batch, int channels, int H, int W, float eps) {
    if (batch <= 0 || channels <= 0 || H <= 0 || W <= 0) return;
    const size_t n = (size_t)batch * channels * H * W;
    float *dx = up(SLOT_A, x, n);
    /* the four per-channel vectors share one slot */
    float *dv = (float *)slot(SLOT_B, (size_t)4 * channels * sizeof(float));
    if (!dx || !dv) { fail("iris_batch_norm", out, n); return; }
    float *dm = dv, *dvar = dv + channels, *dg = gamma ? dv + 2 * channels : NULL, *db = beta ? dv + 3 * channels : NULL;
    const size_t cb = (size_t)channels * sizeof(float);
    if (iris_hip_memcpy_h2d(dm, running_mean, cb) || iris_hip_memcpy_h2d(dvar, running_var, cb) ||
        (dg && iris_hip_memcpy_h2d(dg, gamma, cb)) || (db && iris_hip_memcpy_h2d(db, beta, cb)) ||
        iris_hip_batch_norm(dx, dx, dm, dvar, dg, db, batch, channels, H * W, eps) || down(out, dx, n))
        fail("iris_batch_norm", out, n);
}

/* ---- softmax ---- */
static void softmax_rows(const char *name, float *x, int rows, int cols) {
    if (rows <= 0 || cols <= 0) return;
    const size_t n = (size_t)rows * cols;
    float *dx = up(SLOT_A, x, n);
    if (!dx || iris_hip_softmax_rows(dx, rows, cols) || down(x, dx, n)) fail(name, x, n);
}
void iris_softmax(float *x, int rows, int cols) { softmax_rows("iris_softmax", x, rows, cols); }
void iris_softmax_cpu(float *x, int rows, int cols) { softmax_rows("iris_softmax_cpu", x, rows, cols); }

/* ---- attention ---- */
void iris_attention(float *out, const float *Q, const float *K, const float *V, int batch, int heads, int seq_q,
                    int seq_k, int head_dim, float scale) {
    if (batch <= 0 || heads <= 0 || seq_q <= 0 || seq_k <= 0 || head_dim <= 0) return;
    const size_t nq = (size_t)batch * heads * seq_q * head_dim, nk = (size_t)batch * heads * seq_k * head_dim;
    float *dq = up(SLOT_A, Q, nq), *dk = up(SLOT_B, K, nk), *dv = up(SLOT_D, V, nk);
    float *dout = (float *)slot(SLOT_C, nq * sizeof(float));
    const long long q_sh = (long long)seq_q * head_dim, k_sh = (long long)seq_k * head_dim;
    if (!dq || !dk || !dv || !dout ||
        iris_hip_attention_f32(dout, dq, dk, dv, batch, heads, seq_q, seq_k, head_dim, scale, q_sh * heads, q_sh,
                               k_sh * heads, k_sh, head_dim) ||
        down(out, dout, nq))
        fail("iris_attention", out, nq);
}

void iris_flash_attention(float *out, const float *Q, const float *K, const float *V, int seq_q, int seq_k,
                          int heads, int head_dim, float scale) {
    if (heads <= 0 || seq_q <= 0 || seq_k <= 0 || head_dim <= 0) return;
    const size_t nq = (size_t)seq_q * heads * head_dim, nk = (size_t)seq_k * heads * head_dim;
    float *dq = up(SLOT_A, Q, nq), *dk = up(SLOT_B, K, nk), *dv = up(SLOT_D, V, nk);
    float *dout = (float *)slot(SLOT_C, nq * sizeof(float));
    if (!dq || !dk || !dv || !dout ||
        iris_hip_attention_f32(dout, dq, dk, dv, 1, heads, seq_q, seq_k, head_dim, scale, 0, head_dim, 0, head_dim,
                               heads * head_dim) ||
        down(out, dout, nq))
        fail("iris_flash_attention", out, nq);
}

/* ---- reshapes ---- */
void iris_upsample_nearest(float *out, const float *in, int batch, int channels, int H, int W, int scale_h,
                           int scale_w) {
    if (batch <= 0 || channels <= 0 || H <= 0 || W <= 0 || scale_h <= 0 || scale_w <= 0) return;
    const size_t nin = (size_t)batch * channels * H * W, nout = nin * scale_h * scale_w;
    float *din = up(SLOT_A, in, nin);
    float *dout = (float *)slot(SLOT_C, nout * sizeof(float));
    if (!din || !dout || iris_hip_upsample_nearest(dout, din, batch * channels, H, W, scale_h, scale_w) ||
        down(out, dout, nout))
        fail("iris_upsample_nearest", out, nout);
}

void iris_patchify(float *out, const float *in, int batch, int channels, int H, int W, int patch_size) {
    if (batch <= 0 || channels <= 0 || H <= 0 || W <= 0) return;
    const size_t n = (size_t)batch * channels * H * W;
    float *din = up(SLOT_A, in, n);
    float *dout = (float *)slot(SLOT_C, n * sizeof(float));
    if (!din || !dout || iris_hip_space_to_depth(dout, din, batch, channels, H, W, patch_size, 0) ||
        down(out, dout, n))
        fail("iris_patchify", out, n);
}

void iris_unpatchify(float *out, const float *in, int batch, int channels, int H, int W, int patch_size) {
    const int p = patch_size;
    if (p <= 0 || batch <= 0 || channels <= 0 || H <= 0 || W <= 0) return;
    const size_t n = (size_t)batch * channels * p * p * H * W;
    if (!n) return;
    float *din = up(SLOT_A, in, n);
    float *dout = (float *)slot(SLOT_C, n * sizeof(float));
    if (!din || !dout || iris_hip_space_to_depth(dout, din, batch, channels, H * p, W * p, p, 1) ||
        down(out, dout, n))
        fail("iris_unpatchify", out, n);
}

/* ---- batching: no-ops (each call is complete when it returns) ---- */
void iris_gpu_begin_batch(void) {}
void iris_gpu_end_batch(void) {}

/* ---- random fills from the shared xoshiro256** stream (iris_kernels.c:98-107) ---- */
void iris_randn(float *out, int n) {
    for (int i = 0; i < n; i++) out[i] = iris_random_normal();
}
void iris_rand(float *out, int n) {
    for (int i = 0; i < n; i++) out[i] = iris_random_uniform();
}
