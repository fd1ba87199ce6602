/*
 * iris_kernels.h - the reference's host-pointer math API, served by the HIP
 * build (iris.c_amd/host/iris_kernels_hip.c).
 *
 * Same names, argument order and meaning as the reference's iris_kernels.h
 * (:21-35 fast_expf, :42-312 the API), so that its callers (the VAE, the text
 * encoder, the samplers, iris.c) link against this library unchanged. Tensors
 * are f32, row-major, caller-owned host arrays. Every compute entry stages its
 * operands into HBM, runs on the GPU and copies the result back before it
 * returns; there is no CPU path behind these names. Products that the
 * reference hands to cblas_sgemm (iris_kernels.c:146-336) are computed with
 * split-bf16 MFMA GEMMs whose error stays near 1e-5 relative to f32.
 *
 * Errors (no GPU, device out of memory, unsupported size) are reported on
 * stderr, recorded in iris_hip_last_error(), and leave the output zeroed, the
 * way the reference's out-of-memory paths do (iris_kernels.c:690-698).
 */
#ifndef IRIS_KERNELS_H
#define IRIS_KERNELS_H

#include <math.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

struct iris_image;

/* e^x by range reduction x = n ln2 + r, |r| <= ln2/2, a degree-5 Taylor
 * polynomial in r, and 2^n put into the exponent field. Outside
 * [-87.3, 88.7] it returns 0 or 1e38. Same operations as the reference's
 * inline (iris_kernels.h:21-35), so callers that use it keep bit-identical
 * results. Relative error: about 3.3e-6 near 0 (the r^6/720 truncation term)
 * rising to 7.3e-6 at |x| ~ 80 (rounding of n * ln2 in f32), not the 2e-6 the
 * reference's comment states. */
static inline float fast_expf(float x) {
    if (x < -87.3f) return 0.0f;
    if (x > 88.7f) return 1e38f;
    const float n = floorf(x * 1.4426950408889634f + 0.5f);
    const float r = x - n * 0.6931471805599453f;
    const float p = 1.0f + r * (1.0f + r * (0.5f + r * (0.16666667f + r * (0.04166667f + r * 0.00833333f))));
    union {
        float f;
        uint32_t u;
    } v;
    v.f = p;
    v.u += (uint32_t)(int32_t)n << 23;
    return v.f;
}

/* ---- elementwise (iris_kernels.h:42-50) ---- */
void iris_add(float *out, const float *a, const float *b, int n);
void iris_add_inplace(float *a, const float *b, int n);
void iris_mul_inplace(float *a, const float *b, int n);
void iris_axpy(float *a, float scale, const float *b, int n);   /* a += scale * b */

/* ---- products (iris_kernels.h:56-88) ---- */
void iris_matmul(float *C, const float *A, const float *B, int M, int K, int N);    /* A[M,K] B[K,N] */
void iris_matmul_t(float *C, const float *A, const float *B, int M, int K, int N);  /* A[M,K] B[N,K]^T */
void iris_linear(float *y, const float *x, const float *W, const float *b, int seq_len, int in_dim, int out_dim);
void iris_linear_nobias(float *y, const float *x, const float *W, int seq_len, int in_dim, int out_dim);
void iris_linear_nobias_bf16(float *y, const float *x, const uint16_t *W_bf16, int seq_len, int in_dim,
                             int out_dim);

/* ---- batching (iris_kernels.h:95-108): every call here already runs on one
 *      in-order stream and returns with its result, so these are no-ops ---- */
void iris_gpu_begin_batch(void);
void iris_gpu_end_batch(void);

/* ---- convolution, in [B, Cin, H, W], weight [Cout, Cin, kH, kW] (iris_kernels.h:121-123) ---- */
void iris_conv2d(float *out, const float *in, const float *weight, const float *bias, int batch, int in_ch,
                 int out_ch, int H, int W, int kH, int kW, int stride, int padding);

/* ---- normalisation (iris_kernels.h:133-149) ---- */
void iris_rms_norm(float *out, const float *x, const float *weight, int seq_len, int hidden, float eps);
void iris_group_norm(float *out, const float *x, const float *gamma, const float *beta, int batch, int channels,
                     int H, int W, int num_groups, float eps);
void iris_batch_norm(float *out, const float *x, const float *running_mean, const float *running_var,
                     const float *gamma, const float *beta, int batch, int channels, int H, int W, float eps);

/* ---- activations and softmax (iris_kernels.h:156-164) ---- */
void iris_silu(float *x, int n);
void iris_silu_mul(float *gate, const float *up, int n);   /* gate = silu(gate) * up */
void iris_softmax(float *x, int rows, int cols);
void iris_softmax_cpu(float *x, int rows, int cols);       /* same contract; named as in the reference */

/* ---- attention (iris_kernels.h:178-197) ---- */
/* Q [B, H, Sq, D], K/V [B, H, Sk, D], out [B, H, Sq, D]; D <= 512, Sk <= 12288 */
void iris_attention(float *out, const float *Q, const float *K, const float *V, int batch, int heads, int seq_q,
                    int seq_k, int head_dim, float scale);
/* Q [Sq, H*D], K/V [Sk, H*D], out [Sq, H*D] */
void iris_flash_attention(float *out, const float *Q, const float *K, const float *V, int seq_q, int seq_k,
                          int heads, int head_dim, float scale);

/* ---- reshapes (iris_kernels.h:204-215) ---- */
void iris_upsample_nearest(float *out, const float *in, int batch, int channels, int H, int W, int scale_h,
                           int scale_w);
void iris_patchify(float *out, const float *in, int batch, int channels, int H, int W, int patch_size);
void iris_unpatchify(float *out, const float *in, int batch, int channels, int H, int W, int patch_size);

/* ---- random numbers, xoshiro256** seeded by SplitMix64 (iris_kernels.h:222-235) ---- */
void iris_rng_seed(uint64_t seed);
float iris_random_uniform(void);
float iris_random_normal(void);
void iris_randn(float *out, int n);
void iris_rand(float *out, int n);

/* ---- utility (iris_kernels.h:242) ---- */
void iris_copy(float *dst, const float *src, int n);

/* ---- progress callbacks and flags (iris_kernels.h:248-312) ---- */
typedef enum {
    IRIS_SUBSTEP_DOUBLE_BLOCK,
    IRIS_SUBSTEP_SINGLE_BLOCK,
    IRIS_SUBSTEP_FINAL_LAYER,
} iris_substep_type_t;

typedef void (*iris_substep_callback_t)(iris_substep_type_t type, int index, int total);
typedef void (*iris_step_callback_t)(int step, int total);
typedef void (*iris_phase_callback_t)(const char *phase, int done);
typedef void (*iris_step_image_callback_t)(int step, int total, const struct iris_image *img);
typedef void (*iris_text_progress_callback_t)(int layer, int total);
typedef void (*iris_vae_progress_callback_t)(int block, int total);

/* Transformer substeps fire after the step's work has been enqueued, in
 * block order; the step callback fires at the start of each sampler step. */
extern iris_substep_callback_t iris_substep_callback;
extern iris_step_callback_t iris_step_callback;
extern iris_phase_callback_t iris_phase_callback;
extern volatile int iris_cancel_requested;
extern iris_step_image_callback_t iris_step_image_callback;
extern void *iris_step_image_vae;
extern iris_text_progress_callback_t iris_text_progress_callback;
extern iris_vae_progress_callback_t iris_vae_progress_callback;
extern int iris_verbose;

#ifdef __cplusplus
}
#endif
#endif /* IRIS_KERNELS_H */
