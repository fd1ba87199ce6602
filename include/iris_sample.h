/*
 * iris_sample.h - schedules, seeded noise and Euler samplers of the HIP build.
 *
 * Same names, arguments and results as the reference's iris_sample.c
 * (schedules :61-244, samplers :313-989, noise :1146-1188) and RNG
 * (iris_kernels.c:50-107). The samplers keep the latent on the device for the
 * whole loop and return a malloc'd host copy of the final latent (the caller
 * frees it), NULL on error or when iris_cancel_requested is set.
 */
#ifndef IRIS_SAMPLE_H
#define IRIS_SAMPLE_H

#include <stdint.h>
#include "iris_transformer.h"

#ifdef __cplusplus
extern "C" {
#endif

#define IRIS_MAX_STEPS 256

extern volatile int iris_cancel_requested;

/* Schedules of num_steps + 1 values from 1 to 0 (iris_sample.c:61-244), with
 * the bits of the reference's -O3 -march=native -ffast-math build on the same
 * host (its vectorized lanes use the CPU's reciprocal estimate). */
float *iris_linear_schedule(int num_steps);                       /* :61-68 */
float *iris_power_schedule(int num_steps, float alpha);           /* :75-84 */
float *iris_sigmoid_schedule(int num_steps, float shift);         /* :90-107 */
float *iris_resolution_schedule(int num_steps, int height, int width);   /* :113-136 */
float *iris_official_schedule(int num_steps, int image_seq_len);  /* :160-182 */
float *iris_zimage_schedule(int num_steps, int image_seq_len);    /* :216-244; shift 3 or IRIS_ZIMAGE_SHIFT */
float *iris_init_noise(int batch, int channels, int h, int w, int64_t seed);
void iris_rng_seed(uint64_t seed);
float iris_random_uniform(void);
float iris_random_normal(void);

float *iris_sample_euler(void *transformer, void *text_encoder, float *z, int batch, int channels, int h, int w,
                         const float *text_emb, int text_seq, const float *schedule, int num_steps,
                         void (*progress_callback)(int step, int total));
float *iris_sample_euler_with_multi_refs(void *transformer, void *text_encoder, float *z, int batch, int channels,
                                         int h, int w, const iris_ref_t *refs, int num_refs, const float *text_emb,
                                         int text_seq, const float *schedule, int num_steps,
                                         void (*progress_callback)(int step, int total));
/* classifier-free guidance; both branches run as one batch-2 pass when the
 * text lengths match, else as two sequential passes (iris_sample.c:717-802) */
float *iris_sample_euler_cfg(void *transformer, void *text_encoder, float *z, int batch, int channels, int h,
                             int w, const float *text_emb_cond, int text_seq_cond, const float *text_emb_uncond,
                             int text_seq_uncond, float guidance_scale, const float *schedule, int num_steps,
                             void (*progress_callback)(int step, int total));
/* one reference image at RoPE T coordinate t_offset (iris_sample.c:543-625) */
float *iris_sample_euler_with_refs(void *transformer, void *text_encoder, float *z, int batch, int channels, int h,
                                   int w, const float *ref_latent, int ref_h, int ref_w, int t_offset,
                                   const float *text_emb, int text_seq, const float *schedule, int num_steps,
                                   void (*progress_callback)(int step, int total));
/* CFG with reference images (iris_sample.c:807-989): the reference tokens join
 * both branches; one batch-2 pass when the text lengths match, else two
 * sequential passes; a CSD style delta acts on both branches, as in the
 * reference */
float *iris_sample_euler_cfg_with_refs(void *transformer, void *text_encoder, float *z, int batch, int channels, int h,
                                       int w, const float *ref_latent, int ref_h, int ref_w, int t_offset,
                                       const float *text_emb_cond, int text_seq_cond, const float *text_emb_uncond,
                                       int text_seq_uncond, float guidance_scale, const float *schedule,
                                       int num_steps, void (*progress_callback)(int step, int total));
float *iris_sample_euler_cfg_with_multi_refs(void *transformer, void *text_encoder, float *z, int batch, int channels,
                                             int h, int w, const iris_ref_t *refs, int num_refs,
                                             const float *text_emb_cond, int text_seq_cond,
                                             const float *text_emb_uncond, int text_seq_uncond, float guidance_scale,
                                             const float *schedule, int num_steps,
                                             void (*progress_callback)(int step, int total));
float *iris_sample_euler_zimage(void *transformer, float *z, int batch, int channels, int h, int w, int patch_size,
                                const float *cap_feats, int cap_seq, const float *schedule, int num_steps,
                                void (*progress_callback)(int step, int total));
/* Euler with noise injection (iris_sample.c:990-1062): after every step but
 * the last, eta * sqrt|dt| times normals from the global generator
 * (iris_rng_seed / iris_randn, drawn in the reference's order) are added to
 * the latent; eta <= 0 is the plain Euler sampler. */
float *iris_sample_euler_ancestral(void *transformer, float *z, int batch, int channels, int h, int w,
                                   const float *text_emb, int text_seq, const float *schedule, int num_steps,
                                   float eta, void (*progress_callback)(int step, int total));
/* Heun's second-order method (iris_sample.c:1063-1145): z_pred = z + dt v(z, t),
 * then z += dt / 2 (v(z, t) + v(z_pred, t_next)); the last step is plain
 * Euler. Two forwards per step. */
float *iris_sample_heun(void *transformer, float *z, int batch, int channels, int h, int w, const float *text_emb,
                        int text_seq, const float *schedule, int num_steps,
                        void (*progress_callback)(int step, int total));

#ifdef __cplusplus
}
#endif
#endif
