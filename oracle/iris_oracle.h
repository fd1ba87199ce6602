/*
 * iris_oracle.h - CPU f32 restatement of the reference denoiser forward.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity oracle and the CPU
 * baseline: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it. The product (iris.c_amd/) never links or calls it.
 *
 * It restates the reference's `make blas` path (all weights widened bf16->f32,
 * linears through cblas_sgemm, per-head sgemm/softmax/sgemm attention) with the
 * same operation order. Each function cites the reference file:line it follows.
 * sgemm is OpenBLAS when orc_set_blas() bound one, else a plain loop nest.
 *
 * How each part is pinned (tests/test_oracle.py, fixtures in tests/golden/
 * written by the reference compiled from its own sources, oracle/Makefile ref):
 *   RoPE tables (Flux img/txt/T-offsets, Z-Image axes), timestep sinusoid,
 *   patchify, noise                     bit-exact (SHA-256) vs the reference;
 *   fast_expf                           reference grid, rel 1e-5, plus the
 *                                       closed-form bound |e/exp - 1| < 1e-5;
 *   schedules                           the reference's own golden arrays
 *                                       (debug/test_zimage_scheduler.c:71-79)
 *                                       and reference outputs, rel 5e-6;
 *   Flux t-embed, modulation, double and single block, forward, multi-ref
 *   forward, 2-step sampler, 4B-shaped single block
 *                                       reference outputs, rel-L2 1e-5..1e-4;
 *   Z-Image t-embed, blocks, forward    reference outputs with the in-place
 *                                       output projection emulated (alias 1),
 *                                       rel-L2 1e-5..1e-4;
 *   Z-Image out-of-place forward (alias 0)
 *                                       reference outputs on upper-triangular
 *                                       output projections, where in-place and
 *                                       out-of-place coincide, rel-L2 1e-4;
 *   softmax, RMSNorm, LayerNorm, SiLU   textbook known answers.
 * Nothing on the path is "parity unpinned"; whether the reference C matches
 * the upstream Python models is outside this oracle (the reference's own
 * parity tests for that are skipped scaffolds).
 */
#ifndef IRIS_ORACLE_H
#define IRIS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

typedef struct orc_flux orc_flux_t;
typedef struct orc_zi orc_zi_t;
typedef struct orc_qwen3 orc_qwen3_t;
typedef struct orc_vae orc_vae_t;

typedef struct {
    const float *latent;
    int h, w;
    int t_offset;
} orc_ref_t;

/* BLAS binding: path of a shared library exporting <prefix>cblas_sgemm. */
int orc_set_blas(const char *so_path, const char *prefix, int threads);
const char *orc_blas_info(void);

/* fast_expf of iris_kernels.h:21-35 */
float orc_fast_expf(float x);

/* --- Flux.2-Klein --- */
orc_flux_t *orc_flux_load(const char *model_dir);
orc_flux_t *orc_flux_create_synth(int hidden, int heads, int n_double, int n_single,
                                  int text_dim, int latent_ch, float mlp_ratio,
                                  float rope_theta, uint64_t seed);
void orc_flux_free(orc_flux_t *m);
int orc_flux_dims(const orc_flux_t *m, int *out8);

float *orc_flux_forward(orc_flux_t *m, const float *latent, int h, int w,
                        const float *txt, int txt_seq, float t);
float *orc_flux_forward_refs(orc_flux_t *m, const float *latent, int h, int w,
                             const orc_ref_t *refs, int n_refs,
                             const float *txt, int txt_seq, float t);
void orc_free(void *p);

/* Pieces, for block- and table-level parity. */
void orc_rope_img(float *cos_out, float *sin_out, int ph, int pw, int axis_dim,
                  float theta, int t_offset);
void orc_rope_txt(float *cos_out, float *sin_out, int txt_seq, int axis_dim, float theta);
void orc_timestep_sincos(float *out, float t, int dim, float max_period);
void orc_flux_time_embed(orc_flux_t *m, float t, float *t_emb);
/* mod outputs: dimg[6h], dtxt[6h], single[3h], final[2h] (any may be NULL) */
void orc_flux_modulation(orc_flux_t *m, const float *t_emb, float *dimg, float *dtxt,
                         float *single, float *final_mod);
void orc_flux_double_block(orc_flux_t *m, int idx, float *img, float *txt,
                           const float *img_mod, const float *txt_mod,
                           const float *img_cos, const float *img_sin,
                           const float *txt_cos, const float *txt_sin,
                           int img_seq, int txt_seq);
void orc_flux_single_block(orc_flux_t *m, int idx, float *x, const float *t_emb,
                           const float *img_cos, const float *img_sin,
                           const float *txt_cos, const float *txt_sin,
                           int seq, int img_offset);
void orc_flux_single_block_k(orc_flux_t *m, int idx, float *x, const float *t_emb,
                             const float *img_cos, const float *img_sin,
                             const float *kimg_cos, const float *kimg_sin,
                             const float *txt_cos, const float *txt_sin,
                             int seq, int img_offset);
/* SREF band control (reference rows' K-side RoPE bands, single blocks only) */
void orc_flux_set_sref_bands(orc_flux_t *m, float shf, float slf);
void orc_sref_band_scale(float *c, float *s, int ref_start, int rows, int axis_dim, float shf, float slf);

/* --- Z-Image S3-DiT --- */
orc_zi_t *orc_zi_load(const char *model_dir, int dim, int heads, int layers, int refiners,
                      int cap_dim, int in_ch, int ps, float theta, const int *axes);
orc_zi_t *orc_zi_create_synth(int dim, int heads, int layers, int refiners, int cap_dim,
                              int in_ch, int ps, float theta, const int *axes, int ffn_dim,
                              int t_mid, uint64_t seed);
void orc_zi_free(orc_zi_t *m);
/* 1: reproduce the reference CPU path's in-place attention output projection. */
void orc_zi_set_reference_aliasing(int on);
float *orc_zi_forward(orc_zi_t *m, const float *latent, int lh, int lw, float t,
                      const float *cap, int cap_len);
void orc_zi_rope_tables(orc_zi_t *m, float *cos_out, float *sin_out, int axis);
void orc_zi_patchify(float *out, const float *latent, int in_ch, int H, int W, int ps);
void orc_zi_t_embed(orc_zi_t *m, float t, float *out);
void orc_zi_block(orc_zi_t *m, int kind, int idx, float *x, const int *pos, const int *mask,
                  const float *t_emb, int seq);

/* --- sampler pieces --- */
float *orc_official_schedule(int n, int image_seq_len);
float *orc_zimage_schedule(int n, float shift);
float *orc_init_noise(int batch, int ch, int h, int w, int64_t seed);

/* Qwen3 text encoder (orc_qwen3.c, iris_qwen3.c): config.json + safetensors
 * directory, or the seeded synthetic weights of iris_synth.h. mode 0 = Flux
 * (layers 8, 17, 26 concatenated), 1 = Z-Image (layer num_layers-2).
 * forward: malloc'd [seq][text_dim]; with last_limit >= 0 below the mode's
 * last layer it stops after that layer and returns the hidden state [seq][h]. */
orc_qwen3_t *orc_qwen3_load(const char *dir);
orc_qwen3_t *orc_qwen3_create_synth(int hidden, int inter, int heads, int kv_heads, int layers, int vocab,
                                    uint64_t seed);
void orc_qwen3_free(orc_qwen3_t *m);
void orc_qwen3_set_mode(orc_qwen3_t *m, int mode);
int orc_qwen3_dims(const orc_qwen3_t *m, int *out4);   /* hidden, layers, text_dim, head_dim */
float *orc_qwen3_forward(orc_qwen3_t *m, const int *ids, const int *mask, int seq, int last_limit);

/* VAE decoder (orc_vae.c, iris_vae.c): weights from a diffusers-layout
 * safetensors file or synthetic (iris_synth_vae_stats); z_channels 32 or 16,
 * scaling 0 = batch-norm denormalization. decode writes rgb [16lh][16lw][3]
 * and the pre-quantization f32 [3][16lh][16lw]; stop_after >= 0 returns the
 * channel count of the activation after that many stages, copied to f32. */
orc_vae_t *orc_vae_load(const char *path, int z, float scaling, float shift);
orc_vae_t *orc_vae_create_synth(int z, float scaling, float shift, uint64_t seed);
void orc_vae_free(orc_vae_t *v);
int orc_vae_decode(orc_vae_t *v, const float *latent, int lh, int lw, uint8_t *rgb, float *f32, int stop_after);
/* iris_vae_encode for one image [3][H][W] -> latent [4z][H/16][W/16]; -1 without encoder weights */
int orc_vae_encode(orc_vae_t *v, const float *img, int H, int W, float *latent);

#endif
