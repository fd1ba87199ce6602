/*
 * iris_transformer.h - denoiser entry points of the HIP build (`make hip`).
 *
 * The first group keeps the reference's C signatures, ownership and error
 * behaviour so a caller written against the reference links unchanged:
 *   - iris_transformer_load_safetensors[_mmap]   iris_transformer_flux.c:5300, :5550
 *   - iris_transformer_free / _free_mmap_cache   :5100-5160, :806-812
 *   - iris_transformer_forward                   :3939
 *   - iris_transformer_forward_with_refs         :4354
 *   - iris_transformer_forward_with_multi_refs   :4579 (iris_ref_t :4569-4573)
 *   - zi_transformer_load_safetensors / _forward / _free
 *                                                iris_transformer_zimage.c:2164, :1696
 * Forwards take caller-owned host f32 arrays and return a malloc'd host f32
 * array the caller frees with free(); NULL plus a message on stderr on error.
 * State is per transformer and per process; calls are not reentrant (one
 * caller thread), as in the reference.
 *
 * The second group has no counterpart in the reference. It keeps the latent,
 * text embedding and velocity resident in device memory across steps (the
 * reference re-uploads nothing because it never leaves the host), so a
 * sampler loop pays no PCIe traffic per step. iris_sample.h's samplers use it.
 */
#ifndef IRIS_TRANSFORMER_H
#define IRIS_TRANSFORMER_H

#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct iris_transformer iris_transformer_t;
typedef struct zi_transformer zi_transformer_t;

typedef struct {
    const float *latent;   /* NCHW [channels, h, w] */
    int h, w;
    int t_offset;          /* RoPE T coordinate */
} iris_ref_t;

/* ---- reference entry points (Flux.2-Klein) ---- */
iris_transformer_t *iris_transformer_load_safetensors(const char *model_dir);
iris_transformer_t *iris_transformer_load_safetensors_mmap(const char *model_dir);
void iris_transformer_free(iris_transformer_t *tf);
void iris_transformer_free_mmap_cache(iris_transformer_t *tf);
float *iris_transformer_forward(iris_transformer_t *tf, const float *img_latent, int img_h, int img_w,
                                const float *txt_emb, int txt_seq, float timestep);
float *iris_transformer_forward_with_refs(iris_transformer_t *tf, const float *img_latent, int img_h, int img_w,
                                          const float *ref_latent, int ref_h, int ref_w, int t_offset,
                                          const float *txt_emb, int txt_seq, float timestep);
float *iris_transformer_forward_with_multi_refs(iris_transformer_t *tf, const float *img_latent, int img_h,
                                                int img_w, const iris_ref_t *refs, int num_refs,
                                                const float *txt_emb, int txt_seq, float timestep);
int iris_transformer_hidden_size(iris_transformer_t *tf);
int iris_transformer_num_double_layers(iris_transformer_t *tf);
int iris_transformer_num_single_layers(iris_transformer_t *tf);
int iris_transformer_text_dim(iris_transformer_t *tf);

/* Adapter setters of the reference (iris_transformer_flux.c:5131-5201; LoRA
 * state and IP-Adapter passed as opaque pointers, same ABI). Ownership passes
 * to the transformer as in the reference. The HIP forward applies LoRA, the
 * CSD style delta and the SREF bands and strength; while an IP-Adapter is
 * attached every forward returns NULL with a message. */
void iris_transformer_set_lora(iris_transformer_t *tf, void *lora);
void iris_transformer_set_csd_delta(iris_transformer_t *tf, float *delta);
void iris_transformer_set_csd_skip(iris_transformer_t *tf, int skip);
/* No counterpart in the reference: whether a CSD style delta is attached (the
 * CFG sampler then runs the two branches as separate forwards so the delta
 * reaches the conditional one only, as the reference's style-CFG). */
int iris_transformer_csd_active(iris_transformer_t *tf);
void iris_transformer_set_sref_bands(iris_transformer_t *tf, float shf, float slf);
void iris_transformer_set_sref_strength(iris_transformer_t *tf, float gamma);
int iris_transformer_set_ip_adapter(iris_transformer_t *tf, void *ip, float *ip_embeds);
int iris_transformer_set_ip_schedule(iris_transformer_t *tf, const char *spec);
void iris_transformer_set_ip_step(iris_transformer_t *tf, int step, int num_steps);
/* legacy single-file loader (:4845): returns NULL (safetensors directories only) */
iris_transformer_t *iris_transformer_load(FILE *f);
/* BLAS profile counters of the CPU path (:55-80): no-ops here */
void iris_print_blas_profile(void);
void iris_reset_blas_profile(void);

/* ---- reference entry points (Z-Image) ---- */
zi_transformer_t *zi_transformer_load_safetensors(const char *model_dir, int dim, int n_heads, int n_layers,
                                                  int n_refiner, int cap_feat_dim, int in_channels,
                                                  int patch_size, float rope_theta, const int *axes_dims);
void zi_transformer_free(zi_transformer_t *tf);
float *zi_transformer_forward(zi_transformer_t *tf, const float *latent, int latent_h, int latent_w,
                              float timestep, const float *cap_feats, int cap_seq_len);

/* ---- random-init models (benchmarks, parity tests) ----
 * Same tensors, names and values a safetensors file written by the seeded
 * generator of iris_synth.h would hold (matrices N(0, 0.02), 1-D norm weights
 * 1 + N(0, 0.02), Z-Image biases N(0, 0.02), pad tokens N(0, 1), all bf16). */
iris_transformer_t *iris_transformer_create_synthetic(int hidden, int heads, int n_double, int n_single,
                                                      int text_dim, int latent_ch, float mlp_ratio,
                                                      float rope_theta, uint64_t seed);
zi_transformer_t *zi_transformer_create_synthetic(int dim, int n_heads, int n_layers, int n_refiner,
                                                  int cap_feat_dim, int in_channels, int patch_size,
                                                  float rope_theta, const int *axes_dims, int ffn_dim,
                                                  int t_mid, uint64_t seed);

/* ---- device-resident stepping (no reference counterpart) ----
 * batch > 1 runs independent sequences of identical geometry in one pass
 * (e.g. the conditional and unconditional branch of classifier-free
 * guidance); latents and texts are then stacked [batch][...]. */
int iris_flux_prepare(iris_transformer_t *tf, int img_h, int img_w, const iris_ref_t *refs, int num_refs,
                      int txt_seq, int batch);
int iris_flux_upload(iris_transformer_t *tf, const float *img_latent, const iris_ref_t *refs,
                     const float *txt_emb);
/* velocity of the resident latent at timestep t, left on the device */
int iris_flux_velocity(iris_transformer_t *tf, float t);
/* z += (t_next - t_curr) * v, where v is computed at t_curr (CFG when batch == 2:
 * v = v_uncond + g (v_cond - v_uncond) with batch slot 0 = uncond, 1 = cond) */
int iris_flux_step(iris_transformer_t *tf, float t_curr, float t_next, float guidance);
int iris_flux_download_latent(iris_transformer_t *tf, float *img_latent);
int iris_flux_download_velocity(iris_transformer_t *tf, float *velocity);
/* device pointers of the resident buffers (tests, benchmarks): "x" residual
 * [B][S][h] f32 in [txt | img | refs] row order, "mod" (double img 6h | double
 * txt 6h | single 3h | final 2h), "latent", "velocity", "tokens", "rope_cos",
 * "rope_sin", "t_emb", "txt", and the block scratch "a", "qkv", "q", "k", "vt", "cat" */
void *iris_flux_device_buffer(iris_transformer_t *tf, const char *name);
/* One block on the resident residual stream with the resident modulation and
 * RoPE tables; the reference's static block functions as entry points
 * (double_block_forward :2366-2614, single_block_forward :3761-3928). */
int iris_flux_double_block_forward(iris_transformer_t *tf, int idx);
int iris_flux_single_block_forward(iris_transformer_t *tf, int idx);

int zi_prepare(zi_transformer_t *tf, int latent_h, int latent_w, int cap_len);
int zi_upload(zi_transformer_t *tf, const float *latent, const float *cap_feats);
int zi_velocity(zi_transformer_t *tf, float timestep);
/* Z-Image update: z += (sigma_next - sigma) * (-v), v at timestep 1 - sigma */
int zi_step(zi_transformer_t *tf, float sigma, float sigma_next);
int zi_download_latent(zi_transformer_t *tf, float *latent);
/* Device buffers of the prepared geometry: "x" (unified [image (padded) |
 * caption (padded)] residual stream, f32 [U][dim]), "t_emb" (adaLN input,
 * [256]), "latent", "velocity", "rope_cos", "rope_sin", "patches", and the
 * block scratch "a", "qkv", "cat" */
void *zi_device_buffer(zi_transformer_t *tf, const char *name);
/* One block on the resident stream, the reference's zi_block_forward
 * (iris_transformer_zimage.c:790-870) as an entry point: kind 0 = noise
 * refiner idx on the image rows, 1 = context refiner idx on the caption rows,
 * 2 = main layer idx on the unified sequence, each with the forward's key
 * masks; the modulated kinds take their modulation from the resident t_emb. */
int zi_block_forward_resident(zi_transformer_t *tf, int kind, int idx);

#ifdef __cplusplus
}
#endif
#endif
