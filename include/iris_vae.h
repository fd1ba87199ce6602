/*
 * iris_vae.h - the VAE on the GPU: latent -> RGB image, image -> latent.
 *
 * Replaces the reference's decoder path, iris_vae.c:835-998 (iris_vae_decode),
 * and encoder path, iris_vae.c:363-482 (iris_vae_encode), with the weights of
 * iris_vae_load_safetensors_ex (iris_vae.c:1227-1386).
 * Architecture fixed as in the reference: base 128 channels, ch_mult
 * {1, 2, 4, 4}, 2 + 1 resblocks per up level, 32 groups, a single-head
 * attention block at the bottleneck, nearest 2x upsampling; z_channels 32
 * (Flux.2, batch-norm denormalization + post_quant_conv) or 16 (Z-Image,
 * x / scaling + shift). Weights are uploaded once as bf16 (convolutions) and
 * f32 (norms, biases); activations stay on the device, channels-last.
 */
#ifndef IRIS_VAE_H
#define IRIS_VAE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IRIS_VAE_MAX_DIM 1792   /* largest image side, as the reference (iris.h:52) */

/* Same layout as the reference's iris_image (iris.h:73-78). */
typedef struct iris_image {
    int width;
    int height;
    int channels;
    uint8_t *data;   /* row-major, channel-interleaved RGB */
} iris_image;

typedef struct iris_vae_gpu iris_vae_gpu_t;

/* cf. iris_vae_load_safetensors_ex (iris_vae.c:1227): path of
 * vae/diffusion_pytorch_model.safetensors (f32, bf16 or f16 tensors),
 * z_channels 32 (Flux) or 16 (Z-Image), scaling_factor 0 selects the Flux
 * batch-norm denormalization (bn.running_mean / running_var, identity when
 * absent), otherwise latent / scaling_factor + shift_factor. eps is 1e-4 for
 * Flux and 1e-6 for Z-Image, as the reference. NULL on error
 * (iris_hip_last_error). */
iris_vae_gpu_t *iris_vae_gpu_load(const char *path, int z_channels, float scaling_factor, float shift_factor);
/* cf. iris.c:332-392: reads <model_dir>/vae/config.json (latent_channels,
 * scaling_factor, shift_factor, iris_vae_config.h) and loads
 * <model_dir>/vae/diffusion_pytorch_model.safetensors. */
iris_vae_gpu_t *iris_vae_gpu_load_dir(const char *model_dir);
/* No counterpart in the reference: random-init weights of the same
 * architecture (iris_synth.h, iris_synth_vae_stats), for benchmarks. */
iris_vae_gpu_t *iris_vae_gpu_create_synthetic(int z_channels, float scaling_factor, float shift_factor,
                                              uint64_t seed);
void iris_vae_gpu_free(iris_vae_gpu_t *vae);

/* cf. iris_vae_decode (iris_vae.c:835): latent [batch][4 z][latent_h][latent_w]
 * f32 (host); returns the image of batch item 0, (16 latent_w) x
 * (16 latent_h) RGB, as the reference does; free with iris_image_free. */
iris_image *iris_vae_gpu_decode(iris_vae_gpu_t *vae, const float *latent, int batch, int latent_h, int latent_w);
void iris_image_free(iris_image *img);

/* Host buffers: rgb [16h][16w][3] uint8; f32 (or NULL) receives the
 * pre-quantization output [3][16h][16w]. Returns 0 on success. */
int iris_vae_gpu_decode_to(iris_vae_gpu_t *vae, const float *latent, int latent_h, int latent_w, uint8_t *rgb,
                           float *f32);
/* Device-resident: d_latent, d_rgb, d_f32 (or NULL) in device memory; the
 * work is queued on the library stream (iris_hip_sync to wait). Buffers grow
 * on the first call at a larger size, so a graph capture must follow one
 * uncaptured call at the same size. */
int iris_vae_gpu_decode_device(iris_vae_gpu_t *vae, const float *d_latent, int latent_h, int latent_w,
                               uint8_t *d_rgb, float *d_f32);
int iris_vae_gpu_z_channels(const iris_vae_gpu_t *vae);

/* cf. iris_vae_encode (iris_vae.c:363-482): images [batch][3][H][W] f32 in
 * [-1, 1] (host), H and W multiples of 16 up to IRIS_VAE_MAX_DIM; returns
 * malloc'd latents [batch][4z][H/16][W/16] (mean of the posterior, patchified
 * and normalized) and their size in out_h, out_w; NULL on error or when the
 * file had no encoder tensors. */
float *iris_vae_gpu_encode(iris_vae_gpu_t *vae, const float *img, int batch, int H, int W, int *out_h, int *out_w);
/* Device-resident encode of one image: d_img [3][H][W] -> d_latent. */
int iris_vae_gpu_encode_device(iris_vae_gpu_t *vae, const float *d_img, int H, int W, float *d_latent);
int iris_vae_gpu_has_encoder(const iris_vae_gpu_t *vae);

#ifdef __cplusplus
}
#endif
#endif
