/*
 * iris_sample.c - seeded noise and Euler samplers (host C).
 *
 * Noise follows iris_sample.c:1146-1188 and the xoshiro256** RNG of
 * iris_kernels.c:50-107 (same seeds give the same noise); the schedules are
 * in iris_schedule.c.
 * The Euler loops (iris_sample.c:313-405, :412-536, :543-702, :717-989), the
 * ancestral Euler loop (:990-1062) and Heun's (:1063-1145) keep the latent
 * resident on the device: one upload, one graph replay and one update kernel
 * per forward, one download at the end.
 */
#include "../../include/iris_sample.h"
#include "../../include/iris_hip.h"
#include "../../include/iris_kernels.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

volatile int iris_cancel_requested = 0;

/* xoshiro256** seeded with SplitMix64; Box-Muller normals */
static uint64_t rng[4] = {0x853c49e6748fea9bULL, 0xda3e39cb94b95bdbULL, 0x647c4677a2884327ULL,
                          0xc6e7918d2e2969f5ULL};
static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
static uint64_t next64(void) {
    uint64_t r = rotl64(rng[1] * 5, 7) * 9, t = rng[1] << 17;
    rng[2] ^= rng[0]; rng[3] ^= rng[1]; rng[1] ^= rng[2]; rng[0] ^= rng[3];
    rng[2] ^= t; rng[3] = rotl64(rng[3], 45);
    return r;
}
void iris_rng_seed(uint64_t seed) {
    for (int i = 0; i < 4; i++) {
        seed += 0x9e3779b97f4a7c15ULL;
        uint64_t z = seed;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
        rng[i] = z ^ (z >> 31);
    }
}
float iris_random_uniform(void) { return (float)((next64() >> 11) * (1.0 / 9007199254740992.0)); }
float iris_random_normal(void) {
    float u1 = iris_random_uniform(), u2 = iris_random_uniform();
    while (u1 == 0.0f) u1 = iris_random_uniform();
    return sqrtf(-2.0f * logf(u1)) * cosf(2.0f * 3.14159265358979323846f * u2);
}

/* iris_init_noise: a 112x112 field subsampled for smaller latents so a seed
 * gives the same image at every size (:1146-1188) */
float *iris_init_noise(int batch, int ch, int h, int w, int64_t seed) {
    size_t n = (size_t)batch * ch * h * w;
    float *out = (float *)malloc(n * sizeof(float));
    if (!out) return NULL;
    if (seed >= 0) iris_rng_seed((uint64_t)seed);
    const int M = 112;
    if (h >= M && w >= M) {
        for (size_t i = 0; i < n; i++) out[i] = iris_random_normal();
        return out;
    }
    size_t mn = (size_t)batch * ch * M * M;
    float *mx = (float *)malloc(mn * sizeof(float));
    if (!mx) { free(out); return NULL; }
    for (size_t i = 0; i < mn; i++) mx[i] = iris_random_normal();
    for (int b = 0; b < batch; b++)
        for (int c = 0; c < ch; c++)
            for (int y = 0; y < h; y++)
                for (int x = 0; x < w; x++)
                    out[(((size_t)b * ch + c) * h + y) * w + x] =
                        mx[(((size_t)b * ch + c) * M + y * M / h) * M + x * M / w];
    free(mx);
    return out;
}

static float *flux_loop(iris_transformer_t *tf, const float *z, int channels, int h, int w, const iris_ref_t *refs,
                        int nrefs, const float *txt, int T, int B, float g, const float *sched, int n,
                        void (*cb)(int, int)) {
    if (n > IRIS_MAX_STEPS) {
        fprintf(stderr, "iris_sample: num_steps %d exceeds IRIS_MAX_STEPS %d\n", n, IRIS_MAX_STEPS);
        return NULL;
    }
    (void)channels;
    if (iris_flux_prepare(tf, h, w, refs, nrefs, T, B) || iris_flux_upload(tf, z, refs, txt)) return NULL;
    for (int i = 0; i < n; i++) {
        /* step callback, then the cancel check (iris_sample.c:345-348) */
        if (iris_step_callback) iris_step_callback(i + 1, n);
        if (iris_cancel_requested) return NULL;
        if (iris_flux_step(tf, sched[i], sched[i + 1], g)) return NULL;
        if (cb) cb(i + 1, n);
    }
    size_t sz = (size_t)channels * h * w;
    float *out = (float *)malloc(sz * sizeof(float));
    if (!out || iris_flux_download_latent(tf, out)) { free(out); return NULL; }
    return out;
}

float *iris_sample_euler(void *transformer, void *text_encoder, float *z, int batch, int channels, int h, int w,
                         const float *text_emb, int text_seq, const float *schedule, int num_steps,
                         void (*progress_callback)(int, int)) {
    (void)text_encoder; (void)batch;
    return flux_loop((iris_transformer_t *)transformer, z, channels, h, w, NULL, 0, text_emb, text_seq, 1, 0.0f,
                     schedule, num_steps, progress_callback);
}

float *iris_sample_euler_with_multi_refs(void *transformer, void *text_encoder, float *z, int batch, int channels,
                                         int h, int w, const iris_ref_t *refs, int num_refs, const float *text_emb,
                                         int text_seq, const float *schedule, int num_steps,
                                         void (*progress_callback)(int, int)) {
    (void)text_encoder; (void)batch;
    return flux_loop((iris_transformer_t *)transformer, z, channels, h, w, refs, num_refs, text_emb, text_seq, 1, 0.0f,
                     schedule, num_steps, progress_callback);
}

/* Two sequential forwards per step (v_u, then v_c) with the guided Euler
 * update on the device; style_cfg: the CSD style delta is suppressed on the
 * unconditional forward (the plain CFG sampler, iris_sample.c:750-760; the
 * reference-image CFG samplers :807-989 keep it on both). */
static float *cfg_two_pass(iris_transformer_t *tf, const float *z, int channels, int h, int w, const iris_ref_t *refs,
                           int nrefs, const float *tc, int Tc, const float *tu, int Tu, float g, const float *sched,
                           int num_steps, void (*cb)(int, int), int style_cfg) {
    if (num_steps > IRIS_MAX_STEPS) {
        fprintf(stderr, "iris_sample: num_steps %d exceeds IRIS_MAX_STEPS %d\n", num_steps, IRIS_MAX_STEPS);
        return NULL;
    }
    size_t n = (size_t)channels * h * w;
    float *zc = (float *)malloc(n * sizeof(float));
    float *dz = (float *)iris_hip_malloc(3 * n * sizeof(float));
    if (!zc || !dz) {
        free(zc);
        iris_hip_free(dz);
        return NULL;
    }
    float *dvu = dz + n, *dvc = dz + 2 * n;
    int ok = iris_hip_memcpy_h2d(dz, z, n * sizeof(float)) == 0;
    for (int i = 0; ok && i < num_steps; i++) {
        if (iris_step_callback) iris_step_callback(i + 1, num_steps);
        if (iris_cancel_requested || iris_hip_memcpy_d2h(zc, dz, n * sizeof(float))) { ok = 0; break; }
        if (style_cfg) iris_transformer_set_csd_skip(tf, 1);
        float *vu = iris_transformer_forward_with_multi_refs(tf, zc, h, w, refs, nrefs, tu, Tu, sched[i]);
        if (style_cfg) iris_transformer_set_csd_skip(tf, 0);
        float *vc = vu ? iris_transformer_forward_with_multi_refs(tf, zc, h, w, refs, nrefs, tc, Tc, sched[i]) : NULL;
        ok = vu && vc && !iris_hip_memcpy_h2d(dvu, vu, n * sizeof(float)) &&
             !iris_hip_memcpy_h2d(dvc, vc, n * sizeof(float)) &&
             !iris_hip_euler(dz, dvu, dvc, g, sched[i + 1] - sched[i], 1.0f, n) && !iris_hip_sync();
        free(vu);
        free(vc);
        if (ok && cb) cb(i + 1, num_steps);
    }
    if (ok && iris_hip_memcpy_d2h(zc, dz, n * sizeof(float))) ok = 0;
    iris_hip_free(dz);
    if (!ok) {
        free(zc);
        return NULL;
    }
    return zc;
}

/* both CFG branches as one batch-2 pass: slot 0 = uncond, slot 1 = cond */
static float *cfg_batch2(iris_transformer_t *tf, const float *z, int channels, int h, int w, const iris_ref_t *refs,
                         int nrefs, const float *tc, const float *tu, int T, float g, const float *sched,
                         int num_steps, void (*cb)(int, int)) {
    size_t tsz = (size_t)T * iris_transformer_text_dim(tf);
    float *both = (float *)malloc(2 * tsz * sizeof(float));
    if (!both) return NULL;
    memcpy(both, tu, tsz * sizeof(float));
    memcpy(both + tsz, tc, tsz * sizeof(float));
    float *r = flux_loop(tf, z, channels, h, w, refs, nrefs, both, T, 2, g, sched, num_steps, cb);
    free(both);
    return r;
}

float *iris_sample_euler_cfg(void *transformer, void *text_encoder, float *z, int batch, int channels, int h, int w,
                             const float *text_emb_cond, int text_seq_cond, const float *text_emb_uncond,
                             int text_seq_uncond, float guidance_scale, const float *schedule, int num_steps,
                             void (*progress_callback)(int, int)) {
    (void)text_encoder; (void)batch;
    iris_transformer_t *tf = (iris_transformer_t *)transformer;
    if (text_seq_cond == text_seq_uncond && !iris_transformer_csd_active(tf))
        return cfg_batch2(tf, z, channels, h, w, NULL, 0, text_emb_cond, text_emb_uncond, text_seq_cond,
                          guidance_scale, schedule, num_steps, progress_callback);
    /* different text lengths, or a CSD style delta (applied to the
     * conditional forward only): two sequential forwards per step */
    return cfg_two_pass(tf, z, channels, h, w, NULL, 0, text_emb_cond, text_seq_cond, text_emb_uncond,
                        text_seq_uncond, guidance_scale, schedule, num_steps, progress_callback, 1);
}

/* iris_sample_euler_with_refs (iris_sample.c:543-625): one reference image
 * at RoPE T coordinate t_offset */
float *iris_sample_euler_with_refs(void *transformer, void *text_encoder, float *z, int batch, int channels, int h,
                                   int w, const float *ref_latent, int ref_h, int ref_w, int t_offset,
                                   const float *text_emb, int text_seq, const float *schedule, int num_steps,
                                   void (*progress_callback)(int, int)) {
    const iris_ref_t r = {ref_latent, ref_h, ref_w, t_offset};
    return iris_sample_euler_with_multi_refs(transformer, text_encoder, z, batch, channels, h, w, &r,
                                             ref_latent ? 1 : 0, text_emb, text_seq, schedule, num_steps,
                                             progress_callback);
}

/* iris_sample_euler_cfg_with_multi_refs (iris_sample.c:898-989): the
 * reference tokens join both branches; a CSD delta stays on both (the
 * reference toggles it only in the plain CFG sampler) */
float *iris_sample_euler_cfg_with_multi_refs(void *transformer, void *text_encoder, float *z, int batch, int channels,
                                             int h, int w, const iris_ref_t *refs, int num_refs,
                                             const float *text_emb_cond, int text_seq_cond,
                                             const float *text_emb_uncond, int text_seq_uncond, float guidance_scale,
                                             const float *schedule, int num_steps,
                                             void (*progress_callback)(int, int)) {
    (void)text_encoder; (void)batch;
    iris_transformer_t *tf = (iris_transformer_t *)transformer;
    if (!refs) num_refs = 0;
    if (text_seq_cond == text_seq_uncond)
        return cfg_batch2(tf, z, channels, h, w, refs, num_refs, text_emb_cond, text_emb_uncond, text_seq_cond,
                          guidance_scale, schedule, num_steps, progress_callback);
    return cfg_two_pass(tf, z, channels, h, w, refs, num_refs, text_emb_cond, text_seq_cond, text_emb_uncond,
                        text_seq_uncond, guidance_scale, schedule, num_steps, progress_callback, 0);
}

/* iris_sample_euler_cfg_with_refs (iris_sample.c:807-893) */
float *iris_sample_euler_cfg_with_refs(void *transformer, void *text_encoder, float *z, int batch, int channels, int h,
                                       int w, const float *ref_latent, int ref_h, int ref_w, int t_offset,
                                       const float *text_emb_cond, int text_seq_cond, const float *text_emb_uncond,
                                       int text_seq_uncond, float guidance_scale, const float *schedule,
                                       int num_steps, void (*progress_callback)(int, int)) {
    const iris_ref_t r = {ref_latent, ref_h, ref_w, t_offset};
    return iris_sample_euler_cfg_with_multi_refs(transformer, text_encoder, z, batch, channels, h, w, &r,
                                                 ref_latent ? 1 : 0, text_emb_cond, text_seq_cond, text_emb_uncond,
                                                 text_seq_uncond, guidance_scale, schedule, num_steps,
                                                 progress_callback);
}

/* iris_sample_euler_zimage (iris_sample.c:412-536): velocity at timestep
 * 1 - sigma, z += (sigma_next - sigma) * (-v); one image per call, as the
 * reference transformer forward handles one latent. */
float *iris_sample_euler_zimage(void *transformer, float *z, int batch, int channels, int h, int w, int patch_size,
                                const float *cap_feats, int cap_seq, const float *schedule, int num_steps,
                                void (*progress_callback)(int, int)) {
    zi_transformer_t *tf = (zi_transformer_t *)transformer;
    (void)channels; (void)patch_size;
    if (num_steps > IRIS_MAX_STEPS) {
        fprintf(stderr, "iris_sample: num_steps %d exceeds IRIS_MAX_STEPS %d\n", num_steps, IRIS_MAX_STEPS);
        return NULL;
    }
    if (batch != 1) {
        fprintf(stderr, "iris_sample_euler_zimage: batch %d unsupported (one latent per call)\n", batch);
        return NULL;
    }
    if (zi_prepare(tf, h, w, cap_seq) || zi_upload(tf, z, cap_feats)) return NULL;
    for (int i = 0; i < num_steps; i++) {
        if (iris_step_callback) iris_step_callback(i + 1, num_steps);
        if (iris_cancel_requested) return NULL;
        if (zi_step(tf, schedule[i], schedule[i + 1])) return NULL;
        if (progress_callback) progress_callback(i + 1, num_steps);
    }
    size_t n = (size_t)channels * h * w;
    float *out = (float *)malloc(n * sizeof(float));
    if (!out || zi_download_latent(tf, out)) { free(out); return NULL; }
    return out;
}

/* iris_sample_euler_ancestral (iris_sample.c:990-1062): the Euler step on the
 * device, then for eta > 0 and every step but the last sigma = eta sqrt|dt|
 * times a latent of normals drawn on the host from the global generator
 * (iris_randn: same generator, same order as the reference's), uploaded and
 * added by the update kernel. The reference checks for cancellation before
 * each step and calls no step callback. */
float *iris_sample_euler_ancestral(void *transformer, float *z, int batch, int channels, int h, int w,
                                   const float *text_emb, int text_seq, const float *schedule, int num_steps,
                                   float eta, void (*progress_callback)(int, int)) {
    iris_transformer_t *tf = (iris_transformer_t *)transformer;
    (void)batch;
    if (num_steps > IRIS_MAX_STEPS) {
        fprintf(stderr, "iris_sample: num_steps %d exceeds IRIS_MAX_STEPS %d\n", num_steps, IRIS_MAX_STEPS);
        return NULL;
    }
    if (iris_flux_prepare(tf, h, w, NULL, 0, text_seq, 1) || iris_flux_upload(tf, z, NULL, text_emb)) return NULL;
    const size_t n = (size_t)channels * h * w;
    float *lat = (float *)iris_flux_device_buffer(tf, "latent"), *vel = (float *)iris_flux_device_buffer(tf, "velocity");
    float *noise = (float *)malloc(n * sizeof(float)), *out = (float *)malloc(n * sizeof(float));
    int ok = noise && out && lat && vel;
    for (int i = 0; ok && i < num_steps; i++) {
        if (iris_cancel_requested) { ok = 0; break; }
        const float dt = schedule[i + 1] - schedule[i];
        ok = !iris_flux_step(tf, schedule[i], schedule[i + 1], 0.0f);
        if (ok && eta > 0.0f && i < num_steps - 1) {
            /* the velocity buffer is free until the next forward */
            iris_randn(noise, (int)n);
            ok = !iris_hip_memcpy_h2d(vel, noise, n * sizeof(float)) &&
                 !iris_hip_euler(lat, vel, NULL, 0.0f, eta * sqrtf(fabsf(dt)), 1.0f, n);
        }
        if (ok && progress_callback) progress_callback(i + 1, num_steps);
    }
    free(noise);
    if (ok && iris_flux_download_latent(tf, out)) ok = 0;
    if (!ok) {
        free(out);
        return NULL;
    }
    return out;
}

/* iris_sample_heun (iris_sample.c:1063-1145): v1 = v(z, t); except on the last
 * step, z_pred = z + dt v1 in the latent buffer, v2 = v(z_pred, t_next), then
 * z (kept aside with v1) += dt (v1 + (v2 - v1) / 2), the update kernel's
 * guided form of dt / 2 (v1 + v2). */
float *iris_sample_heun(void *transformer, float *z, int batch, int channels, int h, int w, const float *text_emb,
                        int text_seq, const float *schedule, int num_steps, void (*progress_callback)(int, int)) {
    iris_transformer_t *tf = (iris_transformer_t *)transformer;
    (void)batch;
    if (num_steps > IRIS_MAX_STEPS) {
        fprintf(stderr, "iris_sample: num_steps %d exceeds IRIS_MAX_STEPS %d\n", num_steps, IRIS_MAX_STEPS);
        return NULL;
    }
    if (iris_flux_prepare(tf, h, w, NULL, 0, text_seq, 1) || iris_flux_upload(tf, z, NULL, text_emb)) return NULL;
    const size_t n = (size_t)channels * h * w, nb = n * sizeof(float);
    float *lat = (float *)iris_flux_device_buffer(tf, "latent"), *vel = (float *)iris_flux_device_buffer(tf, "velocity");
    float *keep = (float *)iris_hip_malloc(2 * nb);   /* z of the step, then v1 */
    float *out = (float *)malloc(nb);
    int ok = keep && out && lat && vel;
    for (int i = 0; ok && i < num_steps; i++) {
        const float dt = schedule[i + 1] - schedule[i];
        ok = !iris_flux_velocity(tf, schedule[i]);
        if (ok && i < num_steps - 1) {
            ok = !iris_hip_memcpy_d2d(keep, lat, nb) && !iris_hip_memcpy_d2d(keep + n, vel, nb) &&
                 !iris_hip_euler(lat, vel, NULL, 0.0f, dt, 1.0f, n) && !iris_flux_velocity(tf, schedule[i + 1]) &&
                 !iris_hip_memcpy_d2d(lat, keep, nb) && !iris_hip_euler(lat, keep + n, vel, 0.5f, dt, 1.0f, n);
        } else if (ok) {
            ok = !iris_hip_euler(lat, vel, NULL, 0.0f, dt, 1.0f, n);
        }
        if (ok && progress_callback) progress_callback(i + 1, num_steps);
    }
    if (ok && iris_flux_download_latent(tf, out)) ok = 0;
    iris_hip_free(keep);
    if (!ok) {
        free(out);
        return NULL;
    }
    return out;
}
