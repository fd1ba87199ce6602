/*
 * ref_harness_zimage.c - exposes static pieces of the reference Z-Image forward
 * for golden generation. TEST INFRASTRUCTURE ONLY (see ref_harness_flux.c).
 */
#include "iris_transformer_zimage.c"

void ref_zi_rope_table(zi_transformer_t *tf, float *c, float *s, int axis) {
    int half = tf->axes_dims[axis] / 2;
    memcpy(c, tf->rope_cos[axis], (size_t)tf->axes_lens[axis] * half * sizeof(float));
    memcpy(s, tf->rope_sin[axis], (size_t)tf->axes_lens[axis] * half * sizeof(float));
}

void ref_zi_patchify(float *out, const float *latent, int in_ch, int H, int W, int ps) {
    zi_patchify(out, latent, in_ch, H, W, ps);
}

void ref_zi_t_embed(zi_transformer_t *tf, float t, float *out) {
    zi_timestep_embed(tf, out, t);
}

/* kind: 0 noise_refiner, 1 context_refiner, 2 main layer */
int ref_zi_block(zi_transformer_t *tf, int kind, int idx, float *x, const int *pos,
                 const int *mask, const float *t_emb, int seq) {
    size_t needed = (size_t)seq * tf->dim * 4 + (size_t)seq * tf->dim * 3 +
                    (size_t)seq * seq + (size_t)seq * tf->ffn_dim * 2;
    if (needed > tf->work_alloc || tf->max_seq < seq) {
        free(tf->work_x); free(tf->work_tmp); free(tf->work_qkv); free(tf->work_attn); free(tf->work_ffn);
        tf->work_x = malloc((size_t)seq * tf->dim * sizeof(float));
        tf->work_tmp = malloc((size_t)seq * tf->dim * 4 * sizeof(float));
        tf->work_qkv = malloc((size_t)seq * tf->dim * 3 * sizeof(float));
        tf->work_attn = malloc((size_t)seq * seq * sizeof(float));
        tf->work_ffn = malloc((size_t)seq * tf->ffn_dim * 2 * sizeof(float));
        tf->work_alloc = needed;
        tf->max_seq = seq;
    }
    const zi_block_t *b = kind == 0 ? &tf->noise_refiner[idx] :
                          kind == 1 ? &tf->context_refiner[idx] : &tf->layers[idx];
    zi_block_forward(x, b, pos, mask, kind == 1 ? NULL : t_emb, seq, tf);
    return 0;
}

void ref_zi_sincos(float *out, float t) {
    zi_sinusoidal_embedding(out, t, 256);
}
