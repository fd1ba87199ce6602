/*
 * ref_harness_flux.c - exposes static pieces of the reference Flux forward for
 * golden generation. TEST INFRASTRUCTURE ONLY: built by oracle/Makefile's
 * `ref` target from the reference sources where they lie (-I<reference>), into
 * oracle/_ref/, never shipped. Nothing here restates reference code: each
 * wrapper forwards to the reference function of the same role.
 */
#include "iris_transformer_flux.c"

void ref_rope_img(float *c, float *s, int ph, int pw, int axis_dim, float theta, int t_offset) {
    if (t_offset == 0) compute_rope_2d(c, s, ph, pw, axis_dim, theta);
    else compute_rope_2d_with_t_offset(c, s, ph, pw, axis_dim, theta, t_offset);
}

void ref_rope_txt(float *c, float *s, int txt_seq, int axis_dim, float theta) {
    compute_rope_text(c, s, txt_seq, axis_dim, theta);
}

void ref_timestep_sincos(float *out, float t, int dim, float max_period) {
    get_timestep_embedding(out, t, dim, max_period);
}

void ref_time_embed(iris_transformer_t *tf, float t, float *out) {
    float sc[256];
    get_timestep_embedding(sc, t * 1000.0f, 256, 10000.0f);
    time_embed_forward(out, sc, &tf->time_embed, tf->hidden_size, tf->t_emb_silu);
}

/* Modulation vectors exactly as the forward computes them (:4059-4069, :4270-4277);
 * single-block modulation as single_block_forward computes it (:3787-3797). */
void ref_modulation(iris_transformer_t *tf, const float *t_emb, float *dimg, float *dtxt,
                    float *single, float *final_mod) {
    int h = tf->hidden_size;
    for (int j = 0; j < h; j++) { float x = t_emb[j]; tf->t_emb_silu[j] = x / (1.0f + expf(-x)); }
    if (dimg) iris_linear_nobias(dimg, tf->t_emb_silu, tf->adaln_double_img_weight, 1, h, 6 * h);
    if (dtxt) iris_linear_nobias(dtxt, tf->t_emb_silu, tf->adaln_double_txt_weight, 1, h, 6 * h);
    if (single) iris_linear_nobias(single, tf->t_emb_silu, tf->adaln_single_weight, 1, h, 3 * h);
    if (final_mod) iris_linear_nobias(final_mod, tf->t_emb_silu, tf->final_norm_weight, 1, h, 2 * h);
}

int ref_double_block(iris_transformer_t *tf, int idx, float *img, float *txt,
                     const float *img_mod, const float *txt_mod,
                     const float *ic, const float *is, const float *tc, const float *ts,
                     int img_seq, int txt_seq) {
    if (ensure_work_buffers(tf, img_seq + txt_seq) < 0) return -1;
    if (ensure_attn_scores(tf, img_seq, txt_seq) < 0) return -1;
    double_block_forward(img, txt, &tf->double_blocks[idx], img_mod, txt_mod,
                         ic, is, tc, ts, img_seq, txt_seq, idx, tf);
    return 0;
}

int ref_single_block(iris_transformer_t *tf, int idx, float *x, const float *t_emb,
                     const float *ic, const float *is, const float *tc, const float *ts,
                     int seq, int img_offset) {
    if (ensure_work_buffers(tf, seq) < 0) return -1;
    if (ensure_attn_scores(tf, seq - img_offset, img_offset) < 0) return -1;
    tf->sref_krope_cos = NULL;
    tf->sref_krope_sin = NULL;
    single_block_forward(x, &tf->single_blocks[idx], t_emb, tf->adaln_single_weight,
                         ic, is, tc, ts, seq, img_offset, idx, tf);
    return 0;
}

float ref_fast_expf(float x) { return fast_expf(x); }
