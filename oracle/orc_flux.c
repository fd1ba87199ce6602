/*
 * orc_flux.c - f32 restatement of the Flux.2-Klein denoiser forward
 * (reference iris_transformer_flux.c, BLAS build: use_bf16 = 0).
 * TEST INFRASTRUCTURE ONLY (see iris_oracle.h).
 */
#include "orc_internal.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

typedef struct {
    float *img_q, *img_k, *img_v, *img_nq, *img_nk, *img_o, *img_gate, *img_up, *img_down;
    float *txt_q, *txt_k, *txt_v, *txt_nq, *txt_nk, *txt_o, *txt_gate, *txt_up, *txt_down;
} orc_dbl_t;

typedef struct {
    float *qkv_mlp, *nq, *nk, *out;
} orc_sgl_t;

struct orc_flux {
    int hidden, heads, head_dim, mlp, n_double, n_single, text_dim, latent_ch, axis_dim;
    float theta;
    float *img_in, *txt_in, *t_fc1, *t_fc2;
    float *mod_dimg, *mod_dtxt, *mod_single, *final_mod, *proj_out;
    orc_dbl_t *dbl;
    orc_sgl_t *sgl;
    /* SREF RoPE band control (iris_transformer_flux.c:326-335); off when both are 1 */
    float sref_shf, sref_slf;
    int sref_set;   /* 0: never set (calloc), bands off */
};

/* ------------------------------------------------------------------ config */

/* parse_transformer_config, iris_transformer_flux.c:395-455 */
static int parse_config(const char *dir, orc_flux_t *m) {
    char path[2048];
    snprintf(path, sizeof(path), "%s/transformer/config.json", dir);
    FILE *f = fopen(path, "r");
    if (!f) return -1;
    char buf[4096];
    size_t n = fread(buf, 1, sizeof(buf) - 1, f);
    buf[n] = 0;
    fclose(f);
    int heads = 0, hd = 0, nl = 0, ns = 0, jd = 0, ic = 0;
    float ratio = 0, theta = 0;
    char *p;
#define GETI(key, var) if ((p = strstr(buf, "\"" key "\"")) && (p = strchr(p, ':'))) var = atoi(p + 1)
#define GETF(key, var) if ((p = strstr(buf, "\"" key "\"")) && (p = strchr(p, ':'))) var = (float)atof(p + 1)
    GETI("num_attention_heads", heads);
    GETI("attention_head_dim", hd);
    GETI("num_layers", nl);
    GETI("num_single_layers", ns);
    GETI("joint_attention_dim", jd);
    GETI("in_channels", ic);
    GETF("mlp_ratio", ratio);
    GETF("rope_theta", theta);
#undef GETI
#undef GETF
    if (heads <= 0 || hd <= 0) return -1;
    m->heads = heads;
    m->head_dim = hd;
    m->hidden = heads * hd;
    m->mlp = (int)(m->hidden * (ratio > 0 ? ratio : 3.0f));
    m->n_double = nl > 0 ? nl : 5;
    m->n_single = ns > 0 ? ns : 20;
    m->text_dim = jd > 0 ? jd : 7680;
    m->latent_ch = ic > 0 ? ic : 128;
    m->theta = theta > 0 ? theta : 2000.0f;
    m->axis_dim = hd / 4;
    return 0;
}

static void set_defaults(orc_flux_t *m) {
    m->hidden = 3072; m->heads = 24; m->head_dim = 128; m->mlp = 9216;
    m->n_double = 5; m->n_single = 20; m->text_dim = 7680; m->latent_ch = 128;
    m->theta = 2000.0f; m->axis_dim = 32;
}

/* ------------------------------------------------------------- weight load */

typedef float *(*getter_t)(void *ctx, const char *name, size_t n, int is_norm);

static float *get_st(void *ctx, const char *name, size_t n, int is_norm) {
    (void)n; (void)is_norm;
    return orc_load_f32((const iris_st_set_t *)ctx, name);
}

static float *get_synth(void *ctx, const char *name, size_t n, int is_norm) {
    uint64_t seed = *(const uint64_t *)ctx;
    return orc_synth_f32(seed, name, n, is_norm ? 1.0f : 0.0f, 0.02f);
}

static int load_all(orc_flux_t *m, getter_t get, void *ctx) {
    size_t h = m->hidden, mlp = m->mlp, hd = m->head_dim;
    char nm[256];
#define GET(dst, name, n, norm) do { if (!((dst) = get(ctx, (name), (n), (norm)))) return -1; } while (0)
    /* tensor names: iris_transformer_flux.c:5349-5497 */
    GET(m->img_in, "x_embedder.weight", h * m->latent_ch, 0);
    GET(m->txt_in, "context_embedder.weight", h * m->text_dim, 0);
    GET(m->t_fc1, "time_guidance_embed.timestep_embedder.linear_1.weight", h * 256, 0);
    GET(m->t_fc2, "time_guidance_embed.timestep_embedder.linear_2.weight", h * h, 0);
    GET(m->mod_dimg, "double_stream_modulation_img.linear.weight", 6 * h * h, 0);
    GET(m->mod_dtxt, "double_stream_modulation_txt.linear.weight", 6 * h * h, 0);
    GET(m->mod_single, "single_stream_modulation.linear.weight", 3 * h * h, 0);
    m->dbl = (orc_dbl_t *)calloc((size_t)m->n_double, sizeof(orc_dbl_t));
    m->sgl = (orc_sgl_t *)calloc((size_t)m->n_single, sizeof(orc_sgl_t));
    for (int i = 0; i < m->n_double; i++) {
        orc_dbl_t *b = &m->dbl[i];
#define BLK(dst, fmt, n, norm) do { snprintf(nm, sizeof(nm), fmt, i); GET(dst, nm, n, norm); } while (0)
        BLK(b->img_nq, "transformer_blocks.%d.attn.norm_q.weight", hd, 1);
        BLK(b->img_nk, "transformer_blocks.%d.attn.norm_k.weight", hd, 1);
        BLK(b->img_q, "transformer_blocks.%d.attn.to_q.weight", h * h, 0);
        BLK(b->img_k, "transformer_blocks.%d.attn.to_k.weight", h * h, 0);
        BLK(b->img_v, "transformer_blocks.%d.attn.to_v.weight", h * h, 0);
        BLK(b->img_o, "transformer_blocks.%d.attn.to_out.0.weight", h * h, 0);
        BLK(b->img_gate, "transformer_blocks.%d.ff.linear_in.weight", 2 * mlp * h, 0);
        b->img_up = b->img_gate + mlp * h;      /* gate rows then up rows, :633-640 */
        BLK(b->img_down, "transformer_blocks.%d.ff.linear_out.weight", h * mlp, 0);
        BLK(b->txt_nq, "transformer_blocks.%d.attn.norm_added_q.weight", hd, 1);
        BLK(b->txt_nk, "transformer_blocks.%d.attn.norm_added_k.weight", hd, 1);
        BLK(b->txt_q, "transformer_blocks.%d.attn.add_q_proj.weight", h * h, 0);
        BLK(b->txt_k, "transformer_blocks.%d.attn.add_k_proj.weight", h * h, 0);
        BLK(b->txt_v, "transformer_blocks.%d.attn.add_v_proj.weight", h * h, 0);
        BLK(b->txt_o, "transformer_blocks.%d.attn.to_add_out.weight", h * h, 0);
        BLK(b->txt_gate, "transformer_blocks.%d.ff_context.linear_in.weight", 2 * mlp * h, 0);
        b->txt_up = b->txt_gate + mlp * h;
        BLK(b->txt_down, "transformer_blocks.%d.ff_context.linear_out.weight", h * mlp, 0);
    }
    for (int i = 0; i < m->n_single; i++) {
        orc_sgl_t *b = &m->sgl[i];
        BLK(b->nq, "single_transformer_blocks.%d.attn.norm_q.weight", hd, 1);
        BLK(b->nk, "single_transformer_blocks.%d.attn.norm_k.weight", hd, 1);
        BLK(b->qkv_mlp, "single_transformer_blocks.%d.attn.to_qkv_mlp_proj.weight", (3 * h + 2 * mlp) * h, 0);
        BLK(b->out, "single_transformer_blocks.%d.attn.to_out.weight", h * (h + mlp), 0);
#undef BLK
    }
    GET(m->final_mod, "norm_out.linear.weight", 2 * h * h, 0);
    GET(m->proj_out, "proj_out.weight", (size_t)m->latent_ch * h, 0);
#undef GET
    return 0;
}

orc_flux_t *orc_flux_load(const char *dir) {
    orc_flux_t *m = (orc_flux_t *)calloc(1, sizeof(*m));
    if (!m) return NULL;
    if (parse_config(dir, m)) set_defaults(m);
    iris_st_set_t s;
    if (iris_st_set_open(&s, dir)) { free(m); return NULL; }
    int rc = load_all(m, get_st, &s);
    iris_st_set_close(&s);
    if (rc) { orc_flux_free(m); return NULL; }
    return m;
}

orc_flux_t *orc_flux_create_synth(int hidden, int heads, int n_double, int n_single,
                                  int text_dim, int latent_ch, float mlp_ratio,
                                  float rope_theta, uint64_t seed) {
    orc_flux_t *m = (orc_flux_t *)calloc(1, sizeof(*m));
    if (!m) return NULL;
    m->hidden = hidden; m->heads = heads; m->head_dim = hidden / heads;
    m->mlp = (int)(hidden * mlp_ratio); m->n_double = n_double; m->n_single = n_single;
    m->text_dim = text_dim; m->latent_ch = latent_ch; m->theta = rope_theta;
    m->axis_dim = m->head_dim / 4;
    if (load_all(m, get_synth, &seed)) { orc_flux_free(m); return NULL; }
    return m;
}

void orc_flux_free(orc_flux_t *m) {
    if (!m) return;
    free(m->img_in); free(m->txt_in); free(m->t_fc1); free(m->t_fc2);
    free(m->mod_dimg); free(m->mod_dtxt); free(m->mod_single); free(m->final_mod); free(m->proj_out);
    for (int i = 0; m->dbl && i < m->n_double; i++) {
        orc_dbl_t *b = &m->dbl[i];
        free(b->img_q); free(b->img_k); free(b->img_v); free(b->img_nq); free(b->img_nk);
        free(b->img_o); free(b->img_gate); free(b->img_down);
        free(b->txt_q); free(b->txt_k); free(b->txt_v); free(b->txt_nq); free(b->txt_nk);
        free(b->txt_o); free(b->txt_gate); free(b->txt_down);
    }
    for (int i = 0; m->sgl && i < m->n_single; i++) {
        free(m->sgl[i].qkv_mlp); free(m->sgl[i].nq); free(m->sgl[i].nk); free(m->sgl[i].out);
    }
    free(m->dbl); free(m->sgl); free(m);
}

int orc_flux_dims(const orc_flux_t *m, int *o) {
    o[0] = m->hidden; o[1] = m->heads; o[2] = m->head_dim; o[3] = m->mlp;
    o[4] = m->n_double; o[5] = m->n_single; o[6] = m->text_dim; o[7] = m->latent_ch;
    return 0;
}

/* ------------------------------------------------------------------- RoPE */

/* compute_rope_2d / compute_rope_2d_with_t_offset, iris_transformer_flux.c:896-1018.
 * t_offset 0 reproduces compute_rope_2d (axis 0 identity). */
void orc_rope_img(float *cos_out, float *sin_out, int ph, int pw, int axis_dim,
                  float theta, int t_offset) {
    int half = axis_dim / 2;
    float base[64];
    orc_rope_bases(base, half, axis_dim, theta);
    for (int y = 0; y < ph; y++) {
        for (int x = 0; x < pw; x++) {
            int pos = y * pw + x;
            float *c = cos_out + (size_t)pos * axis_dim * 4;
            float *s = sin_out + (size_t)pos * axis_dim * 4;
            if (t_offset == 0) {
                for (int d = 0; d < axis_dim; d++) { c[d] = 1.0f; s[d] = 0.0f; }
            } else {
                for (int d = 0; d < half; d++) {
                    float a = (float)t_offset * base[d];
                    float cv = cosf(a), sv = sinf(a);
                    c[2 * d] = cv; c[2 * d + 1] = cv; s[2 * d] = sv; s[2 * d + 1] = sv;
                }
            }
            for (int d = 0; d < half; d++) {
                float a = (float)y * base[d];
                float cv = cosf(a), sv = sinf(a);
                c[axis_dim + 2 * d] = cv; c[axis_dim + 2 * d + 1] = cv;
                s[axis_dim + 2 * d] = sv; s[axis_dim + 2 * d + 1] = sv;
            }
            for (int d = 0; d < half; d++) {
                float a = (float)x * base[d];
                float cv = cosf(a), sv = sinf(a);
                c[2 * axis_dim + 2 * d] = cv; c[2 * axis_dim + 2 * d + 1] = cv;
                s[2 * axis_dim + 2 * d] = sv; s[2 * axis_dim + 2 * d + 1] = sv;
            }
            for (int d = 0; d < axis_dim; d++) { c[3 * axis_dim + d] = 1.0f; s[3 * axis_dim + d] = 0.0f; }
        }
    }
}

/* compute_rope_text, iris_transformer_flux.c:1055-1087 */
void orc_rope_txt(float *cos_out, float *sin_out, int txt_seq, int axis_dim, float theta) {
    int half = axis_dim / 2, hd = axis_dim * 4;
    float base[64];
    orc_rope_bases(base, half, axis_dim, theta);
    for (int t = 0; t < txt_seq; t++) {
        float *c = cos_out + (size_t)t * hd, *s = sin_out + (size_t)t * hd;
        for (int d = 0; d < axis_dim * 3; d++) { c[d] = 1.0f; s[d] = 0.0f; }
        for (int d = 0; d < half; d++) {
            float a = (float)t * base[d];
            float cv = cosf(a), sv = sinf(a);
            c[3 * axis_dim + 2 * d] = cv; c[3 * axis_dim + 2 * d + 1] = cv;
            s[3 * axis_dim + 2 * d] = sv; s[3 * axis_dim + 2 * d + 1] = sv;
        }
    }
}

/* apply_rope_2d, iris_transformer_flux.c:1026-1048 */
static void apply_rope(float *x, const float *cs, const float *sn, int seq, int heads, int hd) {
#pragma omp parallel for schedule(static) if (seq >= 256)
    for (int s = 0; s < seq; s++) {
        const float *c = cs + (size_t)s * hd, *si = sn + (size_t)s * hd;
        for (int h = 0; h < heads; h++) {
            float *v = x + ((size_t)s * heads + h) * hd;
            for (int d = 0; d < hd; d += 2) {
                float x0 = v[d], x1 = v[d + 1];
                v[d] = x0 * c[d] - x1 * si[d];
                v[d + 1] = x1 * c[d] + x0 * si[d];
            }
        }
    }
}

/* ------------------------------------------------------- t-emb, modulation */

/* get_timestep_embedding, iris_transformer_flux.c:1349-1360 */
void orc_timestep_sincos(float *out, float t, int dim, float max_period) {
    int half = dim / 2;
    float lm = logf(max_period);
    for (int i = 0; i < half; i++) {
        float a = t * expf(-lm * (float)i / (float)half);   /* scalar expf, as built */
        out[i] = cosf(a);
        out[i + half] = sinf(a);
    }
}

/* time_embed_forward, iris_transformer_flux.c:1366-1379; t scaled by 1000 at :3967 */
void orc_flux_time_embed(orc_flux_t *m, float t, float *t_emb) {
    float sc[256];
    orc_timestep_sincos(sc, t * 1000.0f, 256, 10000.0f);
    float *w = (float *)malloc((size_t)m->hidden * sizeof(float));
    orc_linear(w, sc, m->t_fc1, NULL, 1, 256, m->hidden);
    orc_silu(w, m->hidden);
    orc_linear(t_emb, w, m->t_fc2, NULL, 1, m->hidden, m->hidden);
    free(w);
}

/* SiLU(t_emb) with expf then GEMV: iris_transformer_flux.c:4059-4069 (double),
 * :3787-3797 (single), :4270-4277 (final). */
void orc_flux_modulation(orc_flux_t *m, const float *t_emb, float *dimg, float *dtxt,
                         float *single, float *final_mod) {
    int h = m->hidden;
    float *s = (float *)malloc((size_t)h * sizeof(float));
    for (int j = 0; j < h; j++) { float x = t_emb[j]; s[j] = x / (1.0f + expf(-x)); }
    if (dimg) orc_linear(dimg, s, m->mod_dimg, NULL, 1, h, 6 * h);
    if (dtxt) orc_linear(dtxt, s, m->mod_dtxt, NULL, 1, h, 6 * h);
    if (single) orc_linear(single, s, m->mod_single, NULL, 1, h, 3 * h);
    if (final_mod) orc_linear(final_mod, s, m->final_mod, NULL, 1, h, 2 * h);
    free(s);
}

/* ------------------------------------------------------------ block pieces */

/* apply_adaln (scalar branch), iris_transformer_flux.c:1431-1459 */
static void adaln(float *out, const float *x, const float *shift, const float *scale,
                  int seq, int h, float eps) {
#pragma omp parallel for schedule(static) if (seq >= 256)
    for (int s = 0; s < seq; s++) {
        const float *xr = x + (size_t)s * h;
        float *o = out + (size_t)s * h;
        float sum = 0.0f;
        for (int i = 0; i < h; i++) sum += xr[i];
        float mean = sum / h;
        float vs = 0.0f;
        for (int i = 0; i < h; i++) { float d = xr[i] - mean; vs += d * d; }
        float inv = 1.0f / sqrtf(vs / h + eps);
        for (int i = 0; i < h; i++) o[i] = (1.0f + scale[i]) * ((xr[i] - mean) * inv) + shift[i];
    }
}

/* apply_qk_norm (scalar branch), iris_transformer_flux.c:1490-1517 */
static void qk_norm(float *q, float *k, const float *qw, const float *kw,
                    int seq, int heads, int hd, float eps) {
#pragma omp parallel for schedule(static) if (seq >= 256)
    for (int s = 0; s < seq; s++) {
        for (int h = 0; h < heads; h++) {
            float *v = q + ((size_t)s * heads + h) * hd;
            float ss = 0.0f;
            for (int d = 0; d < hd; d++) ss += v[d] * v[d];
            float inv = 1.0f / sqrtf(ss / hd + eps);
            for (int d = 0; d < hd; d++) v[d] = v[d] * inv * qw[d];
            v = k + ((size_t)s * heads + h) * hd;
            ss = 0.0f;
            for (int d = 0; d < hd; d++) ss += v[d] * v[d];
            inv = 1.0f / sqrtf(ss / hd + eps);
            for (int d = 0; d < hd; d++) v[d] = v[d] * inv * kw[d];
        }
    }
}

/* gated_add, iris_transformer_flux.c:136-143 */
static void gated_add(float *out, const float *gate, const float *proj, int seq, int h) {
#pragma omp parallel for schedule(static) if (seq >= 256)
    for (int s = 0; s < seq; s++)
        for (int i = 0; i < h; i++) out[(size_t)s * h + i] += gate[i] * proj[(size_t)s * h + i];
}

/* Per-head attention of the BLAS build, iris_transformer_flux.c:1703-1723 and
 * :1886-2022: scores = scale * Q_h K_h^T (sgemm), iris_softmax_cpu, out_h = P V_h.
 * K, V rows are [txt, img] for joint attention; all tensors have row stride hidden.
 * Heads run in parallel as the reference's pthread workers do. */
static void attention(float *out, const float *q, const float *k, const float *v,
                      int seq_q, int seq_k, int heads, int hd) {
    int hidden = heads * hd;
    float scale = 1.0f / sqrtf((float)hd);
    long ncpu = sysconf(_SC_NPROCESSORS_ONLN);
    int nt = (int)(ncpu < 1 ? 1 : ncpu);
    if (nt > heads) nt = heads;
    while (heads % nt) nt--;
    float *scores = (float *)malloc((size_t)heads * seq_q * seq_k * sizeof(float));
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int h = 0; h < heads; h++) {
        float *sh = scores + (size_t)h * seq_q * seq_k;
        orc_sgemm_nt(seq_q, seq_k, hd, scale, q + h * hd, hidden, k + h * hd, hidden, 0.0f, sh, seq_k);
        orc_softmax(sh, seq_q, seq_k);
        orc_sgemm_nn(seq_q, hd, seq_k, 1.0f, sh, seq_k, v + h * hd, hidden, 0.0f, out + h * hd, hidden);
    }
    free(scores);
}

/* swiglu_ffn_bf16 (f32 weights), iris_transformer_flux.c:2299-2324 */
static void swiglu_ffn(float *out, const float *x, const float *wg, const float *wu,
                       const float *wd, int seq, int h, int mlp) {
    float *g = (float *)malloc((size_t)seq * mlp * sizeof(float));
    float *u = (float *)malloc((size_t)seq * mlp * sizeof(float));
    orc_linear(g, x, wg, NULL, seq, h, mlp);
    orc_linear(u, x, wu, NULL, seq, h, mlp);
    orc_silu_mul(g, u, (size_t)seq * mlp);
    orc_linear(out, g, wd, NULL, seq, mlp, h);
    free(g); free(u);
}

/* double_block_forward, iris_transformer_flux.c:2366-2614 (LoRA/IP hooks off) */
void orc_flux_double_block(orc_flux_t *m, int idx, float *img, float *txt,
                           const float *img_mod, const float *txt_mod,
                           const float *img_cos, const float *img_sin,
                           const float *txt_cos, const float *txt_sin,
                           int I, int T) {
    const orc_dbl_t *b = &m->dbl[idx];
    int h = m->hidden, H = m->heads, hd = m->head_dim, mlp = m->mlp, S = I + T;
    float eps = 1e-6f;
    const float *is1 = img_mod, *isc1 = img_mod + h, *ig1 = img_mod + 2 * h;
    const float *is2 = img_mod + 3 * h, *isc2 = img_mod + 4 * h, *ig2 = img_mod + 5 * h;
    const float *ts1 = txt_mod, *tsc1 = txt_mod + h, *tg1 = txt_mod + 2 * h;
    const float *ts2 = txt_mod + 3 * h, *tsc2 = txt_mod + 4 * h, *tg2 = txt_mod + 5 * h;
    size_t hs = (size_t)h * sizeof(float);
    float *inorm = (float *)malloc(I * hs), *tnorm = (float *)malloc(T * hs);
    float *iq = (float *)malloc(I * hs), *ik = (float *)malloc(I * hs), *iv = (float *)malloc(I * hs);
    float *tq = (float *)malloc(T * hs), *tk = (float *)malloc(T * hs), *tv = (float *)malloc(T * hs);
    adaln(inorm, img, is1, isc1, I, h, eps);
    orc_linear(iq, inorm, b->img_q, NULL, I, h, h);
    orc_linear(ik, inorm, b->img_k, NULL, I, h, h);
    orc_linear(iv, inorm, b->img_v, NULL, I, h, h);
    qk_norm(iq, ik, b->img_nq, b->img_nk, I, H, hd, eps);
    apply_rope(iq, img_cos, img_sin, I, H, hd);
    apply_rope(ik, img_cos, img_sin, I, H, hd);
    adaln(tnorm, txt, ts1, tsc1, T, h, eps);
    orc_linear(tq, tnorm, b->txt_q, NULL, T, h, h);
    orc_linear(tk, tnorm, b->txt_k, NULL, T, h, h);
    orc_linear(tv, tnorm, b->txt_v, NULL, T, h, h);
    qk_norm(tq, tk, b->txt_nq, b->txt_nk, T, H, hd, eps);
    apply_rope(tq, txt_cos, txt_sin, T, H, hd);
    apply_rope(tk, txt_cos, txt_sin, T, H, hd);
    /* cat K/V as [TXT, IMG], :1902-1905 */
    float *ck = (float *)malloc(S * hs), *cv = (float *)malloc(S * hs);
    memcpy(ck, tk, T * hs); memcpy(ck + (size_t)T * h, ik, I * hs);
    memcpy(cv, tv, T * hs); memcpy(cv + (size_t)T * h, iv, I * hs);
    float *iattn = (float *)malloc(I * hs), *tattn = (float *)malloc(T * hs);
    attention(iattn, iq, ck, cv, I, S, H, hd);
    attention(tattn, tq, ck, cv, T, S, H, hd);
    float *iproj = (float *)malloc(I * hs), *tproj = (float *)malloc(T * hs);
    orc_linear(iproj, iattn, b->img_o, NULL, I, h, h);
    orc_linear(tproj, tattn, b->txt_o, NULL, T, h, h);
    gated_add(img, ig1, iproj, I, h);
    gated_add(txt, tg1, tproj, T, h);
    adaln(inorm, img, is2, isc2, I, h, eps);
    swiglu_ffn(iproj, inorm, b->img_gate, b->img_up, b->img_down, I, h, mlp);
    gated_add(img, ig2, iproj, I, h);
    adaln(tnorm, txt, ts2, tsc2, T, h, eps);
    swiglu_ffn(tproj, tnorm, b->txt_gate, b->txt_up, b->txt_down, T, h, mlp);
    gated_add(txt, tg2, tproj, T, h);
    free(inorm); free(tnorm); free(iq); free(ik); free(iv); free(tq); free(tk); free(tv);
    free(ck); free(cv); free(iattn); free(tattn); free(iproj); free(tproj);
}

/* single_block_forward, iris_transformer_flux.c:3761-3928 (LoRA/IP off).
 * seq = txt + img rows, img_offset = txt rows. K of the img rows rotates with
 * kimg_cos/kimg_sin: the SREF band-scaled table when band control is on
 * (:3869-3875), else the Q table. */
void orc_flux_single_block_k(orc_flux_t *m, int idx, float *x, const float *t_emb,
                             const float *img_cos, const float *img_sin,
                             const float *kimg_cos, const float *kimg_sin,
                             const float *txt_cos, const float *txt_sin,
                             int seq, int img_offset) {
    const orc_sgl_t *b = &m->sgl[idx];
    int h = m->hidden, H = m->heads, hd = m->head_dim, mlp = m->mlp;
    int fused = 3 * h + 2 * mlp, I = seq - img_offset, T = img_offset;
    float eps = 1e-6f;
    float *ts = (float *)malloc((size_t)h * sizeof(float));
    for (int i = 0; i < h; i++) { float v = t_emb[i]; ts[i] = v / (1.0f + expf(-v)); }
    float *mod = (float *)malloc((size_t)3 * h * sizeof(float));
    orc_linear(mod, ts, m->mod_single, NULL, 1, h, 3 * h);
    const float *shift = mod, *scale = mod + h, *gate = mod + 2 * h;
    float *norm = (float *)malloc((size_t)seq * h * sizeof(float));
    adaln(norm, x, shift, scale, seq, h, eps);
    float *fo = (float *)malloc((size_t)seq * fused * sizeof(float));
    orc_linear(fo, norm, b->qkv_mlp, NULL, seq, h, fused);
    float *q = (float *)malloc((size_t)seq * h * sizeof(float));
    float *k = (float *)malloc((size_t)seq * h * sizeof(float));
    float *v = (float *)malloc((size_t)seq * h * sizeof(float));
    float *g = (float *)malloc((size_t)seq * mlp * sizeof(float));
    float *u = (float *)malloc((size_t)seq * mlp * sizeof(float));
    for (int s = 0; s < seq; s++) {      /* split, :3833-3840 */
        const float *r = fo + (size_t)s * fused;
        memcpy(q + (size_t)s * h, r, h * sizeof(float));
        memcpy(k + (size_t)s * h, r + h, h * sizeof(float));
        memcpy(v + (size_t)s * h, r + 2 * h, h * sizeof(float));
        memcpy(g + (size_t)s * mlp, r + 3 * h, mlp * sizeof(float));
        memcpy(u + (size_t)s * mlp, r + 3 * h + mlp, mlp * sizeof(float));
    }
    free(fo);
    qk_norm(q, k, b->nq, b->nk, seq, H, hd, eps);
    apply_rope(q, txt_cos, txt_sin, T, H, hd);
    apply_rope(k, txt_cos, txt_sin, T, H, hd);
    apply_rope(q + (size_t)T * h, img_cos, img_sin, I, H, hd);
    apply_rope(k + (size_t)T * h, kimg_cos, kimg_sin, I, H, hd);
    float *attn = (float *)malloc((size_t)seq * h * sizeof(float));
    attention(attn, q, k, v, seq, seq, H, hd);
    orc_silu_mul(g, u, (size_t)seq * mlp);
    float *cat = (float *)malloc((size_t)seq * (h + mlp) * sizeof(float));
    for (int s = 0; s < seq; s++) {      /* concat [attn | mlp], :3897-3902 */
        memcpy(cat + (size_t)s * (h + mlp), attn + (size_t)s * h, h * sizeof(float));
        memcpy(cat + (size_t)s * (h + mlp) + h, g + (size_t)s * mlp, mlp * sizeof(float));
    }
    orc_linear(norm, cat, b->out, NULL, seq, h + mlp, h);
    gated_add(x, gate, norm, seq, h);
    free(ts); free(mod); free(norm); free(q); free(k); free(v); free(g); free(u);
    free(attn); free(cat);
}

void orc_flux_single_block(orc_flux_t *m, int idx, float *x, const float *t_emb,
                           const float *img_cos, const float *img_sin,
                           const float *txt_cos, const float *txt_sin,
                           int seq, int img_offset) {
    orc_flux_single_block_k(m, idx, x, t_emb, img_cos, img_sin, img_cos, img_sin, txt_cos, txt_sin, seq,
                            img_offset);
}

/* iris_transformer_set_sref_bands, iris_transformer_flux.c:5153-5157: out-of-range values switch off */
void orc_flux_set_sref_bands(orc_flux_t *m, float shf, float slf) {
    m->sref_shf = (shf >= 0.0f && shf <= 1.0f) ? shf : 1.0f;
    m->sref_slf = (slf >= 1.0f) ? slf : 1.0f;
    m->sref_set = 1;
}

/* band_scale_ref_krope, iris_transformer_flux.c:1271-1292: the H (axis 1)
 * and W (axis 2) rotation pairs d of rows [ref_start, rows) scaled by
 * shf + (slf - shf) (d / (half - 1))^2, tables [rows][4 * axis_dim] */
void orc_sref_band_scale(float *c, float *s, int ref_start, int rows, int axis_dim, float shf, float slf) {
    const int half = axis_dim / 2;
    float sd[64];
    for (int d = 0; d < half && d < 64; d++) {
        const float dn = half > 1 ? (float)d / (float)(half - 1) : 0.0f;
        sd[d] = shf + (slf - shf) * dn * dn;
    }
    for (int r = ref_start; r < rows; r++) {
        float *cr = c + (size_t)r * axis_dim * 4, *sr = s + (size_t)r * axis_dim * 4;
        for (int d = 0; d < half; d++) {
            const int a = axis_dim + 2 * d, b = 2 * axis_dim + 2 * d;
            cr[a] *= sd[d]; cr[a + 1] *= sd[d]; sr[a] *= sd[d]; sr[a + 1] *= sd[d];
            cr[b] *= sd[d]; cr[b + 1] *= sd[d]; sr[b] *= sd[d]; sr[b + 1] *= sd[d];
        }
    }
}

/* ---------------------------------------------------------------- forward */

/* Shared body of iris_transformer_forward (:3939-4326) and the reference-token
 * variants (:4354-4563, :4579-4829): img rows = target then references; only
 * the target rows reach the final layer. */
static float *forward_impl(orc_flux_t *m, const float *latent, int ih, int iw,
                           const orc_ref_t *refs, int n_refs,
                           const float *txt, int T, float t) {
    int h = m->hidden, C = m->latent_ch, ad = m->axis_dim, hd = m->head_dim;
    int I0 = ih * iw, I = I0;
    for (int r = 0; r < n_refs; r++) I += refs[r].h * refs[r].w;
    int S = I + T;
    float *t_emb = (float *)malloc((size_t)h * sizeof(float));
    orc_flux_time_embed(m, t, t_emb);
    /* RoPE: target (T=0) then refs with their T offsets (:4634-4657) */
    float *icos = (float *)malloc((size_t)I * hd * sizeof(float));
    float *isin = (float *)malloc((size_t)I * hd * sizeof(float));
    orc_rope_img(icos, isin, ih, iw, ad, m->theta, 0);
    size_t off = (size_t)I0 * hd;
    for (int r = 0; r < n_refs; r++) {
        orc_rope_img(icos + off, isin + off, refs[r].h, refs[r].w, ad, m->theta, refs[r].t_offset);
        off += (size_t)refs[r].h * refs[r].w * hd;
    }
    float *tcos = (float *)malloc((size_t)T * hd * sizeof(float));
    float *tsin = (float *)malloc((size_t)T * hd * sizeof(float));
    orc_rope_txt(tcos, tsin, T, ad, m->theta);
    /* SREF K-side table (set_kside_krope, :1297-1322, built at :4660): a copy
     * of the image table with the reference rows band-scaled; single blocks
     * rotate K with it, double blocks with the plain table */
    float *kcos = icos, *ksin = isin;
    if (n_refs > 0 && m->sref_set && !(m->sref_shf == 1.0f && m->sref_slf == 1.0f)) {
        kcos = (float *)malloc((size_t)I * hd * sizeof(float));
        ksin = (float *)malloc((size_t)I * hd * sizeof(float));
        memcpy(kcos, icos, (size_t)I * hd * sizeof(float));
        memcpy(ksin, isin, (size_t)I * hd * sizeof(float));
        orc_sref_band_scale(kcos, ksin, I0, I, ad, m->sref_shf, m->sref_slf);
    }
    /* NCHW -> NLC, :3986-3993 and :4667-4689 */
    float *tok = (float *)malloc((size_t)I * C * sizeof(float));
    for (int p = 0; p < I0; p++)
        for (int c = 0; c < C; c++) tok[(size_t)p * C + c] = latent[(size_t)c * I0 + p];
    int row = I0;
    for (int r = 0; r < n_refs; r++) {
        int rs = refs[r].h * refs[r].w;
        for (int p = 0; p < rs; p++)
            for (int c = 0; c < C; c++) tok[(size_t)(row + p) * C + c] = refs[r].latent[(size_t)c * rs + p];
        row += rs;
    }
    float *img = (float *)malloc((size_t)I * h * sizeof(float));
    float *txth = (float *)malloc((size_t)T * h * sizeof(float));
    orc_linear(img, tok, m->img_in, NULL, I, C, h);
    orc_linear(txth, txt, m->txt_in, NULL, T, m->text_dim, h);
    free(tok);
    float *dimg = (float *)malloc((size_t)6 * h * sizeof(float));
    float *dtxt = (float *)malloc((size_t)6 * h * sizeof(float));
    orc_flux_modulation(m, t_emb, dimg, dtxt, NULL, NULL);
    for (int i = 0; i < m->n_double; i++)
        orc_flux_double_block(m, i, img, txth, dimg, dtxt, icos, isin, tcos, tsin, I, T);
    float *cat = (float *)malloc((size_t)S * h * sizeof(float));       /* [txt, img], :4110-4114 */
    memcpy(cat, txth, (size_t)T * h * sizeof(float));
    memcpy(cat + (size_t)T * h, img, (size_t)I * h * sizeof(float));
    for (int i = 0; i < m->n_single; i++)
        orc_flux_single_block_k(m, i, cat, t_emb, icos, isin, kcos, ksin, tcos, tsin, S, T);
    if (kcos != icos) { free(kcos); free(ksin); }
    /* final layer, :4254-4301: (scale, shift) order */
    float *fm = (float *)malloc((size_t)2 * h * sizeof(float));
    orc_flux_modulation(m, t_emb, NULL, NULL, NULL, fm);
    float *fn = (float *)malloc((size_t)I0 * h * sizeof(float));
    adaln(fn, cat + (size_t)T * h, fm + h, fm, I0, h, 1e-6f);
    float *nlc = (float *)malloc((size_t)I0 * C * sizeof(float));
    orc_linear(nlc, fn, m->proj_out, NULL, I0, h, C);
    float *out = (float *)malloc((size_t)I0 * C * sizeof(float));
    for (int p = 0; p < I0; p++)
        for (int c = 0; c < C; c++) out[(size_t)c * I0 + p] = nlc[(size_t)p * C + c];
    free(t_emb); free(icos); free(isin); free(tcos); free(tsin); free(img); free(txth);
    free(dimg); free(dtxt); free(cat); free(fm); free(fn); free(nlc);
    return out;
}

float *orc_flux_forward(orc_flux_t *m, const float *latent, int h, int w,
                        const float *txt, int txt_seq, float t) {
    return forward_impl(m, latent, h, w, NULL, 0, txt, txt_seq, t);
}

float *orc_flux_forward_refs(orc_flux_t *m, const float *latent, int h, int w,
                             const orc_ref_t *refs, int n_refs,
                             const float *txt, int txt_seq, float t) {
    return forward_impl(m, latent, h, w, refs, n_refs, txt, txt_seq, t);
}
