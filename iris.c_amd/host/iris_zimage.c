/*
 * iris_zimage.c - Z-Image S3-DiT denoiser forward of the HIP build (host C).
 *
 * Keeps zi_transformer_load_safetensors / zi_transformer_forward /
 * zi_transformer_free (iris_transformer_zimage.c:2164, :1696) and the block
 * structure of zi_block_forward (:790-870), running every block on the device:
 *   - one f32 residual buffer holds the unified [image | caption] sequence
 *     (:1904-1907); the noise refiner runs on its image rows and the context
 *     refiner on its caption rows in place, so no concatenation copies;
 *   - padding rows (sequences padded to multiples of 32, :1769-1789) are
 *     excluded from attention by key ranges instead of a -1e9 mask (:730-737;
 *     the masked probabilities are exactly 0 either way);
 *   - the 3-axis RoPE is expanded on the host into per-row cos/sin tables from
 *     the same per-axis values (zi_precompute_rope :595-613, zi_apply_rope
 *     :620-650) and applied in the QK-norm kernel.
 * The attention output projection computes attn . Wo^T as the model defines
 * it; the reference CPU path runs that product in place over its own input
 * (tf->work_tmp is both zi_attention's scratch :716 and its output :796),
 * which its GPU path does not do.
 */
#include "../../include/iris_transformer.h"
#include "../../include/iris_hip.h"
#include "../../include/iris_synth.h"
#include "iris_st.h"
#include "iris_tables.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define ZI_EPS 1e-5f          /* iris_transformer_zimage.c:41 */
#define ZI_MULT 32            /* :40 */
#define SWIGLU_GROUP 32

typedef struct {
    uint16_t *qkv, *o, *w13, *w2, *ada_w;    /* w13: w1 (gate) / w3 (up) rows interleaved by 32 */
    float *nq, *nk, *n1, *n2, *fn1, *fn2, *ada_b;
} zi_dev_block_t;

/* split-K partials of one product on few rows (iris_hip_gemm_fill picks the
 * chunk count that fits) */
#define ZI_FILL_WS_BYTES ((size_t)64 << 20)

typedef struct {
    int valid, lh, lw, cap_len;
    int I, Ip, Cp, U, U_pad;
    float *x, *y, *rope_cos, *rope_sin, *tsin, *tmp, *temb, *mods, *fscale, *lat, *vel, *capf, *fout;
    float *rp_cos, *rp_sin;       /* [U][64]: one value per rotation pair (the attention's Q prologue) */
    uint16_t *a, *qkv, *q, *k, *vt, *attn, *ffn, *patches;
    float *tsin_host;
    void *attn_ws;                /* the attention's balanced-schedule workspace (zeroed) */
    size_t attn_ws_bytes;
    float *fill_ws;               /* split-K partials of the products on few rows (iris_hip_gemm_fill) */
    void *graph;
} zi_work_t;

struct zi_transformer {
    int dim, heads, layers, refiners, ffn, in_ch, ps, adaln_dim, cap_dim, t_mid;
    float theta;
    int axes[3], lens[3];
    uint16_t *t0_w, *t2_w, *cap_w, *x_w, *f_ada_w, *f_lin_w;
    float *t0_b, *t2_b, *cap_norm, *cap_b, *x_b, *x_pad, *cap_pad, *f_ada_b1, *f_lin_b;
    zi_dev_block_t *nr, *cr, *ly;
    /* the modulated blocks' adaLN weights [refiners + layers][4 dim][adaln_dim]
     * and biases, noise refiners first: one GEMV yields every block's
     * modulation (the blocks' ada_w / ada_b point into them) */
    uint16_t *ada_all_w;
    float *ada_all_b;
    zi_work_t w;
};

/* ------------------------------------------------------------ weight upload */

typedef struct {
    const iris_st_set_t *st;
    uint64_t seed;
    float *stage;
    size_t stage_n;
    uint16_t *stage16;
    size_t stage16_n;
} zsrc_t;

/* Host f32 copy of a tensor (exact widening of bf16 files; synthetic values as
 * a bf16 file written by the seeded generator would hold them). */
static const float *zget(zsrc_t *s, const char *name, size_t n, float mean, float std) {
    if (s->stage_n < n) {
        free(s->stage);
        s->stage = (float *)malloc(n * sizeof(float));
        s->stage_n = s->stage ? n : 0;
        if (!s->stage) return NULL;
    }
    if (s->st) {
        const iris_st_file_t *f;
        const iris_st_tensor_t *t = iris_st_set_find(s->st, name, &f);
        if (!t) { fprintf(stderr, "Z-Image: required tensor %s not found\n", name); return NULL; }
        if ((size_t)iris_st_numel(t) != n) {
            fprintf(stderr, "Z-Image: tensor %s has %lld elements, expected %zu\n", name,
                    (long long)iris_st_numel(t), n);
            return NULL;
        }
        if (iris_st_read_f32(f, t, s->stage)) return NULL;
        return s->stage;
    }
    uint64_t ts = iris_synth_seed(s->seed, name);
    iris_synth_fill_f32(s->stage, n, ts, 0, mean, std);
    for (size_t i = 0; i < n; i++) s->stage[i] = iris_bf16_to_f32(iris_f32_to_bf16(s->stage[i]));
    return s->stage;
}

static float *up_f32(zsrc_t *s, const char *name, size_t n, float mean, float std, float add) {
    const float *h = zget(s, name, n, mean, std);
    if (!h) return NULL;
    float *d = (float *)iris_hip_malloc(n * 4);
    if (!d) return NULL;
    if (add != 0.0f) {
        float *t = (float *)malloc(n * 4);
        if (!t) { iris_hip_free(d); return NULL; }
        for (size_t i = 0; i < n; i++) t[i] = h[i] + add;
        int rc = iris_hip_memcpy_h2d(d, t, n * 4) || iris_hip_sync();
        free(t);
        if (rc) { iris_hip_free(d); return NULL; }
        return d;
    }
    if (iris_hip_memcpy_h2d(d, h, n * 4) || iris_hip_sync()) { iris_hip_free(d); return NULL; }
    return d;
}

static int to_bf16_stage(zsrc_t *s, const float *h, size_t n) {
    if (s->stage16_n < n) {
        free(s->stage16);
        s->stage16 = (uint16_t *)malloc(n * 2);
        s->stage16_n = s->stage16 ? n : 0;
        if (!s->stage16) return -1;
    }
    for (size_t i = 0; i < n; i++) s->stage16[i] = iris_f32_to_bf16(h[i]);
    return 0;
}

/* bf16 device copy of rows [r0, r0 + rows) of the destination matrix */
static int up_rows(zsrc_t *s, const char *name, uint16_t *d, size_t rows, size_t cols) {
    const float *h = zget(s, name, rows * cols, 0.0f, 0.02f);
    if (!h || to_bf16_stage(s, h, rows * cols)) return -1;
    if (iris_hip_memcpy_h2d(d, s->stage16, rows * cols * 2)) return -1;
    return iris_hip_sync();
}

static uint16_t *up_bf16(zsrc_t *s, const char *name, size_t rows, size_t cols) {
    uint16_t *d = (uint16_t *)iris_hip_malloc(rows * cols * 2);
    if (!d) return NULL;
    if (up_rows(s, name, d, rows, cols)) { iris_hip_free(d); return NULL; }
    return d;
}

/* slot: the block's row in ada_all_w / ada_all_b, or -1 (unmodulated) */
static int load_block(zi_transformer_t *tf, zsrc_t *s, zi_dev_block_t *b, const char *pre, int slot) {
    size_t d = tf->dim, f = tf->ffn;
    char nm[256];
    b->qkv = (uint16_t *)iris_hip_malloc(3 * d * d * 2);
    b->w13 = (uint16_t *)iris_hip_malloc(2 * f * d * 2);
    if (!b->qkv || !b->w13) return -1;
    /* names: iris_transformer_zimage.c:2024-2075 */
    static const char *const qkv[3] = {"to_q", "to_k", "to_v"};
    for (int j = 0; j < 3; j++) {
        snprintf(nm, sizeof(nm), "%s.attention.%s.weight", pre, qkv[j]);
        if (up_rows(s, nm, b->qkv + j * d * d, d, d)) return -1;
    }
    snprintf(nm, sizeof(nm), "%s.attention.to_out.0.weight", pre);
    if (!(b->o = up_bf16(s, nm, d, d))) return -1;
    /* w1 (gate) and w3 (up) interleaved in groups of 32 rows for the SwiGLU epilogue */
    {
        const size_t G = SWIGLU_GROUP;
        for (int which = 0; which < 2; which++) {
            snprintf(nm, sizeof(nm), "%s.feed_forward.%s.weight", pre, which ? "w3" : "w1");
            const float *h = zget(s, nm, f * d, 0.0f, 0.02f);
            if (!h || to_bf16_stage(s, h, f * d)) return -1;
            for (size_t g = 0; g < f / G; g++)
                if (iris_hip_memcpy_h2d(b->w13 + (2 * g + which) * G * d, s->stage16 + g * G * d, G * d * 2)) return -1;
            if (iris_hip_sync()) return -1;
        }
    }
    snprintf(nm, sizeof(nm), "%s.feed_forward.w2.weight", pre);
    if (!(b->w2 = up_bf16(s, nm, d, f))) return -1;
#define NORM(dst, suf, n) do { snprintf(nm, sizeof(nm), "%s.%s", pre, suf); \
        if (!((dst) = up_f32(s, nm, (n), 1.0f, 0.02f, 0.0f))) return -1; } while (0)
    NORM(b->nq, "attention.norm_q.weight", 128);
    NORM(b->nk, "attention.norm_k.weight", 128);
    NORM(b->n1, "attention_norm1.weight", d);
    NORM(b->n2, "attention_norm2.weight", d);
    NORM(b->fn1, "ffn_norm1.weight", d);
    NORM(b->fn2, "ffn_norm2.weight", d);
#undef NORM
    if (slot >= 0) {
        snprintf(nm, sizeof(nm), "%s.adaLN_modulation.0.weight", pre);
        b->ada_w = tf->ada_all_w + (size_t)slot * 4 * d * tf->adaln_dim;
        if (up_rows(s, nm, b->ada_w, 4 * d, tf->adaln_dim)) return -1;
        /* bias with 1 folded into the two scale segments: the GEMV then yields
         * 1 + scale_msa and 1 + scale_mlp directly (:809-816) */
        snprintf(nm, sizeof(nm), "%s.adaLN_modulation.0.bias", pre);
        const float *h = zget(s, nm, 4 * d, 0.0f, 0.02f);
        if (!h) return -1;
        float *t = (float *)malloc(4 * d * 4);
        if (!t) return -1;
        for (size_t i = 0; i < 4 * d; i++) t[i] = h[i] + ((i < d || (i >= 2 * d && i < 3 * d)) ? 1.0f : 0.0f);
        b->ada_b = tf->ada_all_b + (size_t)slot * 4 * d;
        int rc = iris_hip_memcpy_h2d(b->ada_b, t, 4 * d * 4) || iris_hip_sync();
        free(t);
        if (rc) return -1;
    }
    return 0;
}

static void free_block(zi_dev_block_t *b) {
    void *p[] = {b->qkv, b->o, b->w13, b->w2, b->nq, b->nk, b->n1, b->n2, b->fn1, b->fn2};
    for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) iris_hip_free(p[i]);
}

static void zwork_free(zi_work_t *w);

void zi_transformer_free(zi_transformer_t *tf) {
    if (!tf) return;
    zwork_free(&tf->w);
    void *p[] = {tf->t0_w, tf->t2_w, tf->cap_w, tf->x_w, tf->f_ada_w, tf->f_lin_w, tf->t0_b, tf->t2_b, tf->cap_norm,
                 tf->cap_b, tf->x_b, tf->x_pad, tf->cap_pad, tf->f_ada_b1, tf->f_lin_b, tf->ada_all_w, tf->ada_all_b};
    for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) iris_hip_free(p[i]);
    for (int i = 0; tf->nr && i < tf->refiners; i++) free_block(&tf->nr[i]);
    for (int i = 0; tf->cr && i < tf->refiners; i++) free_block(&tf->cr[i]);
    for (int i = 0; tf->ly && i < tf->layers; i++) free_block(&tf->ly[i]);
    free(tf->nr); free(tf->cr); free(tf->ly);
    free(tf);
}

static int load_all(zi_transformer_t *tf, zsrc_t *s) {
    size_t d = tf->dim, ad = tf->adaln_dim, pf = (size_t)tf->ps * tf->ps * tf->in_ch;
    char nm[256];
    /* names: iris_transformer_zimage.c:2290-2395 */
    if (!(tf->t0_w = up_bf16(s, "t_embedder.mlp.0.weight", tf->t_mid, 256))) return -1;
    if (!(tf->t0_b = up_f32(s, "t_embedder.mlp.0.bias", tf->t_mid, 0.0f, 0.02f, 0.0f))) return -1;
    if (!(tf->t2_w = up_bf16(s, "t_embedder.mlp.2.weight", ad, tf->t_mid))) return -1;
    if (!(tf->t2_b = up_f32(s, "t_embedder.mlp.2.bias", ad, 0.0f, 0.02f, 0.0f))) return -1;
    if (!(tf->cap_norm = up_f32(s, "cap_embedder.0.weight", tf->cap_dim, 1.0f, 0.02f, 0.0f))) return -1;
    if (!(tf->cap_w = up_bf16(s, "cap_embedder.1.weight", d, tf->cap_dim))) return -1;
    if (!(tf->cap_b = up_f32(s, "cap_embedder.1.bias", d, 0.0f, 0.02f, 0.0f))) return -1;
    snprintf(nm, sizeof(nm), "all_x_embedder.%d-1.weight", tf->ps);
    if (!(tf->x_w = up_bf16(s, nm, d, pf))) return -1;
    snprintf(nm, sizeof(nm), "all_x_embedder.%d-1.bias", tf->ps);
    if (!(tf->x_b = up_f32(s, nm, d, 0.0f, 0.02f, 0.0f))) return -1;
    if (!(tf->x_pad = up_f32(s, "x_pad_token", d, 0.0f, 1.0f, 0.0f))) return -1;
    if (!(tf->cap_pad = up_f32(s, "cap_pad_token", d, 0.0f, 1.0f, 0.0f))) return -1;
    tf->nr = (zi_dev_block_t *)calloc((size_t)tf->refiners, sizeof(zi_dev_block_t));
    tf->cr = (zi_dev_block_t *)calloc((size_t)tf->refiners, sizeof(zi_dev_block_t));
    tf->ly = (zi_dev_block_t *)calloc((size_t)tf->layers, sizeof(zi_dev_block_t));
    if (!tf->nr || !tf->cr || !tf->ly) return -1;
    const size_t nmod = (size_t)tf->refiners + tf->layers;
    tf->ada_all_w = (uint16_t *)iris_hip_malloc(nmod * 4 * d * ad * 2);
    tf->ada_all_b = (float *)iris_hip_malloc(nmod * 4 * d * 4);
    if (!tf->ada_all_w || !tf->ada_all_b) return -1;
    for (int i = 0; i < tf->refiners; i++) {
        snprintf(nm, sizeof(nm), "noise_refiner.%d", i);
        if (load_block(tf, s, &tf->nr[i], nm, i)) return -1;
        snprintf(nm, sizeof(nm), "context_refiner.%d", i);
        if (load_block(tf, s, &tf->cr[i], nm, -1)) return -1;
    }
    for (int i = 0; i < tf->layers; i++) {
        snprintf(nm, sizeof(nm), "layers.%d", i);
        if (load_block(tf, s, &tf->ly[i], nm, tf->refiners + i)) return -1;
    }
    snprintf(nm, sizeof(nm), "all_final_layer.%d-1.adaLN_modulation.1.weight", tf->ps);
    if (!(tf->f_ada_w = up_bf16(s, nm, d, ad))) return -1;
    /* final scale = 1 + W silu(t) + b (:1563-1574): the 1 is folded into the bias */
    snprintf(nm, sizeof(nm), "all_final_layer.%d-1.adaLN_modulation.1.bias", tf->ps);
    if (!(tf->f_ada_b1 = up_f32(s, nm, d, 0.0f, 0.02f, 1.0f))) return -1;
    snprintf(nm, sizeof(nm), "all_final_layer.%d-1.linear.weight", tf->ps);
    if (!(tf->f_lin_w = up_bf16(s, nm, pf, d))) return -1;
    snprintf(nm, sizeof(nm), "all_final_layer.%d-1.linear.bias", tf->ps);
    if (!(tf->f_lin_b = up_f32(s, nm, pf, 0.0f, 0.02f, 0.0f))) return -1;
    return 0;
}

static zi_transformer_t *zi_init(int dim, int heads, int layers, int refiners, int cap_dim, int in_ch, int ps,
                                 float theta, const int *axes) {
    /* zi_transformer_load_safetensors, iris_transformer_zimage.c:2164-2190 */
    if (!iris_hip_available()) {
        fprintf(stderr, "Z-Image: no usable HIP device: %s\n", iris_hip_last_error());
        return NULL;
    }
    if (dim / heads != 128 || axes[0] + axes[1] + axes[2] != 128) {
        fprintf(stderr, "Z-Image: head_dim 128 with axes summing to 128 required\n");
        return NULL;
    }
    zi_transformer_t *tf = (zi_transformer_t *)calloc(1, sizeof(*tf));
    if (!tf) return NULL;
    tf->dim = dim; tf->heads = heads; tf->layers = layers; tf->refiners = refiners;
    tf->ffn = (8 * dim / 3 + 255) / 256 * 256; tf->in_ch = in_ch; tf->ps = ps;
    tf->adaln_dim = dim < 256 ? dim : 256; tf->theta = theta; tf->cap_dim = cap_dim; tf->t_mid = 1024;
    for (int i = 0; i < 3; i++) { tf->axes[i] = axes[i]; tf->lens[i] = 1024; }
    return tf;
}

static int zi_check(const zi_transformer_t *tf) {
    int pf = tf->ps * tf->ps * tf->in_ch;
    if (tf->dim % 64 || tf->cap_dim % 64 || pf % 64 || tf->ffn % 32 || tf->t_mid % 8 || tf->adaln_dim % 64 ||
        tf->dim > 4096 || tf->cap_dim > 4096) {
        fprintf(stderr, "Z-Image: unsupported dims (dim %d cap %d patch %d ffn %d)\n", tf->dim, tf->cap_dim, pf, tf->ffn);
        return -1;
    }
    return 0;
}

static zi_transformer_t *zi_finish(zi_transformer_t *tf, zsrc_t *s) {
    int rc = zi_check(tf) || load_all(tf, s);
    free(s->stage);
    free(s->stage16);
    if (rc) {
        fprintf(stderr, "Z-Image: weight upload failed: %s\n", iris_hip_last_error());
        zi_transformer_free(tf);
        return NULL;
    }
    return tf;
}

zi_transformer_t *zi_transformer_load_safetensors(const char *model_dir, int dim, int n_heads, int n_layers,
                                                  int n_refiner, int cap_feat_dim, int in_channels, int patch_size,
                                                  float rope_theta, const int *axes_dims) {
    zi_transformer_t *tf = zi_init(dim, n_heads, n_layers, n_refiner, cap_feat_dim, in_channels, patch_size,
                                   rope_theta, axes_dims);
    if (!tf) return NULL;
    iris_st_set_t st;
    if (iris_st_set_open(&st, model_dir)) {
        fprintf(stderr, "Z-Image: failed to open transformer safetensors\n");
        free(tf);
        return NULL;
    }
    const iris_st_tensor_t *t = iris_st_set_find(&st, "layers.0.feed_forward.w1.weight", NULL);
    if (t) tf->ffn = (int)t->shape[0];           /* ffn_dim probe, :2271-2277 */
    t = iris_st_set_find(&st, "t_embedder.mlp.0.weight", NULL);
    if (t) tf->t_mid = (int)t->shape[0];         /* :2279-2284 */
    zsrc_t s = {&st, 0, NULL, 0, NULL, 0};
    tf = zi_finish(tf, &s);
    iris_st_set_close(&st);
    return tf;
}

zi_transformer_t *zi_transformer_create_synthetic(int dim, int n_heads, int n_layers, int n_refiner,
                                                  int cap_feat_dim, int in_channels, int patch_size, float rope_theta,
                                                  const int *axes_dims, int ffn_dim, int t_mid, uint64_t seed) {
    zi_transformer_t *tf = zi_init(dim, n_heads, n_layers, n_refiner, cap_feat_dim, in_channels, patch_size,
                                   rope_theta, axes_dims);
    if (!tf) return NULL;
    if (ffn_dim > 0) tf->ffn = ffn_dim;
    if (t_mid > 0) tf->t_mid = t_mid;
    zsrc_t s = {NULL, seed, NULL, 0, NULL, 0};
    return zi_finish(tf, &s);
}

/* -------------------------------------------------------------- workspace */

static void zwork_free(zi_work_t *w) {
    iris_hip_graph_destroy(w->graph);
    void *p[] = {w->x, w->y, w->rope_cos, w->rope_sin, w->rp_cos, w->rp_sin, w->tsin, w->tmp, w->temb, w->mods, w->fscale, w->lat, w->vel,
                 w->capf, w->fout, w->a, w->qkv, w->q, w->k, w->vt, w->attn, w->ffn, w->patches, w->attn_ws, w->fill_ws};
    for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) iris_hip_free(p[i]);
    free(w->tsin_host);
    memset(w, 0, sizeof(*w));
}

static int zi_enqueue(zi_transformer_t *tf);

int zi_prepare(zi_transformer_t *tf, int lh, int lw, int cap_len) {
    zi_work_t *w = &tf->w;
    if (lh <= 0 || lw <= 0 || cap_len <= 0 || lh % tf->ps || lw % tf->ps) {
        fprintf(stderr, "Z-Image: bad geometry %dx%d cap %d\n", lh, lw, cap_len);
        return -1;
    }
    if (w->valid && w->lh == lh && w->lw == lw && w->cap_len == cap_len) return 0;
    zwork_free(w);
    int d = tf->dim, H = tf->heads, pf = tf->ps * tf->ps * tf->in_ch;
    int Ht = lh / tf->ps, Wt = lw / tf->ps;
    w->lh = lh; w->lw = lw; w->cap_len = cap_len;
    w->I = Ht * Wt;
    w->Ip = w->I + (ZI_MULT - w->I % ZI_MULT) % ZI_MULT;            /* :1736-1741 */
    w->Cp = cap_len + (ZI_MULT - cap_len % ZI_MULT) % ZI_MULT;
    w->U = w->Ip + w->Cp;
    w->U_pad = (w->U + 63) / 64 * 64;
    size_t U = w->U, nmod = (size_t)(tf->refiners + tf->layers);
    size_t acols = d > tf->cap_dim ? d : tf->cap_dim;
#define DA(dst, bytes) do { if (!((dst) = iris_hip_malloc(bytes))) goto fail; } while (0)
    DA(w->x, U * d * 4);
    DA(w->y, U * d * 4);
    DA(w->rope_cos, U * 128 * 4);
    DA(w->rp_cos, U * 64 * 4);
    DA(w->rp_sin, U * 64 * 4);
    DA(w->rope_sin, U * 128 * 4);
    DA(w->tsin, 256 * 4);
    DA(w->tmp, (size_t)tf->t_mid * 4);
    DA(w->temb, 256 * 4);
    DA(w->mods, nmod * 4 * d * 4);
    DA(w->fscale, (size_t)d * 4);
    DA(w->lat, (size_t)tf->in_ch * lh * lw * 4);
    DA(w->vel, (size_t)tf->in_ch * lh * lw * 4);
    DA(w->capf, (size_t)cap_len * tf->cap_dim * 4);
    DA(w->fout, (size_t)w->I * pf * 4);
    DA(w->a, U * acols * 2);
    DA(w->qkv, U * 3 * d * 2);
    DA(w->q, U * d * 2);
    DA(w->k, U * d * 2);
    DA(w->vt, (size_t)H * 128 * w->U_pad * 2);
    DA(w->attn, U * d * 2);
    DA(w->ffn, U * tf->ffn * 2);
    DA(w->patches, (size_t)w->I * pf * 2);
    DA(w->fill_ws, ZI_FILL_WS_BYTES);
    w->attn_ws_bytes = iris_hip_attention_workspace_bytes();
    DA(w->attn_ws, w->attn_ws_bytes);
    if (iris_hip_memset(w->attn_ws, 0, w->attn_ws_bytes) || iris_hip_sync()) goto fail;
#undef DA
    w->tsin_host = (float *)malloc(256 * sizeof(float));
    if (!w->tsin_host) goto fail;
    {
        /* position ids (:1830-1862): image (Cp + 1, h, w), padding (0, 0, 0),
         * caption (1 + s, 0, 0) for every padded caption row */
        int *pos = (int *)calloc(U * 3, sizeof(int));
        float *c = (float *)malloc(U * 128 * 4), *s = (float *)malloc(U * 128 * 4);
        if (!pos || !c || !s) { free(pos); free(c); free(s); goto fail; }
        for (int i = 0; i < w->I; i++) {
            pos[i * 3] = w->Cp + 1; pos[i * 3 + 1] = i / Wt; pos[i * 3 + 2] = i % Wt;
        }
        for (int j = 0; j < w->Cp; j++) pos[(w->Ip + j) * 3] = 1 + j;
        iris_rope_zimage(c, s, pos, (int)U, tf->axes, tf->lens, tf->theta);
        float *pc = (float *)malloc(U * 64 * 4), *ps = (float *)malloc(U * 64 * 4);
        int rc = !pc || !ps;
        if (!rc) iris_rope_pairs(pc, ps, c, s, U);
        rc = rc || iris_hip_memcpy_h2d(w->rope_cos, c, U * 128 * 4) || iris_hip_memcpy_h2d(w->rope_sin, s, U * 128 * 4) ||
             iris_hip_memcpy_h2d(w->rp_cos, pc, U * 64 * 4) || iris_hip_memcpy_h2d(w->rp_sin, ps, U * 64 * 4) ||
             iris_hip_sync();
        free(pos); free(c); free(s); free(pc); free(ps);
        if (rc) goto fail;
    }
    w->valid = 1;
    if (iris_hip_graph_begin()) goto fail;
    if (zi_enqueue(tf)) {
        iris_hip_graph_destroy(iris_hip_graph_end());
        goto fail;
    }
    if (!(w->graph = iris_hip_graph_end())) goto fail;
    return 0;
fail:
    fprintf(stderr, "zi_prepare: %s\n", iris_hip_last_error());
    zwork_free(w);
    return -1;
}

/* ------------------------------------------------------------- the forward */

#define CK(x) do { if ((x) != 0) return -1; } while (0)

static iris_gemm_problem_t zprob(const void *A, int lda, const uint16_t *W, void *out, int ldo, const float *vec,
                                 int M, int N, int K, int epi) {
    iris_gemm_problem_t p;
    memset(&p, 0, sizeof(p));
    p.A = (const uint16_t *)A; p.lda = lda; p.W = W; p.ldw = K; p.out = out; p.ldo = ldo; p.vec = vec;
    p.M = M; p.N = N; p.K = K; p.epi = epi;
    return p;
}

/* one product: split over K through the forward's workspace when its tiles
 * leave most of the chip idle (the context refiner's 512 caption rows, the
 * caption embedder, the final projection), else the plain launch */
static int zgemm(zi_transformer_t *tf, const iris_gemm_problem_t *p) {
    return iris_hip_gemm_fill(p, tf->w.fill_ws, ZI_FILL_WS_BYTES);
}

static int rms(zi_transformer_t *tf, const float *x, uint16_t *out, int rows, const float *w, const float *scale) {
    iris_norm_args_t a;
    memset(&a, 0, sizeof(a));
    a.x = x; a.ldx = tf->dim; a.out = out; a.ldo = tf->dim; a.out_bf16 = 1;
    a.rows = rows; a.cols = tf->dim; a.mode = IRIS_NORM_RMS; a.eps = ZI_EPS;
    a.split = rows; a.wA = w; a.scaleA = scale;
    return iris_hip_rownorm(&a);
}

/* zi_block_forward (:790-870) on rows [r0, r0 + n) of the unified sequence;
 * keys outside [klo0, khi0) U [klo1, khi1) (relative to r0) are padding. mod
 * is NULL for the unmodulated context refiner, else 1+scale_msa | gate_msa |
 * 1+scale_mlp | gate_mlp, the gates already through tanh (iris_hip_tanh_cols
 * after the modulation GEMV). */
static int zi_block_forward(zi_transformer_t *tf, const zi_dev_block_t *b, const float *mod, int r0, int n,
                            int klo0, int khi0, int klo1, int khi1) {
    zi_work_t *w = &tf->w;
    int d = tf->dim, f = tf->ffn;
    float *x = w->x + (size_t)r0 * d;
    /* attention: h = attention(norm1(x) * (1 + scale_msa)) */
    CK(rms(tf, x, w->a, n, b->n1, mod));
    iris_gemm_problem_t p = zprob(w->a, d, b->qkv, w->qkv, 3 * d, NULL, n, 3 * d, d, IRIS_EPI_BF16);
    CK(zgemm(tf, &p));
    iris_qkprep_args_t q;
    memset(&q, 0, sizeof(q));
    q.qkv = w->qkv; q.ld_qkv = 3 * d; q.col_k = d; q.col_v = 2 * d;
    q.k_out = w->k; q.vt_out = w->vt; q.ld_vt = w->U_pad;
    q.rows = n; q.heads = tf->heads;
    q.wkA = b->nk; q.wkB = b->nk; q.split = n;
    q.cos_t = w->rope_cos + (size_t)r0 * 128; q.sin_t = w->rope_sin + (size_t)r0 * 128;
    q.eps = ZI_EPS;
    CK(iris_hip_kv_prepare(&q));
    /* Q: zi_qk_norm + zi_apply_rope in the attention kernel's prologue */
    iris_attn_args_t at;
    memset(&at, 0, sizeof(at));
    at.q = w->qkv; at.k = w->k; at.vt = w->vt; at.o = w->attn;
    at.ld_q = 3 * d; at.ld_k = d; at.ld_vt = w->U_pad; at.ld_o = d;
    at.sq = n; at.sk = n; at.heads = tf->heads; at.batch = 1;
    at.scale = 1.0f / sqrtf(128.0f);
    at.kv_lo0 = klo0; at.kv_hi0 = khi0; at.kv_lo1 = klo1; at.kv_hi1 = khi1;
    at.qn_wA = b->nq; at.qn_wB = b->nq; at.qn_split = n; at.qn_eps = ZI_EPS;
    at.rope_cos = w->rp_cos + (size_t)r0 * 64; at.rope_sin = w->rp_sin + (size_t)r0 * 64;
    at.ws = w->attn_ws; at.ws_bytes = w->attn_ws_bytes;
    CK(iris_hip_attention(&at));
    p = zprob(w->attn, d, b->o, w->y, d, NULL, n, d, d, IRIS_EPI_F32);
    CK(zgemm(tf, &p));
    /* x += tanh(gate_msa) * norm2(attn_out) */
    CK(iris_hip_rms_gated_add(x, w->y, b->n2, mod ? mod + d : NULL, n, d, ZI_EPS, 0));
    /* FFN: x += tanh(gate_mlp) * norm2(w2(silu(w1 h) * w3 h)), h = norm1(x) * (1 + scale_mlp) */
    CK(rms(tf, x, w->a, n, b->fn1, mod ? mod + 2 * d : NULL));
    p = zprob(w->a, d, b->w13, w->ffn, f, NULL, n, 2 * f, d, IRIS_EPI_SWIGLU);
    CK(zgemm(tf, &p));
    p = zprob(w->ffn, f, b->w2, w->y, d, NULL, n, d, f, IRIS_EPI_F32);
    CK(zgemm(tf, &p));
    CK(iris_hip_rms_gated_add(x, w->y, b->fn2, mod ? mod + 3 * d : NULL, n, d, ZI_EPS, 0));
    return 0;
}

static int zi_enqueue(zi_transformer_t *tf) {
    zi_work_t *w = &tf->w;
    int d = tf->dim, pf = tf->ps * tf->ps * tf->in_ch, I = w->I, Ip = w->Ip, Cp = w->Cp, U = w->U;
    /* timestep MLP with biases (:561-584) */
    CK(iris_hip_gemv(w->tmp, tf->t0_w, w->tsin, tf->t0_b, tf->t_mid, 256, 0));
    CK(iris_hip_gemv(w->temb, tf->t2_w, w->tmp, tf->t2_b, tf->adaln_dim, tf->t_mid, 1));
    /* per-block modulation W t_emb + b, no SiLU (:806-807), for every
     * modulated block in one GEMV over their stacked weights; final scale
     * 1 + W SiLU(t_emb) + b (:1563-1574) */
    CK(iris_hip_gemv(w->mods, tf->ada_all_w, w->temb, tf->ada_all_b, (tf->refiners + tf->layers) * 4 * d,
                     tf->adaln_dim, 0));
    /* tanh of the gate columns ([d, 2d) and [3d, 4d) of each block's 4d),
     * once: viewed as rows of 2d, the gates are columns [d, 2d) of each */
    CK(iris_hip_tanh_cols(w->mods, 2 * (tf->refiners + tf->layers), 2 * d, d, d));
    CK(iris_hip_gemv(w->fscale, tf->f_ada_w, w->temb, tf->f_ada_b1, d, tf->adaln_dim, 1));
    /* patchify (ph, pw, c) and embed image rows [0, I); padding rows get x_pad_token */
    CK(iris_hip_patchify(w->patches, w->lat, tf->in_ch, w->lh, w->lw, tf->ps));
    iris_gemm_problem_t p = zprob(w->patches, pf, tf->x_w, w->x, d, tf->x_b, I, d, pf, IRIS_EPI_F32);
    CK(zgemm(tf, &p));
    CK(iris_hip_fill_rows(w->x, tf->x_pad, I, Ip, d));
    /* caption: RMSNorm * w then linear + b into rows [Ip, Ip + cap_len); padding rows get cap_pad_token */
    iris_norm_args_t a;
    memset(&a, 0, sizeof(a));
    a.x = w->capf; a.ldx = tf->cap_dim; a.out = w->a; a.ldo = tf->cap_dim; a.out_bf16 = 1;
    a.rows = w->cap_len; a.cols = tf->cap_dim; a.mode = IRIS_NORM_RMS; a.eps = ZI_EPS;
    a.split = w->cap_len; a.wA = tf->cap_norm;
    CK(iris_hip_rownorm(&a));
    p = zprob(w->a, tf->cap_dim, tf->cap_w, w->x + (size_t)Ip * d, d, tf->cap_b, w->cap_len, d, tf->cap_dim,
              IRIS_EPI_F32);
    CK(zgemm(tf, &p));
    CK(iris_hip_fill_rows(w->x, tf->cap_pad, Ip + w->cap_len, U, d));
    /* refiners: noise refiner on image rows, context refiner on caption rows */
    for (int i = 0; i < tf->refiners; i++)
        CK(zi_block_forward(tf, &tf->nr[i], w->mods + (size_t)i * 4 * d, 0, Ip, 0, I, 0, 0));
    for (int i = 0; i < tf->refiners; i++)
        CK(zi_block_forward(tf, &tf->cr[i], NULL, Ip, Cp, 0, w->cap_len, 0, 0));
    /* main layers on the unified [image | caption] sequence */
    for (int i = 0; i < tf->layers; i++)
        CK(zi_block_forward(tf, &tf->ly[i], w->mods + (size_t)(tf->refiners + i) * 4 * d, 0, U, 0, I, Ip,
                            Ip + w->cap_len));
    /* final layer on the image rows: LayerNorm (eps 1e-6) * scale, linear + b, unpatchify */
    memset(&a, 0, sizeof(a));
    a.x = w->x; a.ldx = d; a.out = w->a; a.ldo = d; a.out_bf16 = 1;
    a.rows = I; a.cols = d; a.mode = IRIS_NORM_LN_SCALE; a.eps = 1e-6f;
    a.split = I; a.scaleA = w->fscale;
    CK(iris_hip_rownorm(&a));
    p = zprob(w->a, d, tf->f_lin_w, w->fout, pf, tf->f_lin_b, I, pf, d, IRIS_EPI_F32);
    CK(zgemm(tf, &p));
    CK(iris_hip_unpatchify(w->vel, w->fout, tf->in_ch, w->lh, w->lw, tf->ps));
    return 0;
}

/* One block outside the captured graph (the forward's rows, masks and
 * modulation GEMV for that block). */
int zi_block_forward_resident(zi_transformer_t *tf, int kind, int idx) {
    zi_work_t *w = &tf->w;
    const int d = tf->dim;
    if (!w->valid || kind < 0 || kind > 2 || idx < 0 || idx >= (kind == 2 ? tf->layers : tf->refiners)) return -1;
    if (kind == 1) {
        if (zi_block_forward(tf, &tf->cr[idx], NULL, w->Ip, w->Cp, 0, w->cap_len, 0, 0)) return -1;
        return iris_hip_sync();
    }
    const zi_dev_block_t *b = kind == 0 ? &tf->nr[idx] : &tf->ly[idx];
    float *mod = w->mods + (size_t)(kind == 0 ? idx : tf->refiners + idx) * 4 * d;
    if (iris_hip_gemv(mod, b->ada_w, w->temb, b->ada_b, 4 * d, tf->adaln_dim, 0)) return -1;
    if (iris_hip_tanh_cols(mod, 2, 2 * d, d, d)) return -1;
    if (kind == 0 ? zi_block_forward(tf, b, mod, 0, w->Ip, 0, w->I, 0, 0)
                  : zi_block_forward(tf, b, mod, 0, w->U, 0, w->I, w->Ip, w->Ip + w->cap_len))
        return -1;
    return iris_hip_sync();
}

/* -------------------------------------------------------- step entry points */

int zi_upload(zi_transformer_t *tf, const float *latent, const float *cap) {
    zi_work_t *w = &tf->w;
    if (!w->valid) return -1;
    if (latent && iris_hip_memcpy_h2d(w->lat, latent, (size_t)tf->in_ch * w->lh * w->lw * 4)) return -1;
    if (cap && iris_hip_memcpy_h2d(w->capf, cap, (size_t)w->cap_len * tf->cap_dim * 4)) return -1;
    return iris_hip_sync();
}

int zi_velocity(zi_transformer_t *tf, float timestep) {
    zi_work_t *w = &tf->w;
    if (!w->valid) return -1;
    iris_timestep_sincos(w->tsin_host, timestep * 1000.0f, 256, 10000.0f);   /* :550-556 */
    if (iris_hip_memcpy_h2d(w->tsin, w->tsin_host, 256 * 4)) return -1;
    /* profiled: the same launches one by one, each timed */
    if (iris_hip_profile_enabled()) return zi_enqueue(tf);
    return iris_hip_graph_launch(w->graph);
}

/* iris_sample_euler_zimage update (:456-474): v at timestep 1 - sigma, z += dt * (-v) */
int zi_step(zi_transformer_t *tf, float sigma, float sigma_next) {
    if (zi_velocity(tf, 1.0f - sigma)) return -1;
    return iris_hip_euler(tf->w.lat, tf->w.vel, NULL, 0.0f, sigma_next - sigma, -1.0f,
                          (size_t)tf->in_ch * tf->w.lh * tf->w.lw);
}

int zi_download_latent(zi_transformer_t *tf, float *latent) {
    return iris_hip_memcpy_d2h(latent, tf->w.lat, (size_t)tf->in_ch * tf->w.lh * tf->w.lw * 4);
}

void *zi_device_buffer(zi_transformer_t *tf, const char *name) {
    zi_work_t *w = &tf->w;
    if (!strcmp(name, "x")) return w->x;
    if (!strcmp(name, "latent")) return w->lat;
    if (!strcmp(name, "velocity")) return w->vel;
    if (!strcmp(name, "rope_cos")) return w->rope_cos;
    if (!strcmp(name, "rope_sin")) return w->rope_sin;
    if (!strcmp(name, "t_emb")) return w->temb;
    if (!strcmp(name, "patches")) return w->patches;
    if (!strcmp(name, "a")) return w->a;
    if (!strcmp(name, "qkv")) return w->qkv;
    if (!strcmp(name, "cat")) return w->ffn;
    return NULL;
}

float *zi_transformer_forward(zi_transformer_t *tf, const float *latent, int latent_h, int latent_w, float timestep,
                              const float *cap_feats, int cap_seq_len) {
    if (!tf || !latent || !cap_feats) return NULL;
    if (zi_prepare(tf, latent_h, latent_w, cap_seq_len) || zi_upload(tf, latent, cap_feats) ||
        zi_velocity(tf, timestep))
        return NULL;
    size_t n = (size_t)tf->in_ch * latent_h * latent_w;
    float *out = (float *)malloc(n * sizeof(float));
    if (!out) return NULL;
    if (iris_hip_memcpy_d2h(out, tf->w.vel, n * sizeof(float))) {
        fprintf(stderr, "zi_transformer_forward: %s\n", iris_hip_last_error());
        free(out);
        return NULL;
    }
    return out;
}
