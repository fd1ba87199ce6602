/*
 * orc_vae.c - f32 CPU restatement of the reference's VAE decoder and encoder
 * (TEST INFRASTRUCTURE ONLY: the reference for the GPU VAE in the tests, never shipped).
 *
 * Follows iris_vae.c of the reference: iris_vae_decode (:835-998),
 * iris_vae_encode (:363-482),
 * resblock_forward (:203-251), attnblock_forward (:260-357), and the weight
 * naming of iris_vae_load_safetensors_ex (:1227-1386); planar NCHW f32 like
 * the reference. GroupNorm follows iris_group_norm (iris_kernels.c:542-582)
 * with float64 sums (the reference sums in f32); swish and softmax use the
 * reference's fast_expf (orc_silu, orc_softmax).
 */
#include "iris_oracle.h"
#include "orc_internal.h"
#include "../include/iris_synth.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static const int ch_mult[4] = {1, 2, 4, 4};

typedef struct {
    float *n1g, *n1b, *c1, *c1b, *n2g, *n2b, *c2, *c2b, *sk, *skb;
    int cin, cout;
} ores_t;

typedef struct {
    float *g, *b, *qw, *qb, *kw, *kb, *vw, *vb, *ow, *ob;
} oattn_t;

struct orc_vae {
    int z, lc;
    float eps, scaling, shift;
    float *bn_mean, *bn_var, *pqw, *pqb;
    float *cin_w, *cin_b;
    ores_t mid1, mid2, up[12];
    oattn_t attn;
    float *ups_w[3], *ups_b[3];
    float *no_g, *no_b, *co_w, *co_b;
    /* encoder */
    int has_enc;
    float *e_cin_w, *e_cin_b, *e_ds_w[3], *e_ds_b[3], *e_no_g, *e_no_b, *e_co_w, *e_co_b, *qcw, *qcb;
    ores_t e_down[8], e_mid1, e_mid2;
    oattn_t e_attn;
};

static void free_attn(oattn_t *a) {
    float *q[] = {a->g, a->b, a->qw, a->qb, a->kw, a->kb, a->vw, a->vb, a->ow, a->ob};
    for (size_t i = 0; i < sizeof(q) / sizeof(q[0]); i++) free(q[i]);
}

typedef struct {
    iris_st_file_t *f;
    uint64_t seed;
    int bad;
} osrc_t;

static float *get(osrc_t *s, const char *name, size_t n, int fan_in) {
    float *h = (float *)malloc(n * sizeof(float));
    if (!h) { s->bad = 1; return NULL; }
    if (s->f) {
        const iris_st_tensor_t *t = iris_st_find(s->f, name);
        if (!t || (size_t)iris_st_numel(t) != n || iris_st_read_f32(s->f, t, h)) {
            fprintf(stderr, "orc_vae: tensor %s missing or wrong size\n", name);
            free(h);
            s->bad = 1;
            return NULL;
        }
        return h;
    }
    float mean, std;
    iris_synth_vae_stats(name, fan_in, &mean, &std);
    iris_synth_fill_f32(h, n, iris_synth_seed(s->seed, name), 0, mean, std);
    return h;
}

static int has(osrc_t *s, const char *name) { return !s->f || iris_st_find(s->f, name) != NULL; }

static void load_attn(osrc_t *s, oattn_t *a, const char *p);

/* load_resblock_sf (iris_vae.c:1140-1182) */
static void load_res(osrc_t *s, ores_t *r, const char *p, int cin, int cout) {
    char n[256];
    r->cin = cin;
    r->cout = cout;
#define G(field, suffix, count, fan)                               \
    do {                                                           \
        snprintf(n, sizeof(n), "%s.%s", p, suffix);                \
        r->field = get(s, n, count, fan);                          \
    } while (0)
    G(n1g, "norm1.weight", cin, 0);
    G(n1b, "norm1.bias", cin, 0);
    G(c1, "conv1.weight", (size_t)cout * cin * 9, cin * 9);
    G(c1b, "conv1.bias", cout, 0);
    G(n2g, "norm2.weight", cout, 0);
    G(n2b, "norm2.bias", cout, 0);
    G(c2, "conv2.weight", (size_t)cout * cout * 9, cout * 9);
    G(c2b, "conv2.bias", cout, 0);
    if (cin != cout) {
        G(sk, "conv_shortcut.weight", (size_t)cout * cin, cin);
        G(skb, "conv_shortcut.bias", cout, 0);
    }
#undef G
}

static void free_res(ores_t *r) {
    float *p[] = {r->n1g, r->n1b, r->c1, r->c1b, r->n2g, r->n2b, r->c2, r->c2b, r->sk, r->skb};
    for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) free(p[i]);
}

void orc_vae_free(orc_vae_t *v) {
    if (!v) return;
    free_res(&v->mid1);
    free_res(&v->mid2);
    for (int i = 0; i < 12; i++) free_res(&v->up[i]);
    for (int i = 0; i < 8; i++) free_res(&v->e_down[i]);
    free_res(&v->e_mid1);
    free_res(&v->e_mid2);
    free_attn(&v->attn);
    free_attn(&v->e_attn);
    float *p[] = {v->bn_mean, v->bn_var, v->pqw, v->pqb, v->cin_w, v->cin_b, v->no_g, v->no_b, v->co_w, v->co_b,
                  v->ups_w[0], v->ups_w[1], v->ups_w[2], v->ups_b[0], v->ups_b[1], v->ups_b[2], v->e_cin_w,
                  v->e_cin_b, v->e_ds_w[0], v->e_ds_w[1], v->e_ds_w[2], v->e_ds_b[0], v->e_ds_b[1], v->e_ds_b[2],
                  v->e_no_g, v->e_no_b, v->e_co_w, v->e_co_b, v->qcw, v->qcb};
    for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) free(p[i]);
    free(v);
}

/* iris_vae_load_safetensors_ex (iris_vae.c:1227-1386), decoder tensors */
static orc_vae_t *load(osrc_t *s, int z, float scaling, float shift) {
    orc_vae_t *v = (orc_vae_t *)calloc(1, sizeof(*v));
    char n[256];
    if (!v) return NULL;
    v->z = z;
    v->lc = 4 * z;
    v->scaling = scaling;
    v->shift = shift;
    v->eps = scaling != 0.0f ? 1e-6f : 1e-4f;
    const int mid = 512;
    v->cin_w = get(s, "decoder.conv_in.weight", (size_t)mid * z * 9, z * 9);
    v->cin_b = get(s, "decoder.conv_in.bias", mid, 0);
    load_res(s, &v->mid1, "decoder.mid_block.resnets.0", mid, mid);
    load_res(s, &v->mid2, "decoder.mid_block.resnets.1", mid, mid);
    load_attn(s, &v->attn, "decoder.mid_block.attentions.0");
    for (int i = 0, bi = 0; i < 4; i++) {
        const int level = 3 - i, ch = 128 * ch_mult[level];
        const int prev = level == 3 ? mid : 128 * ch_mult[level + 1];
        for (int r = 0; r < 3; r++) {
            snprintf(n, sizeof(n), "decoder.up_blocks.%d.resnets.%d", i, r);
            load_res(s, &v->up[bi++], n, r == 0 ? prev : ch, ch);
        }
        if (i < 3) {
            snprintf(n, sizeof(n), "decoder.up_blocks.%d.upsamplers.0.conv.weight", i);
            v->ups_w[i] = get(s, n, (size_t)ch * ch * 9, ch * 9);
            snprintf(n, sizeof(n), "decoder.up_blocks.%d.upsamplers.0.conv.bias", i);
            v->ups_b[i] = get(s, n, ch, 0);
        }
    }
    v->no_g = get(s, "decoder.conv_norm_out.weight", 128, 0);
    v->no_b = get(s, "decoder.conv_norm_out.bias", 128, 0);
    v->co_w = get(s, "decoder.conv_out.weight", (size_t)3 * 128 * 9, 128 * 9);
    v->co_b = get(s, "decoder.conv_out.bias", 3, 0);
    if (has(s, "bn.running_mean")) {
        v->bn_mean = get(s, "bn.running_mean", v->lc, 0);
        v->bn_var = get(s, "bn.running_var", v->lc, 0);
    }
    if (has(s, "post_quant_conv.weight")) {
        v->pqw = get(s, "post_quant_conv.weight", (size_t)z * z, z);
        v->pqb = get(s, "post_quant_conv.bias", z, 0);
    }
    if (has(s, "encoder.conv_in.weight")) {   /* encoder half (iris_vae.c:1260-1310) */
        v->has_enc = 1;
        v->e_cin_w = get(s, "encoder.conv_in.weight", (size_t)128 * 3 * 9, 27);
        v->e_cin_b = get(s, "encoder.conv_in.bias", 128, 0);
        for (int level = 0, bi = 0; level < 4; level++) {
            const int ch = 128 * ch_mult[level], prev = level ? 128 * ch_mult[level - 1] : 128;
            for (int r = 0; r < 2; r++) {
                snprintf(n, sizeof(n), "encoder.down_blocks.%d.resnets.%d", level, r);
                load_res(s, &v->e_down[bi++], n, r == 0 && level > 0 ? prev : ch, ch);
            }
            if (level < 3) {
                snprintf(n, sizeof(n), "encoder.down_blocks.%d.downsamplers.0.conv.weight", level);
                v->e_ds_w[level] = get(s, n, (size_t)ch * ch * 9, ch * 9);
                snprintf(n, sizeof(n), "encoder.down_blocks.%d.downsamplers.0.conv.bias", level);
                v->e_ds_b[level] = get(s, n, ch, 0);
            }
        }
        load_res(s, &v->e_mid1, "encoder.mid_block.resnets.0", mid, mid);
        load_attn(s, &v->e_attn, "encoder.mid_block.attentions.0");
        load_res(s, &v->e_mid2, "encoder.mid_block.resnets.1", mid, mid);
        v->e_no_g = get(s, "encoder.conv_norm_out.weight", mid, 0);
        v->e_no_b = get(s, "encoder.conv_norm_out.bias", mid, 0);
        v->e_co_w = get(s, "encoder.conv_out.weight", (size_t)2 * z * mid * 9, mid * 9);
        v->e_co_b = get(s, "encoder.conv_out.bias", 2 * z, 0);
        if (has(s, "quant_conv.weight")) {
            v->qcw = get(s, "quant_conv.weight", (size_t)4 * z * z, 2 * z);
            v->qcb = get(s, "quant_conv.bias", 2 * z, 0);
        }
    }
    if (!v->bn_mean && scaling == 0.0f) {   /* identity statistics (iris_vae.c:1371-1377) */
        v->bn_mean = (float *)calloc(v->lc, sizeof(float));
        v->bn_var = (float *)malloc(v->lc * sizeof(float));
        for (int i = 0; i < v->lc; i++) v->bn_var[i] = 1.0f;
    }
    if (s->bad) {
        orc_vae_free(v);
        return NULL;
    }
    return v;
}

orc_vae_t *orc_vae_load(const char *path, int z, float scaling, float shift) {
    osrc_t s = {iris_st_open(path), 0, 0};
    if (!s.f) return NULL;
    orc_vae_t *v = load(&s, z, scaling, shift);
    iris_st_close(s.f);
    return v;
}

orc_vae_t *orc_vae_create_synth(int z, float scaling, float shift, uint64_t seed) {
    osrc_t s = {NULL, seed, 0};
    return load(&s, z, scaling, shift);
}

/* load_attnblock_sf (iris_vae.c:1184-1225) */
static void load_attn(osrc_t *s, oattn_t *a, const char *p) {
    char n[256];
    const int C = 512;
#define A(field, suffix, count, fan)                               \
    do {                                                           \
        snprintf(n, sizeof(n), "%s.%s", p, suffix);                \
        a->field = get(s, n, count, fan);                          \
    } while (0)
    A(g, "group_norm.weight", C, 0);
    A(b, "group_norm.bias", C, 0);
    A(qw, "to_q.weight", (size_t)C * C, C);
    A(qb, "to_q.bias", C, 0);
    A(kw, "to_k.weight", (size_t)C * C, C);
    A(kb, "to_k.bias", C, 0);
    A(vw, "to_v.weight", (size_t)C * C, C);
    A(vb, "to_v.bias", C, 0);
    A(ow, "to_out.0.weight", (size_t)C * C, C);
    A(ob, "to_out.0.bias", C, 0);
#undef A
}

/* ---------------------------------------------------------------- layers */

/* iris_conv2d, stride 1, padding (k - 1) / 2, k = 1 or 3; planar NCHW */
static void conv(float *out, const float *in, const float *w, const float *b, int cin, int cout, int H, int W,
                 int k) {
    const int pad = k / 2;
    const size_t plane = (size_t)H * W;
#pragma omp parallel for schedule(dynamic, 1)
    for (int o = 0; o < cout; o++) {
        float *dst = out + o * plane;
        for (size_t i = 0; i < plane; i++) dst[i] = b ? b[o] : 0.0f;
        for (int c = 0; c < cin; c++) {
            const float *src = in + c * plane;
            for (int ky = 0; ky < k; ky++)
                for (int kx = 0; kx < k; kx++) {
                    const float wv = w[(((size_t)o * cin + c) * k + ky) * k + kx];
                    const int dy = ky - pad, dx = kx - pad;
                    const int x0 = dx < 0 ? -dx : 0, x1 = dx > 0 ? W - dx : W;
                    for (int y = 0; y < H; y++) {
                        const int yy = y + dy;
                        if (yy < 0 || yy >= H) continue;
                        float *d = dst + (size_t)y * W;
                        const float *s = src + (size_t)yy * W + dx;
                        for (int x = x0; x < x1; x++) d[x] += wv * s[x];
                    }
                }
        }
    }
}

/* iris_group_norm (iris_kernels.c:542-582), sums in float64 */
static void group_norm(float *out, const float *x, const float *g, const float *b, int C, int H, int W, float eps,
                       int swish) {
    const int cpg = C / 32;
    const size_t plane = (size_t)H * W, n = (size_t)cpg * plane;
#pragma omp parallel for schedule(static)
    for (int grp = 0; grp < 32; grp++) {
        const float *xs = x + grp * n;
        double s = 0.0;
        for (size_t i = 0; i < n; i++) s += xs[i];
        const double mean = s / (double)n;
        double q = 0.0;
        for (size_t i = 0; i < n; i++) q += (xs[i] - mean) * (xs[i] - mean);
        const float inv = 1.0f / sqrtf((float)(q / (double)n) + eps);
        for (size_t i = 0; i < n; i++) {
            const int c = grp * cpg + (int)(i / plane);
            out[grp * n + i] = g[c] * (((float)(xs[i] - mean)) * inv) + b[c];
        }
        if (swish) orc_silu(out + grp * n, (int)n);
    }
}

/* resblock_forward (iris_vae.c:203-251) */
static void resblock(float *x, const ores_t *r, int H, int W, float eps, float *w1, float *w2, float *w3) {
    const size_t plane = (size_t)H * W;
    if (r->sk) conv(w3, x, r->sk, r->skb, r->cin, r->cout, H, W, 1);
    else memcpy(w3, x, plane * r->cin * sizeof(float));
    group_norm(w1, x, r->n1g, r->n1b, r->cin, H, W, eps, 1);
    conv(w2, w1, r->c1, r->c1b, r->cin, r->cout, H, W, 3);
    group_norm(w1, w2, r->n2g, r->n2b, r->cout, H, W, eps, 1);
    conv(w2, w1, r->c2, r->c2b, r->cout, r->cout, H, W, 3);
    for (size_t i = 0; i < plane * r->cout; i++) x[i] = w3[i] + w2[i];
}

/* attnblock_forward (iris_vae.c:260-357): one head of width C over H*W */
static void attention(float *x, const orc_vae_t *v, const oattn_t *a, int H, int W, float *w1, float *w2) {
    const int C = 512, S = H * W;
    const size_t plane = (size_t)S;
    float *q = w2, *k = q + plane * C, *vv = k + plane * C;
    group_norm(w1, x, a->g, a->b, C, H, W, v->eps, 0);
    conv(q, w1, a->qw, a->qb, C, C, H, W, 1);
    conv(k, w1, a->kw, a->kb, C, C, H, W, 1);
    conv(vv, w1, a->vw, a->vb, C, C, H, W, 1);
    const float scale = 1.0f / sqrtf((float)C);
    float *qt = (float *)malloc(plane * C * sizeof(float)), *kt = (float *)malloc(plane * C * sizeof(float));
    float *vt = (float *)malloc(plane * C * sizeof(float)), *ot = (float *)malloc(plane * C * sizeof(float));
    float *sc = (float *)malloc(plane * plane * sizeof(float));
    for (int c = 0; c < C; c++)
        for (int i = 0; i < S; i++) {
            qt[(size_t)i * C + c] = q[c * plane + i] * scale;
            kt[(size_t)i * C + c] = k[c * plane + i];
            vt[(size_t)i * C + c] = vv[c * plane + i];
        }
    orc_sgemm_nt(S, S, C, 1.0f, qt, C, kt, C, 0.0f, sc, S);
    orc_softmax(sc, S, S);
    orc_sgemm_nn(S, C, S, 1.0f, sc, S, vt, C, 0.0f, ot, C);
    for (int c = 0; c < C; c++)
        for (int i = 0; i < S; i++) w1[c * plane + i] = ot[(size_t)i * C + c];
    conv(w2, w1, a->ow, a->ob, C, C, H, W, 1);
    for (size_t i = 0; i < plane * C; i++) x[i] += w2[i];
    free(qt);
    free(kt);
    free(vt);
    free(ot);
    free(sc);
}

/* iris_vae_decode (iris_vae.c:835-998) for one latent [4z][lh][lw]: rgb
 * [16lh][16lw][3] uint8, f32 (or NULL) the conv_out output [3][16lh][16lw].
 * stop_after >= 0 ends after that many decoder stages and copies the
 * activation (NCHW) into f32 instead: 0 = conv_in, 1 = mid block, 2.. = each
 * up level. */
int orc_vae_decode(orc_vae_t *v, const float *latent, int lh, int lw, uint8_t *rgb, float *f32, int stop_after) {
    const int H0 = 2 * lh, W0 = 2 * lw, Hf = 16 * lh, Wf = 16 * lw;
    const size_t cap = (size_t)Hf * Wf * 256 * 2;
    float *x = (float *)malloc(cap * sizeof(float)), *t = (float *)malloc(cap * sizeof(float));
    float *w1 = (float *)malloc(cap * sizeof(float)), *w2 = (float *)malloc(cap * sizeof(float));
    float *w3 = (float *)malloc(cap * sizeof(float));
    int rc = -1, stage = 0;
    if (!x || !t || !w1 || !w2 || !w3) goto out;
    {
        const int lc = v->lc, zs = lh * lw;
        for (int c = 0; c < lc; c++)
            for (int i = 0; i < zs; i++) {
                const float val = latent[(size_t)c * zs + i];
                t[(size_t)c * zs + i] = v->scaling != 0.0f ? val / v->scaling + v->shift
                                                           : val * sqrtf(v->bn_var[c] + v->eps) + v->bn_mean[c];
            }
        /* iris_unpatchify: channel c * 4 + pi * 2 + pj at (ph, pw) -> c at (2ph + pi, 2pw + pj) */
        for (int c = 0; c < v->z; c++)
            for (int oy = 0; oy < H0; oy++)
                for (int ox = 0; ox < W0; ox++)
                    x[((size_t)c * H0 + oy) * W0 + ox] =
                        t[((size_t)(c * 4 + (oy & 1) * 2 + (ox & 1)) * lh + oy / 2) * lw + ox / 2];
        if (v->pqw) {
            conv(t, x, v->pqw, v->pqb, v->z, v->z, H0, W0, 1);
            memcpy(x, t, (size_t)v->z * H0 * W0 * sizeof(float));
        }
        conv(t, x, v->cin_w, v->cin_b, v->z, 512, H0, W0, 3);
        memcpy(x, t, (size_t)512 * H0 * W0 * sizeof(float));
        int H = H0, W = W0, C = 512;
        if (stop_after == stage++) goto dump;
        resblock(x, &v->mid1, H, W, v->eps, w1, w2, w3);
        attention(x, v, &v->attn, H, W, w1, w2);
        resblock(x, &v->mid2, H, W, v->eps, w1, w2, w3);
        if (stop_after == stage++) goto dump;
        for (int level = 3, bi = 0; level >= 0; level--) {
            for (int r = 0; r < 3; r++) {
                const ores_t *rb = &v->up[bi++];
                resblock(x, rb, H, W, v->eps, w1, w2, w3);
                C = rb->cout;
            }
            if (level > 0) {
                const size_t plane = (size_t)H * W;
                for (int c = 0; c < C; c++)
                    for (int y = 0; y < 2 * H; y++)
                        for (int xx = 0; xx < 2 * W; xx++)
                            t[(size_t)c * 4 * plane + (size_t)y * 2 * W + xx] = x[c * plane + (size_t)(y / 2) * W + xx / 2];
                H *= 2;
                W *= 2;
                conv(x, t, v->ups_w[3 - level], v->ups_b[3 - level], C, C, H, W, 3);
            }
            if (stop_after == stage++) goto dump;
        }
        group_norm(t, x, v->no_g, v->no_b, 128, H, W, v->eps, 1);
        conv(x, t, v->co_w, v->co_b, 128, 3, H, W, 3);
        for (int y = 0; y < H; y++)
            for (int xx = 0; xx < W; xx++)
                for (int ch = 0; ch < 3; ch++) {
                    float val = x[(size_t)ch * H * W + (size_t)y * W + xx];
                    val = (val + 1.0f) * 0.5f;
                    val = val * 255.0f;
                    if (val < 0) val = 0;
                    if (val > 255) val = 255;
                    rgb[((size_t)y * W + xx) * 3 + ch] = (uint8_t)(val + 0.5f);
                }
        if (f32) memcpy(f32, x, (size_t)3 * H * W * sizeof(float));
        rc = 0;
        goto out;
    dump:
        if (f32) memcpy(f32, x, (size_t)C * H * W * sizeof(float));
        rc = C;
    }
out:
    free(x);
    free(t);
    free(w1);
    free(w2);
    free(w3);
    return rc;
}

/* stride-2 3x3 conv over the input padded by one zero row and column on the
 * right and bottom (vae_pad_right_bottom + vae_conv2d, iris_vae.c:172-193,
 * :407-418); input [C][H][W], output [C][H/2][W/2] */
static void conv_down(float *out, const float *in, const float *w, const float *b, int C, int H, int W) {
    const int Ho = (H + 1 - 3) / 2 + 1, Wo = (W + 1 - 3) / 2 + 1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int o = 0; o < C; o++) {
        float *dst = out + (size_t)o * Ho * Wo;
        for (int i = 0; i < Ho * Wo; i++) dst[i] = b[o];
        for (int c = 0; c < C; c++) {
            const float *src = in + (size_t)c * H * W;
            for (int ky = 0; ky < 3; ky++)
                for (int kx = 0; kx < 3; kx++) {
                    const float wv = w[(((size_t)o * C + c) * 3 + ky) * 3 + kx];
                    for (int y = 0; y < Ho; y++) {
                        const int yy = 2 * y + ky;
                        if (yy >= H) continue;
                        for (int x = 0; x < Wo; x++) {
                            const int xx = 2 * x + kx;
                            if (xx < W) dst[(size_t)y * Wo + x] += wv * src[(size_t)yy * W + xx];
                        }
                    }
                }
        }
    }
}

/* iris_vae_encode (iris_vae.c:363-482) for one image [3][H][W]: latent
 * [4z][H/16][W/16] into lat; -1 without encoder weights */
int orc_vae_encode(orc_vae_t *v, const float *img, int H, int W, float *lat) {
    if (!v->has_enc || H % 16 || W % 16) return -1;
    const size_t cap = (size_t)H * W * 128 * 4;
    float *x = (float *)malloc(cap * sizeof(float)), *t = (float *)malloc(cap * sizeof(float));
    float *w1 = (float *)malloc(cap * sizeof(float)), *w2 = (float *)malloc(cap * sizeof(float));
    float *w3 = (float *)malloc(cap * sizeof(float));
    int rc = -1;
    if (!x || !t || !w1 || !w2 || !w3) goto out;
    {
        conv(x, img, v->e_cin_w, v->e_cin_b, 3, 128, H, W, 3);
        int h = H, w = W, C = 128;
        for (int level = 0, bi = 0; level < 4; level++) {
            for (int r = 0; r < 2; r++) {
                const ores_t *rb = &v->e_down[bi++];
                resblock(x, rb, h, w, v->eps, w1, w2, w3);
                C = rb->cout;
            }
            if (level < 3) {
                conv_down(t, x, v->e_ds_w[level], v->e_ds_b[level], C, h, w);
                h /= 2;
                w /= 2;
                memcpy(x, t, (size_t)C * h * w * sizeof(float));
            }
        }
        resblock(x, &v->e_mid1, h, w, v->eps, w1, w2, w3);
        attention(x, v, &v->e_attn, h, w, w1, w2);
        resblock(x, &v->e_mid2, h, w, v->eps, w1, w2, w3);
        group_norm(t, x, v->e_no_g, v->e_no_b, 512, h, w, v->eps, 1);
        const int z = v->z, z2 = 2 * z;
        conv(x, t, v->e_co_w, v->e_co_b, 512, z2, h, w, 3);
        if (v->qcw) {
            conv(t, x, v->qcw, v->qcb, z2, z2, h, w, 1);
            memcpy(x, t, (size_t)z2 * h * w * sizeof(float));
        }
        /* mean (first z channels), iris_patchify 2x2, normalization */
        const int lh = h / 2, lw = w / 2;
        for (int c = 0; c < z; c++)
            for (int ph = 0; ph < lh; ph++)
                for (int pw = 0; pw < lw; pw++)
                    for (int pi = 0; pi < 2; pi++)
                        for (int pj = 0; pj < 2; pj++) {
                            const int lc = c * 4 + pi * 2 + pj;
                            const float val = x[((size_t)c * h + ph * 2 + pi) * w + pw * 2 + pj];
                            float o;
                            if (v->scaling != 0.0f) {
                                o = (val - v->shift) * v->scaling;
                            } else {
                                const float inv = 1.0f / sqrtf(v->bn_var[lc] + v->eps);
                                o = (val - v->bn_mean[lc]) * inv;
                            }
                            lat[((size_t)lc * lh + ph) * lw + pw] = o;
                        }
        rc = 0;
    }
out:
    free(x);
    free(t);
    free(w1);
    free(w2);
    free(w3);
    return rc;
}
