/*
 * iris_vae.c - host side of the GPU VAE decoder (include/iris_vae.h).
 *
 * Mirrors iris_vae_decode (iris_vae.c:835-998 of the reference) step by step
 * with device-resident, channels-last activations:
 *   latent -> denormalize, unpatchify, post_quant_conv  (iris_hip_vae_front)
 *          -> conv_in 3x3 z -> 512                       (implicit GEMM)
 *          -> mid: resblock, attention, resblock
 *          -> up levels 3..0: 3 resblocks, then nearest 2x + conv 3x3
 *             (levels 3..1; the upsample is folded into the conv's loads)
 *          -> GroupNorm + swish -> conv_out 128 -> 3 -> uint8 RGB.
 * The residual stream x is f32 [pixels][C]; GroupNorm writes the bf16 input
 * of each convolution; convolutions accumulate in f32 and add into x in their
 * epilogue. resblock_forward (iris_vae.c:203-251) and attnblock_forward
 * (iris_vae.c:260-357) map to resblock() and attention() below.
 */
#include "../../include/iris_vae.h"
#include "../../include/iris_hip.h"
#include "../../include/iris_synth.h"
#include "iris_st.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define VAE_BASE 128
#define VAE_MID 512
#define VAE_GROUPS 32
#define VAE_CIN_PAD 64         /* conv_in's input channels, zero-padded */
#define GN_BLOCKS 1024         /* blocks of the GroupNorm statistics pass */
#define SCORE_ELEMS (1u << 28) /* attention probabilities held at once (bf16) */

static const int ch_mult[4] = {1, 2, 4, 4};

typedef struct {
    float *n1g, *n1b, *n2g, *n2b;
    uint16_t *c1, *c2, *sk;    /* [cout][9][cin], [cout][9][cout], [cout][cin] */
    float *c1b, *c2b, *skb;
    int cin, cout;
} vres_t;

typedef struct {
    float *g, *b;              /* group_norm */
    uint16_t *qkv_w, *o_w;     /* [1536][512] (q rows scaled by 1/sqrt(512)), [512][512] */
    float *qkv_b, *o_b;
} vattn_t;

struct iris_vae_gpu {
    int z, lat_ch, divide, has_enc;
    float eps;
    float *lsc, *lsh;          /* per latent channel: x * lsc + lsh (or x / lsc + lsh) */
    float *pqw, *pqb;          /* post_quant_conv [z][z], or NULL */
    uint16_t *cin_w;           /* [512][9][64] */
    float *cin_b;
    vres_t mid1, mid2, up[12];
    vattn_t attn;
    uint16_t *ups_w[3];
    float *ups_b[3];
    float *no_g, *no_b, *co_w, *co_b;   /* conv_out f32 [9][128][4], bias [4] */
    /* encoder (iris_vae_encode, iris_vae.c:363-482) */
    uint16_t *e_cin_w, *e_ds_w[3], *e_co_w;   /* [128][9][64], [C][9][C], [2z][9][512] */
    float *e_cin_b, *e_ds_b[3], *e_co_b;
    vres_t e_down[8], e_mid1, e_mid2;
    vattn_t e_attn;
    float *e_no_g, *e_no_b, *qw, *qb;         /* quant_conv [2z][2z] (Flux) */
    float *esc, *esh;                          /* latent normalization: (x - esh) * esc */
    /* work buffers, sized for cap_pix output pixels */
    size_t cap_pix;
    float *x, *y, *sst, *srow, *ws, *ab, *dlat, *df32;   /* sst, srow: the softmax's row statistics */
    uint16_t *t, *h, *raw, *qkv, *vt, *att, *pm, *front;
    uint8_t *drgb;
    float *dimg;
    double *part;
    size_t ws_bytes;
    /* part holds the GroupNorm sums of st_buf (st_nblk row tiles), written
     * by the convolution that produced it; NULL: none pending */
    const void *st_buf;
    int st_nblk;
};

static int fail(const char *what) {
    fprintf(stderr, "vae: %s: %s\n", what, iris_hip_last_error());
    return -1;
}

/* ------------------------------------------------------------ weight upload */

typedef struct {
    iris_st_file_t *f;     /* NULL: synthetic */
    uint64_t seed;
} vsrc_t;

/* n f32 values of a named tensor (malloc'd), file or synthetic */
static float *vsrc_read(vsrc_t *s, const char *name, size_t n, int fan_in) {
    float *h = (float *)malloc(n * sizeof(float));
    if (!h) return NULL;
    if (s->f) {
        const iris_st_tensor_t *t = iris_st_find(s->f, name);
        if (!t || (size_t)iris_st_numel(t) != n || iris_st_read_f32(s->f, t, h)) {
            fprintf(stderr, "vae: tensor %s missing or not %zu elements\n", name, n);
            free(h);
            return NULL;
        }
        return h;
    }
    float mean, std;
    iris_synth_vae_stats(name, fan_in, &mean, &std);
    iris_synth_fill_f32(h, n, iris_synth_seed(s->seed, name), 0, mean, std);
    return h;
}

static int vsrc_has(vsrc_t *s, const char *name) { return !s->f || iris_st_find(s->f, name) != NULL; }

static void *upload(const void *h, size_t bytes) {
    void *d = iris_hip_malloc(bytes);
    if (!d) return NULL;
    if (iris_hip_memcpy_h2d(d, h, bytes) || iris_hip_sync()) {
        iris_hip_free(d);
        return NULL;
    }
    return d;
}

static float *up_vec(vsrc_t *s, const char *name, size_t n) {
    float *h = vsrc_read(s, name, n, 0);
    float *d = h ? (float *)upload(h, n * sizeof(float)) : NULL;
    free(h);
    return d;
}

/* 3x3 conv [cout][cin][3][3] -> bf16 [cout][9][cin_pad] (zero-padded channels) */
static uint16_t *up_conv3(vsrc_t *s, const char *name, int cout, int cin, int cin_pad) {
    float *h = vsrc_read(s, name, (size_t)cout * cin * 9, cin * 9);
    if (!h) return NULL;
    uint16_t *b = (uint16_t *)calloc((size_t)cout * 9 * cin_pad, sizeof(uint16_t));
    uint16_t *d = NULL;
    if (b) {
        for (int o = 0; o < cout; o++)
            for (int c = 0; c < cin; c++)
                for (int tap = 0; tap < 9; tap++)
                    b[((size_t)o * 9 + tap) * cin_pad + c] = iris_f32_to_bf16(h[((size_t)o * cin + c) * 9 + tap]);
        d = (uint16_t *)upload(b, (size_t)cout * 9 * cin_pad * sizeof(uint16_t));
    }
    free(b);
    free(h);
    return d;
}

/* 1x1 conv / linear [rows][cols] -> bf16 at dst (device), values times scale */
static int up_mat_into(vsrc_t *s, const char *name, int rows, int cols, float scale, uint16_t *dst) {
    float *h = vsrc_read(s, name, (size_t)rows * cols, cols);
    if (!h) return -1;
    uint16_t *b = (uint16_t *)malloc((size_t)rows * cols * sizeof(uint16_t));
    int rc = -1;
    if (b) {
        for (size_t i = 0; i < (size_t)rows * cols; i++) b[i] = iris_f32_to_bf16(h[i] * scale);
        rc = iris_hip_memcpy_h2d(dst, b, (size_t)rows * cols * sizeof(uint16_t)) || iris_hip_sync() ? -1 : 0;
    }
    free(b);
    free(h);
    return rc;
}

static int load_res(vsrc_t *s, vres_t *r, const char *prefix, int cin, int cout) {
    char n[256];
    r->cin = cin;
    r->cout = cout;
#define NAME(suffix) (snprintf(n, sizeof(n), "%s.%s", prefix, suffix), n)
    if (!(r->n1g = up_vec(s, NAME("norm1.weight"), cin)) || !(r->n1b = up_vec(s, NAME("norm1.bias"), cin)) ||
        !(r->c1 = up_conv3(s, NAME("conv1.weight"), cout, cin, cin)) ||
        !(r->c1b = up_vec(s, NAME("conv1.bias"), cout)) || !(r->n2g = up_vec(s, NAME("norm2.weight"), cout)) ||
        !(r->n2b = up_vec(s, NAME("norm2.bias"), cout)) ||
        !(r->c2 = up_conv3(s, NAME("conv2.weight"), cout, cout, cout)) ||
        !(r->c2b = up_vec(s, NAME("conv2.bias"), cout)))
        return -1;
    if (cin != cout) {
        r->sk = (uint16_t *)iris_hip_malloc((size_t)cout * cin * 2);
        if (!r->sk || up_mat_into(s, NAME("conv_shortcut.weight"), cout, cin, 1.0f, r->sk) ||
            !(r->skb = up_vec(s, NAME("conv_shortcut.bias"), cout)))
            return -1;
    }
#undef NAME
    return 0;
}

static void free_res(vres_t *r) {
    void *p[] = {r->n1g, r->n1b, r->n2g, r->n2b, r->c1, r->c2, r->sk, r->c1b, r->c2b, r->skb};
    for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) iris_hip_free(p[i]);
}

/* load_attnblock_sf (iris_vae.c:1184-1225): q, k, v stacked; q (weights and
 * bias) scaled by 1/sqrt(C) as the reference scales q before Q K^T
 * (iris_vae.c:318) */
static int load_attn(vsrc_t *s, vattn_t *a, const char *pre) {
    char n[256];
    const float qs = 1.0f / sqrtf((float)VAE_MID);
    snprintf(n, sizeof(n), "%s.group_norm.weight", pre);
    if (!(a->g = up_vec(s, n, VAE_MID))) return -1;
    snprintf(n, sizeof(n), "%s.group_norm.bias", pre);
    if (!(a->b = up_vec(s, n, VAE_MID))) return -1;
    a->qkv_w = (uint16_t *)iris_hip_malloc((size_t)3 * VAE_MID * VAE_MID * 2);
    a->o_w = (uint16_t *)iris_hip_malloc((size_t)VAE_MID * VAE_MID * 2);
    if (!a->qkv_w || !a->o_w) return -1;
    const char *proj[3] = {"to_q", "to_k", "to_v"};
    float bias[3 * VAE_MID];
    for (int i = 0; i < 3; i++) {
        snprintf(n, sizeof(n), "%s.%s.weight", pre, proj[i]);
        if (up_mat_into(s, n, VAE_MID, VAE_MID, i == 0 ? qs : 1.0f, a->qkv_w + (size_t)i * VAE_MID * VAE_MID))
            return -1;
        snprintf(n, sizeof(n), "%s.%s.bias", pre, proj[i]);
        float *b = vsrc_read(s, n, VAE_MID, 0);
        if (!b) return -1;
        for (int j = 0; j < VAE_MID; j++) bias[i * VAE_MID + j] = b[j] * (i == 0 ? qs : 1.0f);
        free(b);
    }
    if (!(a->qkv_b = (float *)upload(bias, sizeof(bias)))) return -1;
    snprintf(n, sizeof(n), "%s.to_out.0.weight", pre);
    if (up_mat_into(s, n, VAE_MID, VAE_MID, 1.0f, a->o_w)) return -1;
    snprintf(n, sizeof(n), "%s.to_out.0.bias", pre);
    return (a->o_b = up_vec(s, n, VAE_MID)) ? 0 : -1;
}

static void free_attn(vattn_t *a) {
    void *p[] = {a->g, a->b, a->qkv_w, a->o_w, a->qkv_b, a->o_b};
    for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) iris_hip_free(p[i]);
}

/* encoder half of iris_vae_load_safetensors_ex (iris_vae.c:1260-1310) */
static int load_encoder(vsrc_t *s, iris_vae_gpu_t *v) {
    char n[256];
    const int z2 = 2 * v->z;
    if (!(v->e_cin_w = up_conv3(s, "encoder.conv_in.weight", VAE_BASE, 3, VAE_CIN_PAD)) ||
        !(v->e_cin_b = up_vec(s, "encoder.conv_in.bias", VAE_BASE)))
        return -1;
    for (int level = 0, bi = 0; level < 4; level++) {
        const int ch = VAE_BASE * ch_mult[level], prev = level ? VAE_BASE * ch_mult[level - 1] : VAE_BASE;
        for (int r = 0; r < 2; r++, bi++) {
            snprintf(n, sizeof(n), "encoder.down_blocks.%d.resnets.%d", level, r);
            if (load_res(s, &v->e_down[bi], n, r == 0 && level > 0 ? prev : ch, ch)) return -1;
        }
        if (level < 3) {
            snprintf(n, sizeof(n), "encoder.down_blocks.%d.downsamplers.0.conv.weight", level);
            if (!(v->e_ds_w[level] = up_conv3(s, n, ch, ch, ch))) return -1;
            snprintf(n, sizeof(n), "encoder.down_blocks.%d.downsamplers.0.conv.bias", level);
            if (!(v->e_ds_b[level] = up_vec(s, n, ch))) return -1;
        }
    }
    if (load_res(s, &v->e_mid1, "encoder.mid_block.resnets.0", VAE_MID, VAE_MID) ||
        load_attn(s, &v->e_attn, "encoder.mid_block.attentions.0") ||
        load_res(s, &v->e_mid2, "encoder.mid_block.resnets.1", VAE_MID, VAE_MID) ||
        !(v->e_no_g = up_vec(s, "encoder.conv_norm_out.weight", VAE_MID)) ||
        !(v->e_no_b = up_vec(s, "encoder.conv_norm_out.bias", VAE_MID)) ||
        !(v->e_co_w = up_conv3(s, "encoder.conv_out.weight", z2, VAE_MID, VAE_MID)) ||
        !(v->e_co_b = up_vec(s, "encoder.conv_out.bias", z2)))
        return -1;
    if (vsrc_has(s, "quant_conv.weight") &&
        (!(v->qw = up_vec(s, "quant_conv.weight", (size_t)z2 * z2)) || !(v->qb = up_vec(s, "quant_conv.bias", z2))))
        return -1;
    v->has_enc = 1;
    return 0;
}

static void free_work(iris_vae_gpu_t *v) {
    void *p[] = {v->x, v->y, v->sst, v->srow, v->ws, v->ab, v->dlat, v->df32, v->t, v->h, v->raw, v->qkv, v->vt,
                 v->att, v->pm, v->front, v->drgb, v->part, v->dimg};
    for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) iris_hip_free(p[i]);
    v->x = v->y = v->sst = v->srow = v->ws = v->ab = v->dlat = v->df32 = NULL;
    v->t = v->h = v->raw = v->qkv = v->vt = v->att = v->pm = v->front = NULL;
    v->drgb = NULL;
    v->dimg = NULL;
    v->part = NULL;
    v->cap_pix = 0;
}

void iris_vae_gpu_free(iris_vae_gpu_t *v) {
    if (!v) return;
    free_work(v);
    free_res(&v->mid1);
    free_res(&v->mid2);
    for (int i = 0; i < 12; i++) free_res(&v->up[i]);
    for (int i = 0; i < 8; i++) free_res(&v->e_down[i]);
    free_res(&v->e_mid1);
    free_res(&v->e_mid2);
    free_attn(&v->attn);
    free_attn(&v->e_attn);
    void *p[] = {v->lsc, v->lsh, v->pqw, v->pqb, v->cin_w, v->cin_b, v->no_g, v->no_b, v->co_w, v->co_b,
                 v->ups_w[0], v->ups_w[1], v->ups_w[2], v->ups_b[0], v->ups_b[1], v->ups_b[2], v->e_cin_w,
                 v->e_cin_b, v->e_ds_w[0], v->e_ds_w[1], v->e_ds_w[2], v->e_ds_b[0], v->e_ds_b[1], v->e_ds_b[2],
                 v->e_co_w, v->e_co_b, v->e_no_g, v->e_no_b, v->qw, v->qb, v->esc, v->esh};
    for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) iris_hip_free(p[i]);
    free(v);
}

/* iris_vae_load_safetensors_ex (iris_vae.c:1227-1386), decoder half */
static iris_vae_gpu_t *load(vsrc_t *s, int z, float scaling, float shift) {
    if (z <= 0 || z > 32) {
        fprintf(stderr, "vae: z_channels=%d (1..32)\n", z);
        return NULL;
    }
    if (iris_hip_init(0)) return NULL;
    iris_vae_gpu_t *v = (iris_vae_gpu_t *)calloc(1, sizeof(*v));
    if (!v) return NULL;
    v->z = z;
    v->lat_ch = 4 * z;
    v->eps = scaling != 0.0f ? 1e-6f : 1e-4f;
    const int lc = v->lat_ch;
    char n[256];

    /* latent denormalization, per latent channel */
    float sc[128], sh[128];
    if (scaling != 0.0f) {
        v->divide = 1;
        for (int c = 0; c < lc; c++) {
            sc[c] = scaling;
            sh[c] = shift;
        }
    } else if (vsrc_has(s, "bn.running_mean")) {
        float *m = vsrc_read(s, "bn.running_mean", lc, 0);
        float *var = vsrc_read(s, "bn.running_var", lc, 0);
        if (!m || !var) {
            free(m);
            free(var);
            goto bad;
        }
        for (int c = 0; c < lc; c++) {
            sh[c] = m[c];
            sc[c] = sqrtf(var[c] + v->eps);
        }
        free(m);
        free(var);
    } else {
        for (int c = 0; c < lc; c++) {
            sh[c] = 0.0f;
            sc[c] = sqrtf(1.0f + v->eps);
        }
    }
    if (!(v->lsc = (float *)upload(sc, lc * sizeof(float))) || !(v->lsh = (float *)upload(sh, lc * sizeof(float))))
        goto bad;
    /* the encoder's inverse: (x - shift) * scaling, or (x - mean) / sqrt(var + eps)
     * (iris_batch_norm, iris_kernels.c:584-604) */
    {
        float esc[128], esh[128];
        for (int c = 0; c < lc; c++) {
            esc[c] = v->divide ? scaling : 1.0f / sc[c];
            esh[c] = sh[c];
        }
        if (!(v->esc = (float *)upload(esc, lc * sizeof(float))) || !(v->esh = (float *)upload(esh, lc * sizeof(float))))
            goto bad;
    }
    if (vsrc_has(s, "post_quant_conv.weight")) {
        if (!(v->pqw = up_vec(s, "post_quant_conv.weight", (size_t)z * z)) ||
            !(v->pqb = up_vec(s, "post_quant_conv.bias", z)))
            goto bad;
    }
    if (!(v->cin_w = up_conv3(s, "decoder.conv_in.weight", VAE_MID, z, VAE_CIN_PAD)) ||
        !(v->cin_b = up_vec(s, "decoder.conv_in.bias", VAE_MID)))
        goto bad;
    if (load_res(s, &v->mid1, "decoder.mid_block.resnets.0", VAE_MID, VAE_MID) ||
        load_res(s, &v->mid2, "decoder.mid_block.resnets.1", VAE_MID, VAE_MID))
        goto bad;
    if (load_attn(s, &v->attn, "decoder.mid_block.attentions.0")) goto bad;
    /* up blocks: up_blocks.i is level 3 - i */
    for (int i = 0, bi = 0; i < 4; i++) {
        const int level = 3 - i, ch = VAE_BASE * ch_mult[level];
        const int prev = level == 3 ? VAE_MID : VAE_BASE * ch_mult[level + 1];
        for (int r = 0; r < 3; r++, bi++) {
            snprintf(n, sizeof(n), "decoder.up_blocks.%d.resnets.%d", i, r);
            if (load_res(s, &v->up[bi], n, r == 0 ? prev : ch, ch)) goto bad;
        }
        if (i < 3) {
            snprintf(n, sizeof(n), "decoder.up_blocks.%d.upsamplers.0.conv.weight", i);
            if (!(v->ups_w[i] = up_conv3(s, n, ch, ch, ch))) goto bad;
            snprintf(n, sizeof(n), "decoder.up_blocks.%d.upsamplers.0.conv.bias", i);
            if (!(v->ups_b[i] = up_vec(s, n, ch))) goto bad;
        }
    }
    if (!(v->no_g = up_vec(s, "decoder.conv_norm_out.weight", VAE_BASE)) ||
        !(v->no_b = up_vec(s, "decoder.conv_norm_out.bias", VAE_BASE)))
        goto bad;
    {
        float *w = vsrc_read(s, "decoder.conv_out.weight", (size_t)3 * VAE_BASE * 9, VAE_BASE * 9);
        float *b = vsrc_read(s, "decoder.conv_out.bias", 3, 0);
        float *wt = (float *)calloc((size_t)9 * VAE_BASE * 4, sizeof(float));
        float b4[4] = {0, 0, 0, 0};
        int ok = w && b && wt;
        if (ok) {
            for (int o = 0; o < 3; o++) {
                b4[o] = b[o];
                for (int c = 0; c < VAE_BASE; c++)
                    for (int tap = 0; tap < 9; tap++) wt[((size_t)tap * VAE_BASE + c) * 4 + o] = w[((size_t)o * VAE_BASE + c) * 9 + tap];
            }
            v->co_w = (float *)upload(wt, (size_t)9 * VAE_BASE * 4 * sizeof(float));
            v->co_b = (float *)upload(b4, sizeof(b4));
        }
        free(w);
        free(b);
        free(wt);
        if (!ok || !v->co_w || !v->co_b) goto bad;
    }
    if (vsrc_has(s, "encoder.conv_in.weight") && load_encoder(s, v)) goto bad;
    return v;
bad:
    fail("load");
    iris_vae_gpu_free(v);
    return NULL;
}

iris_vae_gpu_t *iris_vae_gpu_load(const char *path, int z_channels, float scaling_factor, float shift_factor) {
    vsrc_t s = {0};
    if (!path || !(s.f = iris_st_open(path))) {
        fprintf(stderr, "vae: cannot open %s\n", path ? path : "(null)");
        return NULL;
    }
    iris_vae_gpu_t *v = load(&s, z_channels, scaling_factor, shift_factor);
    iris_st_close(s.f);
    return v;
}

iris_vae_gpu_t *iris_vae_gpu_create_synthetic(int z_channels, float scaling_factor, float shift_factor,
                                              uint64_t seed) {
    vsrc_t s = {NULL, seed};
    return load(&s, z_channels, scaling_factor, shift_factor);
}

/* iris_parse_vae_config (iris_vae_config.h): override-only key lookup */
static void parse_vae_config(const char *json, int *z, float *scaling, float *shift) {
    const char *p, *colon;
    if ((p = strstr(json, "\"latent_channels\"")) && (colon = strchr(p, ':'))) {
        const int lc = atoi(colon + 1);
        if (lc > 0) *z = lc;
    }
    if ((p = strstr(json, "\"scaling_factor\"")) && (colon = strchr(p, ':'))) *scaling = (float)atof(colon + 1);
    if ((p = strstr(json, "\"shift_factor\"")) && (colon = strchr(p, ':'))) *shift = (float)atof(colon + 1);
}

iris_vae_gpu_t *iris_vae_gpu_load_dir(const char *model_dir) {
    char path[4096];
    int z = 32;
    float scaling = 0.0f, shift = 0.0f;
    if (!model_dir) return NULL;
    snprintf(path, sizeof(path), "%.4000s/vae/config.json", model_dir);
    FILE *f = fopen(path, "r");
    if (f) {
        char buf[4096];
        const size_t n = fread(buf, 1, sizeof(buf) - 1, f);
        buf[n] = '\0';
        fclose(f);
        parse_vae_config(buf, &z, &scaling, &shift);
    }
    snprintf(path, sizeof(path), "%.4000s/vae/diffusion_pytorch_model.safetensors", model_dir);
    return iris_vae_gpu_load(path, z, scaling, shift);
}

int iris_vae_gpu_z_channels(const iris_vae_gpu_t *v) { return v ? v->z : 0; }

/* ------------------------------------------------------------------ decode */

#define ALLOC(ptr, bytes)                                   \
    do {                                                    \
        if (!((ptr) = iris_hip_malloc(bytes))) goto oom;    \
    } while (0)

static int score_rows(int S, int Kp) {
    int r = (int)(SCORE_ELEMS / (unsigned)Kp) & ~255;
    if (r < 256) r = 256;
    return r < S ? r : S;
}

/* work buffers for an image of P = H*W pixels (S = P/64 bottleneck tokens) */
static int ensure_work(iris_vae_gpu_t *v, int lh, int lw) {
    const size_t P = (size_t)256 * lh * lw;
    if (P <= v->cap_pix) return 0;
    free_work(v);
    const size_t S = P / 64, Kp = (S + 63) / 64 * 64;
    /* score_rows keeps every later, smaller call within this many scores */
    const size_t n_sc = S * Kp < SCORE_ELEMS ? S * Kp : SCORE_ELEMS;
    ALLOC(v->x, P * 256 * sizeof(float));
    ALLOC(v->y, P * 256 * sizeof(float));
    ALLOC(v->t, P * 256 * 2);
    ALLOC(v->h, P * 256 * 2);
    ALLOC(v->raw, P * 256 * 2);
    /* the statistics pass's blocks, or one per 256-pixel row tile of a
     * convolution that forms the sums in its epilogue */
    ALLOC(v->part, (size_t)(GN_BLOCKS > (P + 255) / 256 ? GN_BLOCKS : (P + 255) / 256) * VAE_GROUPS * 2 *
                       sizeof(double));
    ALLOC(v->ab, 2 * 512 * sizeof(float));
    ALLOC(v->qkv, S * 3 * VAE_MID * 2);
    ALLOC(v->att, S * VAE_MID * 2);
    ALLOC(v->vt, (size_t)VAE_MID * Kp * 2);
    /* per row chunk: (max, sum) per row and 256-column tile, (max, 1 / sum) per row */
    ALLOC(v->sst, (n_sc / 256 + S) * 2 * sizeof(float));
    ALLOC(v->srow, S * 2 * sizeof(float));
    ALLOC(v->pm, n_sc * 2);
    ALLOC(v->front, S * VAE_CIN_PAD * 2);
    v->ws_bytes = 4 * S * VAE_MID * sizeof(float);   /* split-K at the bottleneck */
    ALLOC(v->ws, v->ws_bytes);
    ALLOC(v->dlat, (size_t)v->lat_ch * lh * lw * sizeof(float));
    ALLOC(v->drgb, P * 3);
    ALLOC(v->df32, P * 3 * sizeof(float));
    ALLOC(v->dimg, P * 3 * sizeof(float));
    v->cap_pix = P;
    return 0;
oom:
    free_work(v);
    return fail("work buffers");
}

static int gn(iris_vae_gpu_t *v, const void *x, int is_bf16, int pix, int C, const float *g, const float *b,
              int swish, uint16_t *y, uint16_t *raw) {
    /* the sums from the producing convolution's epilogue, or a statistics pass */
    const int nblk = v->st_buf == x ? v->st_nblk : iris_hip_gn_stats(x, is_bf16, pix, C, VAE_GROUPS, v->part, GN_BLOCKS);
    v->st_buf = NULL;
    if (nblk < 0 || iris_hip_gn_finalize(v->part, nblk, pix, C, VAE_GROUPS, g, b, v->eps, v->ab)) return -1;
    return iris_hip_gn_apply(x, is_bf16, v->ab, pix, C, swish, y, raw);
}

/* stats: the output feeds a GroupNorm, so an unsplit convolution also forms
 * its GroupNorm sums (cout / VAE_GROUPS channels per group) */
static int conv(iris_vae_gpu_t *v, const uint16_t *in, const uint16_t *w, const float *b, void *out, int H, int W,
                int cin, int cout, int up, int epi, int stats) {
    iris_conv3x3_t c;
    memset(&c, 0, sizeof(c));
    c.in = in;
    c.wt = w;
    c.out = out;
    c.bias = b;
    c.H = H;
    c.W = W;
    c.cin = cin;
    c.cout = cout;
    c.up = up;
    c.ldo = cout;
    c.epi = epi;
    /* fewer tiles than CUs: split K (9 cin) over blocks */
    const long long tiles = ((long long)H * W + 255) / 256 * ((cout + 255) / 256);
    int splits = 1;
    while (tiles * splits * 2 <= 256 && splits < 4 && 9 * cin / 64 / (splits * 2) >= 8) splits *= 2;
    if (splits > 1 && (size_t)splits * H * W * cout * sizeof(float) <= v->ws_bytes) {
        c.splits = splits;
        c.ws = v->ws;
        c.ws_bytes = v->ws_bytes;
    }
    stats = stats && c.splits <= 1 && cout % (4 * VAE_GROUPS) == 0;
    if (stats) {
        c.gn_part = v->part;
        c.gn_groups = VAE_GROUPS;
    }
    v->st_buf = NULL;
    if (iris_hip_conv3x3(&c)) return -1;
    if (stats) {
        v->st_buf = out;
        v->st_nblk = (H * W + 255) / 256;
    }
    return 0;
}

static int gemm(iris_vae_gpu_t *v, const uint16_t *A, int lda, const uint16_t *W, int ldw, void *out, int ldo,
                const float *bias, int M, int N, int K, int epi) {
    v->st_buf = NULL;
    iris_gemm_problem_t p;
    memset(&p, 0, sizeof(p));
    p.A = A; p.W = W; p.out = out; p.vec = bias;
    p.M = M; p.N = N; p.K = K; p.lda = lda; p.ldw = ldw; p.ldo = ldo; p.epi = epi;
    return iris_hip_gemm(&p, 1);
}

static void swap(float **a, float **b) {
    float *t = *a;
    *a = *b;
    *b = t;
}

/* resblock_forward (iris_vae.c:203-251): x += conv2(swish(gn2(conv1(swish(gn1(x)))))),
 * through a 1x1 shortcut into the other stream buffer when cin != cout */
static int resblock(iris_vae_gpu_t *v, const vres_t *r, int H, int W) {
    const int P = H * W;
    if (gn(v, v->x, 0, P, r->cin, r->n1g, r->n1b, 1, v->t, r->sk ? v->raw : NULL) ||
        conv(v, v->t, r->c1, r->c1b, v->h, H, W, r->cin, r->cout, 0, IRIS_EPI_BF16, 1) ||
        gn(v, v->h, 1, P, r->cout, r->n2g, r->n2b, 1, v->t, NULL))
        return -1;
    if (r->sk) {
        if (gemm(v, v->raw, r->cin, r->sk, r->cin, v->y, r->cout, r->skb, P, r->cout, r->cin, IRIS_EPI_F32) ||
            conv(v, v->t, r->c2, r->c2b, v->y, H, W, r->cout, r->cout, 0, IRIS_EPI_ADD, 1))
            return -1;
        swap(&v->x, &v->y);
        return 0;
    }
    return conv(v, v->t, r->c2, r->c2b, v->x, H, W, r->cout, r->cout, 0, IRIS_EPI_ADD, 1);
}

/* attnblock_forward (iris_vae.c:260-357): single head over the S pixels,
 * x += out_proj(softmax(q k^T / sqrt(C)) v) in row chunks; the softmax runs
 * in the epilogues of two passes over the products (no f32 score matrix) */
static int attention(iris_vae_gpu_t *v, const vattn_t *a, int H, int W) {
    const int S = H * W, C = VAE_MID, Kp = (S + 63) / 64 * 64, R = score_rows(S, Kp);
    if (gn(v, v->x, 0, S, C, a->g, a->b, 0, v->t, NULL) ||
        gemm(v, v->t, C, a->qkv_w, C, v->qkv, 3 * C, a->qkv_b, S, 3 * C, C, IRIS_EPI_BF16) ||
        iris_hip_transpose_bf16(v->vt, Kp, Kp, v->qkv + 2 * C, 3 * C, S, C))
        return -1;
    for (int q0 = 0; q0 < S; q0 += R) {
        const int r = S - q0 < R ? S - q0 : R;
        /* q rows carry the 1/sqrt(C) scale (load_attn) */
        if (iris_hip_softmax_scores(v->qkv + (size_t)q0 * 3 * C, 3 * C, v->qkv + C, 3 * C, r, S, C, 1.0f, v->pm, Kp,
                                    Kp, v->sst, v->srow))
            return -1;
        /* P V: 512 output columns leave most CUs idle at one chunk of K; split
         * over K through the convolutions' workspace where that fills them */
        iris_gemm_problem_t p;
        memset(&p, 0, sizeof(p));
        p.A = v->pm; p.lda = Kp; p.W = v->vt; p.ldw = Kp; p.out = v->att + (size_t)q0 * C; p.ldo = C;
        p.M = r; p.N = C; p.K = Kp; p.epi = IRIS_EPI_BF16;
        v->st_buf = NULL;
        if (iris_hip_gemm_fill(&p, v->ws, v->ws_bytes)) return -1;
    }
    return gemm(v, v->att, C, a->o_w, C, v->x, C, a->o_b, S, C, C, IRIS_EPI_ADD);
}

int iris_vae_gpu_decode_device(iris_vae_gpu_t *v, const float *d_lat, int lh, int lw, uint8_t *d_rgb, float *d_f32) {
    if (!v || !d_lat || !d_rgb || lh <= 0 || lw <= 0 || 16 * lh > IRIS_VAE_MAX_DIM || 16 * lw > IRIS_VAE_MAX_DIM) {
        fprintf(stderr, "vae: latent %dx%d (image sides 16..%d)\n", lh, lw, IRIS_VAE_MAX_DIM);
        return -1;
    }
    if (ensure_work(v, lh, lw)) return -1;
    v->st_buf = NULL;
    int H = 2 * lh, W = 2 * lw;
    if (iris_hip_vae_front(v->front, d_lat, v->z, lh, lw, v->lsc, v->lsh, v->divide, v->pqw, v->pqb) ||
        conv(v, v->front, v->cin_w, v->cin_b, v->x, H, W, VAE_CIN_PAD, VAE_MID, 0, IRIS_EPI_F32, 1) ||
        resblock(v, &v->mid1, H, W) || attention(v, &v->attn, H, W) || resblock(v, &v->mid2, H, W))
        return fail("decode (mid block)");
    for (int level = 3, bi = 0; level >= 0; level--) {
        const int ch = VAE_BASE * ch_mult[level];
        for (int r = 0; r < 3; r++)
            if (resblock(v, &v->up[bi++], H, W)) return fail("decode (resblock)");
        if (level > 0) {
            /* nearest 2x + conv: the conv reads the bf16 stream through the upsample */
            if (iris_hip_f32_to_bf16(v->raw, v->x, (size_t)H * W * ch) ||
                conv(v, v->raw, v->ups_w[3 - level], v->ups_b[3 - level], v->y, 2 * H, 2 * W, ch, ch, 1,
                     IRIS_EPI_F32, 1))
                return fail("decode (upsample)");
            swap(&v->x, &v->y);
            H *= 2;
            W *= 2;
        }
    }
    if (gn(v, v->x, 0, H * W, VAE_BASE, v->no_g, v->no_b, 1, v->t, NULL) ||
        iris_hip_vae_conv_out(d_rgb, d_f32, v->t, H, W, VAE_BASE, v->co_w, v->co_b))
        return fail("decode (output)");
    return 0;
}

int iris_vae_gpu_decode_to(iris_vae_gpu_t *v, const float *latent, int lh, int lw, uint8_t *rgb, float *f32) {
    if (!v || !latent || !rgb) return -1;
    if (lh <= 0 || lw <= 0 || 16 * lh > IRIS_VAE_MAX_DIM || 16 * lw > IRIS_VAE_MAX_DIM) {
        fprintf(stderr, "vae: latent %dx%d (image sides 16..%d)\n", lh, lw, IRIS_VAE_MAX_DIM);
        return -1;
    }
    if (ensure_work(v, lh, lw)) return -1;
    const size_t P = (size_t)256 * lh * lw;
    if (iris_hip_memcpy_h2d(v->dlat, latent, (size_t)v->lat_ch * lh * lw * sizeof(float)) ||
        iris_vae_gpu_decode_device(v, v->dlat, lh, lw, v->drgb, f32 ? v->df32 : NULL) ||
        iris_hip_memcpy_d2h(rgb, v->drgb, P * 3) || (f32 && iris_hip_memcpy_d2h(f32, v->df32, P * 3 * sizeof(float))))
        return fail("decode");
    return 0;
}

iris_image *iris_vae_gpu_decode(iris_vae_gpu_t *v, const float *latent, int batch, int lh, int lw) {
    if (!v || !latent || batch < 1 || lh <= 0 || lw <= 0) return NULL;
    iris_image *img = (iris_image *)malloc(sizeof(*img));
    if (!img) return NULL;
    img->width = 16 * lw;
    img->height = 16 * lh;
    img->channels = 3;
    img->data = (uint8_t *)malloc((size_t)img->width * img->height * 3);
    if (!img->data || iris_vae_gpu_decode_to(v, latent, lh, lw, img->data, NULL)) {
        iris_image_free(img);
        return NULL;
    }
    return img;
}

void iris_image_free(iris_image *img) {
    if (!img) return;
    free(img->data);
    free(img);
}

/* ------------------------------------------------------------------ encode */

/* iris_vae_encode (iris_vae.c:363-482) for one image [3][H][W] (device),
 * H and W multiples of 16: latent [4z][H/16][W/16] (device) */
int iris_vae_gpu_encode_device(iris_vae_gpu_t *v, const float *d_img, int H, int W, float *d_lat) {
    if (!v || !d_img || !d_lat || !v->has_enc) {
        fprintf(stderr, "vae: encode needs the encoder weights\n");
        return -1;
    }
    if (H < 16 || W < 16 || H % 16 || W % 16 || H > IRIS_VAE_MAX_DIM || W > IRIS_VAE_MAX_DIM) {
        fprintf(stderr, "vae: image %dx%d (multiples of 16 up to %d)\n", H, W, IRIS_VAE_MAX_DIM);
        return -1;
    }
    if (ensure_work(v, H / 16, W / 16)) return -1;
    v->st_buf = NULL;
    if (iris_hip_vae_img_in(v->raw, d_img, H, W) ||
        conv(v, v->raw, v->e_cin_w, v->e_cin_b, v->x, H, W, VAE_CIN_PAD, VAE_BASE, 0, IRIS_EPI_F32, 1))
        return fail("encode (conv_in)");
    int h = H, w = W;
    for (int level = 0, bi = 0; level < 4; level++) {
        const int ch = VAE_BASE * ch_mult[level];
        for (int r = 0; r < 2; r++)
            if (resblock(v, &v->e_down[bi++], h, w)) return fail("encode (resblock)");
        if (level < 3) {
            /* pad right/bottom + 3x3 stride 2, in the conv's loads */
            if (iris_hip_f32_to_bf16(v->raw, v->x, (size_t)h * w * ch) ||
                conv(v, v->raw, v->e_ds_w[level], v->e_ds_b[level], v->y, h / 2, w / 2, ch, ch, 2, IRIS_EPI_F32, 1))
                return fail("encode (downsample)");
            swap(&v->x, &v->y);
            h /= 2;
            w /= 2;
        }
    }
    if (resblock(v, &v->e_mid1, h, w) || attention(v, &v->e_attn, h, w) || resblock(v, &v->e_mid2, h, w) ||
        gn(v, v->x, 0, h * w, VAE_MID, v->e_no_g, v->e_no_b, 1, v->t, NULL) ||
        conv(v, v->t, v->e_co_w, v->e_co_b, v->y, h, w, VAE_MID, 2 * v->z, 0, IRIS_EPI_F32, 0) ||
        iris_hip_vae_enc_out(d_lat, v->y, v->z, h, w, v->qw, v->qb, v->esc, v->esh))
        return fail("encode (output)");
    return 0;
}

float *iris_vae_gpu_encode(iris_vae_gpu_t *v, const float *img, int batch, int H, int W, int *out_h, int *out_w) {
    if (!v || !img || batch < 1 || H < 16 || W < 16 || H % 16 || W % 16 || H > IRIS_VAE_MAX_DIM ||
        W > IRIS_VAE_MAX_DIM || ensure_work(v, H / 16, W / 16))
        return NULL;
    const size_t per_img = (size_t)3 * H * W, per_lat = (size_t)v->lat_ch * (H / 16) * (W / 16);
    float *lat = (float *)malloc(batch * per_lat * sizeof(float));
    if (!lat) return NULL;
    for (int b = 0; b < batch; b++) {
        if (iris_hip_memcpy_h2d(v->dimg, img + b * per_img, per_img * sizeof(float)) ||
            iris_vae_gpu_encode_device(v, v->dimg, H, W, v->dlat) ||
            iris_hip_memcpy_d2h(lat + b * per_lat, v->dlat, per_lat * sizeof(float))) {
            free(lat);
            return NULL;
        }
    }
    if (out_h) *out_h = H / 16;
    if (out_w) *out_w = W / 16;
    return lat;
}

int iris_vae_gpu_has_encoder(const iris_vae_gpu_t *v) { return v ? v->has_enc : 0; }
