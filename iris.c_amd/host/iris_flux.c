/*
 * iris_flux.c - Flux.2-Klein denoiser forward of the HIP build (host C).
 *
 * Keeps the reference's entry points (iris_transformer_forward*, loaders,
 * free) and the block structure of iris_transformer_flux.c, but runs every
 * block on the device through the C ABI of iris_hip.h:
 *   - weights are uploaded once as bf16 (no per-step bf16->f32 widening,
 *     unlike the BLAS mmap path :4073-4077);
 *   - the residual stream stays f32 in HBM in [txt rows | img rows] order, so
 *     the double blocks' joint attention over cat([txt, img]) (:1899-1905) and
 *     the single blocks' concatenation (:4110-4114) need no copies;
 *   - one forward is captured once per geometry into a hipGraph and replayed
 *     (the reference's Metal path encodes one command buffer per step,
 *     :3565-3691).
 * Block functions keep the reference's names and roles:
 * double_block_forward (:2366-2614), single_block_forward (:3761-3928).
 */
#include "../../include/iris_transformer.h"
#include "../../include/iris_hip.h"
#include "../../include/iris_synth.h"
#include "../../include/iris_kernels.h"
#include "iris_st.h"
#include "iris_tables.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define MAX_REFS 8

/* The reference's LoRA state (iris_lora.h:22-51), same layout: a caller loads
 * it with the reference's lora_load and hands it to iris_transformer_set_lora. */
typedef struct {
    float *lora_A;   /* [rank][in_dim] */
    float *lora_B;   /* [out_dim][rank] */
    int rank, in_dim, out_dim;
} lora_adapter_t;

typedef struct {
    float scale;
    int num_double_blocks;
    lora_adapter_t *double_img_q, *double_img_k, *double_img_v, *double_img_proj;
    lora_adapter_t *double_txt_q, *double_txt_k, *double_txt_v, *double_txt_proj;
    int num_single_blocks;
    lora_adapter_t *single_linear1, *single_linear2;
    float *scratch;
    int scratch_len, max_rank;
} lora_state_t;

/* One adapted linear on the device: its adapters' down projections stacked
 * (dn, bf16 [rp][in], zero rows up to rp) and scale * B scattered into the
 * weight's own row order (up, bf16 [rows][rp], zero where no adapter writes).
 * The GEMM runs as [x | u] [W | up]^T with u = x dn^T. rp == 0: no adapter. */
typedef struct {
    uint16_t *dn, *up;
    int in, rows, rp;
} lora_dev_t;

typedef struct {
    uint16_t *img_qkv, *img_o, *img_ffin, *img_down;    /* ffin rows gate/up interleaved by 32 */
    uint16_t *txt_qkv, *txt_o, *txt_ffin, *txt_down;
    float *img_nq, *img_nk, *txt_nq, *txt_nk;
} dev_double_t;

typedef struct {
    uint16_t *qkv_mlp;   /* [3h + 2mlp][h]: Q,K,V rows, then gate/up interleaved by 32 */
    uint16_t *out;       /* [h][h + mlp] */
    float *nq, *nk;
} dev_single_t;

/* split-K partials of the products on few rows (iris_hip_gemm_fill_n picks the
 * chunk count that fits) */
#define FILL_WS_BYTES ((size_t)64 << 20)

typedef struct {
    int valid;
    int ih, iw, n_refs, T, B;
    int ref_h[MAX_REFS], ref_w[MAX_REFS], ref_t[MAX_REFS];
    int I0, I, S, S_pad;
    size_t cap_S;            /* rows the buffers were sized for */
    /* device buffers */
    float *x;                /* [B][S][h] residual stream */
    uint16_t *a;             /* [B][S][h] normalised activations */
    uint16_t *qkv;           /* [B][S][3h] */
    uint16_t *q, *k;         /* [B][S][h] */
    uint16_t *vt;            /* [B][heads][128][S_pad] */
    uint16_t *cat;           /* [B][S][h + mlp]: attention | SwiGLU output */
    uint16_t *tok;           /* [I][C] */
    uint16_t *txtb;          /* [B][T][text_dim] */
    float *txtf;             /* [B][T][text_dim] */
    float *lat;              /* [C][I] target then refs, NCHW per image */
    float *vel;              /* [B][C][I0] */
    float *rope_cos, *rope_sin;   /* [S][128] */
    float *rp_cos, *rp_sin;       /* [S][64]: one value per rotation pair (the attention's Q prologue) */
    int16_t *rp_pos;              /* [S][4] axis positions (T, H, W, L) of each row, with rp_axis the
                                   * factored form of rp_cos / rp_sin the Q prologue reads (NULL when
                                   * it would not reproduce them bit for bit) */
    float *rp_axis;               /* cos [rp_axis_len][16], then sin */
    int rp_axis_len;
    float *krope_cos, *krope_sin; /* [S][128] K side: the reference rows' H/W bands scaled (SREF) */
    float kshf, kslf;             /* band scales the K tables hold */
    float kgamma;                 /* SREF strength the captured graph applies */
    int csd_on;                   /* the captured graph adds d_csd (the CSD style delta, or
                                   * zeros while it is skipped) to temb */
    unsigned lora_gen;            /* tf->lora_gen the graph was captured at */
    float *tsin;             /* [256] */
    float *tmp, *temb;       /* [h] */
    float *mod;              /* dimg 6h | dtxt 6h | single 3h | final 2h */
    float *tsin_host;        /* host copy of the timestep sinusoid (small uploads are staged out of
                              * it into pinned slots before iris_hip_memcpy_h2d returns) */
    void *attn_ws;           /* the attention's balanced-schedule workspace (zeroed) */
    size_t attn_ws_bytes;
    float *fill_ws;          /* split-K partials of the products on few rows (iris_hip_gemm_fill_n) */
    void *graph;
} work_t;

struct iris_transformer {
    int hidden, heads, head_dim, mlp, n_double, n_single, text_dim, latent_ch, axis_dim;
    float theta;
    uint16_t *img_in, *txt_in, *t_fc1, *t_fc2, *mod_dimg, *mod_dtxt, *mod_single, *final_mod, *proj_out;
    uint16_t *mod_all;   /* [17 h][h]: the four modulation linears stacked (mod_dimg .. final_mod point
                          * into it), so one GEMV fills the step's modulation vector */
    dev_double_t *dbl;
    dev_single_t *sgl;
    work_t w;
    work_t w_alt;                     /* the previous geometry's workspace and graph, kept so
                                       * forwards alternating between two geometries (CFG with
                                       * two text lengths) reuse both */
    /* adapters set through the reference's setters (owned, not applied) */
    void *lora, *ip, *ip_embeds;
    void *lora_built;                 /* the LoRA state the device adapters hold, or NULL */
    int lora_dirty;                   /* set_lora was called since the last build */
    lora_dev_t *ldev;                 /* 4 per double block (img qkv, img proj, txt qkv, txt proj),
                                       * then 2 per single block (linear1, linear2); NULL: none */
    int lrp_max;                      /* widest rp of ldev, the row stride of lu */
    uint16_t *lu;                     /* [rows][lrp_max] bf16: u = x dn^T of the current linear */
    float *lws;                       /* split-K partials of the u products */
    size_t lu_rows, lws_floats;
    unsigned lora_gen;                /* bumped whenever ldev / lu / lws change: a graph captured
                                       * at another value may hold freed LoRA buffers */
    float *d_csd;                     /* device copy of the CSD style delta [hidden] */
    float *csd_delta;
    float *csd_zero;                  /* host zeros uploaded into d_csd while the delta is skipped */
    int csd_skip;
    float sref_shf, sref_slf, sref_strength;
};

/* ------------------------------------------------------------------ config */

/* parse_transformer_config, iris_transformer_flux.c:395-455 */
static int parse_config(const char *dir, iris_transformer_t *tf) {
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
    tf->heads = heads;
    tf->head_dim = hd;
    tf->hidden = heads * hd;
    tf->mlp = (int)(tf->hidden * (ratio > 0 ? ratio : 3.0f));
    tf->n_double = nl > 0 ? nl : 5;
    tf->n_single = ns > 0 ? ns : 20;
    tf->text_dim = jd > 0 ? jd : 7680;
    tf->latent_ch = ic > 0 ? ic : 128;
    tf->theta = theta > 0 ? theta : 2000.0f;
    tf->axis_dim = hd / 4;
    return 0;
}

static void defaults_4b(iris_transformer_t *tf) {   /* :5309-5321 */
    tf->hidden = 3072; tf->heads = 24; tf->head_dim = 128; tf->mlp = 9216;
    tf->n_double = 5; tf->n_single = 20; tf->text_dim = 7680; tf->latent_ch = 128;
    tf->theta = 2000.0f; tf->axis_dim = 32;
}

static int check_dims(const iris_transformer_t *tf) {
    if (tf->head_dim != 128) { fprintf(stderr, "iris_hip: head_dim %d unsupported (128)\n", tf->head_dim); return -1; }
    if (tf->hidden % 64 || tf->mlp % 64 || tf->text_dim % 64 || tf->latent_ch % 64) {
        fprintf(stderr, "iris_hip: hidden/mlp/text_dim/latent_ch must be multiples of 64\n");
        return -1;
    }
    return 0;
}

/* ------------------------------------------------------------ weight upload */

/* A source fills a host bf16 buffer for a named tensor of n elements. */
typedef struct {
    const iris_st_set_t *st;      /* safetensors, or NULL for synthetic */
    uint64_t seed;
    uint16_t *stage;
    size_t stage_n;
} source_t;

static const uint16_t *src_get(source_t *s, const char *name, size_t n, int is_norm) {
    if (s->stage_n < n) {
        free(s->stage);
        s->stage = (uint16_t *)malloc(n * sizeof(uint16_t));
        s->stage_n = s->stage ? n : 0;
        if (!s->stage) return NULL;
    }
    if (s->st) {
        const iris_st_file_t *f;
        const iris_st_tensor_t *t = iris_st_set_find(s->st, name, &f);
        if (!t) { fprintf(stderr, "Error: required tensor %s not found\n", name); return NULL; }
        if ((size_t)iris_st_numel(t) != n) {
            fprintf(stderr, "Error: tensor %s has %lld elements, expected %zu\n", name,
                    (long long)iris_st_numel(t), n);
            return NULL;
        }
        if (t->dtype == IRIS_ST_BF16) return (const uint16_t *)iris_st_ptr(f, t);   /* straight from the map */
        if (iris_st_read_bf16(f, t, s->stage)) return NULL;
        return s->stage;
    }
    iris_synth_fill_bf16(s->stage, n, iris_synth_seed(s->seed, name), 0, is_norm ? 1.0f : 0.0f, 0.02f);
    return s->stage;
}

static uint16_t *upload_bf16(source_t *s, const char *name, size_t n) {
    const uint16_t *h = src_get(s, name, n, 0);
    if (!h) return NULL;
    uint16_t *d = (uint16_t *)iris_hip_malloc(n * 2);
    if (!d || iris_hip_memcpy_h2d(d, h, n * 2)) { iris_hip_free(d); return NULL; }
    if (iris_hip_sync()) { iris_hip_free(d); return NULL; }     /* source buffer is reused */
    return d;
}

/* Uploads [rows][cols] tensors one after another into a device matrix at row offset. */
static int upload_rows(source_t *s, const char *name, uint16_t *d, size_t rows, size_t cols) {
    const uint16_t *h = src_get(s, name, rows * cols, 0);
    if (!h) return -1;
    if (iris_hip_memcpy_h2d(d, h, rows * cols * 2)) return -1;
    return iris_hip_sync();
}

/* linear_in rows are [gate (mlp rows) | up (mlp rows)] (:633-640); the device
 * copy interleaves them in groups of SWIGLU_GROUP rows (gate g, up g, gate g+1,
 * ...) so the SwiGLU epilogue of one 64-column wave tile of the GEMM holds a
 * gate column and its up column in the same lane. */
#define SWIGLU_GROUP 32
static int copy_interleaved(uint16_t *d, const uint16_t *h, size_t mlp, size_t cols) {
    const size_t G = SWIGLU_GROUP;
    for (size_t g = 0; g < mlp / G; g++) {
        if (iris_hip_memcpy_h2d(d + (2 * g) * G * cols, h + g * G * cols, G * cols * 2)) return -1;
        if (iris_hip_memcpy_h2d(d + (2 * g + 1) * G * cols, h + (mlp + g * G) * cols, G * cols * 2)) return -1;
    }
    return iris_hip_sync();
}

static int upload_interleaved(source_t *s, const char *name, uint16_t *d, size_t mlp, size_t cols) {
    const uint16_t *h = src_get(s, name, 2 * mlp * cols, 0);
    if (!h) return -1;
    return copy_interleaved(d, h, mlp, cols);
}

static float *upload_norm(source_t *s, const char *name, size_t n) {
    const uint16_t *h = src_get(s, name, n, 1);
    if (!h) return NULL;
    float tmp[4096];
    if (n > 4096) return NULL;
    for (size_t i = 0; i < n; i++) tmp[i] = iris_bf16_to_f32(h[i]);
    float *d = (float *)iris_hip_malloc(n * sizeof(float));
    if (!d || iris_hip_memcpy_h2d(d, tmp, n * sizeof(float)) || iris_hip_sync()) { iris_hip_free(d); return NULL; }
    return d;
}

static int load_weights(iris_transformer_t *tf, source_t *s) {
    size_t h = tf->hidden, mlp = tf->mlp, C = tf->latent_ch;
    char nm[256];
#define UP(dst, name, n) do { if (!((dst) = upload_bf16(s, (name), (n)))) return -1; } while (0)
    /* tensor names: iris_transformer_flux.c:5349-5497 */
    UP(tf->img_in, "x_embedder.weight", h * C);
    UP(tf->txt_in, "context_embedder.weight", h * tf->text_dim);
    UP(tf->t_fc1, "time_guidance_embed.timestep_embedder.linear_1.weight", h * 256);
    UP(tf->t_fc2, "time_guidance_embed.timestep_embedder.linear_2.weight", h * h);
    if (!(tf->mod_all = (uint16_t *)iris_hip_malloc((size_t)17 * h * h * 2))) return -1;
    tf->mod_dimg = tf->mod_all;
    tf->mod_dtxt = tf->mod_all + (size_t)6 * h * h;
    tf->mod_single = tf->mod_all + (size_t)12 * h * h;
    tf->final_mod = tf->mod_all + (size_t)15 * h * h;
    if (upload_rows(s, "double_stream_modulation_img.linear.weight", tf->mod_dimg, 6 * h, h) ||
        upload_rows(s, "double_stream_modulation_txt.linear.weight", tf->mod_dtxt, 6 * h, h) ||
        upload_rows(s, "single_stream_modulation.linear.weight", tf->mod_single, 3 * h, h) ||
        upload_rows(s, "norm_out.linear.weight", tf->final_mod, 2 * h, h))
        return -1;
    UP(tf->proj_out, "proj_out.weight", C * h);
    tf->dbl = (dev_double_t *)calloc((size_t)tf->n_double, sizeof(dev_double_t));
    tf->sgl = (dev_single_t *)calloc((size_t)tf->n_single, sizeof(dev_single_t));
    if (!tf->dbl || !tf->sgl) return -1;
    for (int i = 0; i < tf->n_double; i++) {
        dev_double_t *b = &tf->dbl[i];
        static const char *const qkv_img[3] = {"to_q", "to_k", "to_v"};
        static const char *const qkv_txt[3] = {"add_q_proj", "add_k_proj", "add_v_proj"};
        b->img_qkv = (uint16_t *)iris_hip_malloc(3 * h * h * 2);
        b->txt_qkv = (uint16_t *)iris_hip_malloc(3 * h * h * 2);
        b->img_ffin = (uint16_t *)iris_hip_malloc(2 * mlp * h * 2);
        b->txt_ffin = (uint16_t *)iris_hip_malloc(2 * mlp * h * 2);
        if (!b->img_qkv || !b->txt_qkv || !b->img_ffin || !b->txt_ffin) return -1;
        for (int j = 0; j < 3; j++) {
            snprintf(nm, sizeof(nm), "transformer_blocks.%d.attn.%s.weight", i, qkv_img[j]);
            if (upload_rows(s, nm, b->img_qkv + j * h * h, h, h)) return -1;
            snprintf(nm, sizeof(nm), "transformer_blocks.%d.attn.%s.weight", i, qkv_txt[j]);
            if (upload_rows(s, nm, b->txt_qkv + j * h * h, h, h)) return -1;
        }
        snprintf(nm, sizeof(nm), "transformer_blocks.%d.attn.to_out.0.weight", i);
        UP(b->img_o, nm, h * h);
        snprintf(nm, sizeof(nm), "transformer_blocks.%d.attn.to_add_out.weight", i);
        UP(b->txt_o, nm, h * h);
        snprintf(nm, sizeof(nm), "transformer_blocks.%d.ff.linear_in.weight", i);
        if (upload_interleaved(s, nm, b->img_ffin, mlp, h)) return -1;
        snprintf(nm, sizeof(nm), "transformer_blocks.%d.ff_context.linear_in.weight", i);
        if (upload_interleaved(s, nm, b->txt_ffin, mlp, h)) return -1;
        snprintf(nm, sizeof(nm), "transformer_blocks.%d.ff.linear_out.weight", i);
        UP(b->img_down, nm, h * mlp);
        snprintf(nm, sizeof(nm), "transformer_blocks.%d.ff_context.linear_out.weight", i);
        UP(b->txt_down, nm, h * mlp);
#define NORM(dst, fmt) do { snprintf(nm, sizeof(nm), fmt, i); if (!((dst) = upload_norm(s, nm, 128))) return -1; } while (0)
        NORM(b->img_nq, "transformer_blocks.%d.attn.norm_q.weight");
        NORM(b->img_nk, "transformer_blocks.%d.attn.norm_k.weight");
        NORM(b->txt_nq, "transformer_blocks.%d.attn.norm_added_q.weight");
        NORM(b->txt_nk, "transformer_blocks.%d.attn.norm_added_k.weight");
    }
    for (int i = 0; i < tf->n_single; i++) {
        dev_single_t *b = &tf->sgl[i];
        size_t fused = 3 * h + 2 * mlp;
        b->qkv_mlp = (uint16_t *)iris_hip_malloc(fused * h * 2);
        if (!b->qkv_mlp) return -1;
        snprintf(nm, sizeof(nm), "single_transformer_blocks.%d.attn.to_qkv_mlp_proj.weight", i);
        const uint16_t *src = src_get(s, nm, fused * h, 0);
        if (!src) return -1;
        if (iris_hip_memcpy_h2d(b->qkv_mlp, src, 3 * h * h * 2)) return -1;
        if (copy_interleaved(b->qkv_mlp + 3 * h * h, src + 3 * h * h, mlp, h)) return -1;
        snprintf(nm, sizeof(nm), "single_transformer_blocks.%d.attn.to_out.weight", i);
        UP(b->out, nm, h * (h + mlp));
        NORM(b->nq, "single_transformer_blocks.%d.attn.norm_q.weight");
        NORM(b->nk, "single_transformer_blocks.%d.attn.norm_k.weight");
#undef NORM
    }
#undef UP
    return 0;
}

static void work_free(work_t *w);
static void release_adapters(iris_transformer_t *tf);
static int adapter_active(const iris_transformer_t *tf);
static int lora_sync(iris_transformer_t *tf);
static int lora_work(iris_transformer_t *tf);
static void lora_dev_free(iris_transformer_t *tf);
static const lora_dev_t *lora_at(const iris_transformer_t *tf, int idx);
static int lora_down(iris_transformer_t *tf, const lora_dev_t *d, const uint16_t *x, int ldx, size_t r0, int M);
static void lora_seg(const iris_transformer_t *tf, iris_gemm_problem_t *p, const lora_dev_t *d, size_t r0, int row0);

void iris_transformer_free(iris_transformer_t *tf) {
    if (!tf) return;
    work_free(&tf->w);
    work_free(&tf->w_alt);
    lora_dev_free(tf);
    free(tf->csd_zero);
    iris_hip_free(tf->d_csd);
    iris_hip_free(tf->img_in); iris_hip_free(tf->txt_in); iris_hip_free(tf->t_fc1); iris_hip_free(tf->t_fc2);
    iris_hip_free(tf->mod_all); iris_hip_free(tf->proj_out);
    for (int i = 0; tf->dbl && i < tf->n_double; i++) {
        dev_double_t *b = &tf->dbl[i];
        iris_hip_free(b->img_qkv); iris_hip_free(b->img_o); iris_hip_free(b->img_ffin); iris_hip_free(b->img_down);
        iris_hip_free(b->txt_qkv); iris_hip_free(b->txt_o); iris_hip_free(b->txt_ffin); iris_hip_free(b->txt_down);
        iris_hip_free(b->img_nq); iris_hip_free(b->img_nk); iris_hip_free(b->txt_nq); iris_hip_free(b->txt_nk);
    }
    for (int i = 0; tf->sgl && i < tf->n_single; i++) {
        iris_hip_free(tf->sgl[i].qkv_mlp); iris_hip_free(tf->sgl[i].out);
        iris_hip_free(tf->sgl[i].nq); iris_hip_free(tf->sgl[i].nk);
    }
    free(tf->dbl);
    free(tf->sgl);
    release_adapters(tf);
    free(tf);
}

static iris_transformer_t *finish_load(iris_transformer_t *tf, source_t *s) {
    tf->sref_shf = tf->sref_slf = tf->sref_strength = 1.0f;
    int rc = load_weights(tf, s);
    free(s->stage);
    if (rc) {
        fprintf(stderr, "iris_transformer_load: weight upload failed: %s\n", iris_hip_last_error());
        iris_transformer_free(tf);
        return NULL;
    }
    return tf;
}

iris_transformer_t *iris_transformer_load_safetensors(const char *model_dir) {
    if (!iris_hip_available()) {
        fprintf(stderr, "iris_transformer_load: no usable HIP device: %s\n", iris_hip_last_error());
        return NULL;
    }
    iris_transformer_t *tf = (iris_transformer_t *)calloc(1, sizeof(*tf));
    if (!tf) return NULL;
    if (parse_config(model_dir, tf)) defaults_4b(tf);
    if (check_dims(tf)) { free(tf); return NULL; }
    iris_st_set_t st;
    if (iris_st_set_open(&st, model_dir)) {
        fprintf(stderr, "iris_transformer_load: failed to open safetensors files\n");
        free(tf);
        return NULL;
    }
    source_t s = {&st, 0, NULL, 0};
    tf = finish_load(tf, &s);
    iris_st_set_close(&st);
    return tf;
}

/* The weights are device-resident either way; mmap mode only changes how the
 * reference's CPU path pages them (:5550-5683). */
iris_transformer_t *iris_transformer_load_safetensors_mmap(const char *model_dir) {
    return iris_transformer_load_safetensors(model_dir);
}

void iris_transformer_free_mmap_cache(iris_transformer_t *tf) { (void)tf; }

iris_transformer_t *iris_transformer_create_synthetic(int hidden, int heads, int n_double, int n_single,
                                                      int text_dim, int latent_ch, float mlp_ratio,
                                                      float rope_theta, uint64_t seed) {
    if (!iris_hip_available()) {
        fprintf(stderr, "iris_transformer_create_synthetic: no usable HIP device: %s\n", iris_hip_last_error());
        return NULL;
    }
    iris_transformer_t *tf = (iris_transformer_t *)calloc(1, sizeof(*tf));
    if (!tf) return NULL;
    tf->hidden = hidden; tf->heads = heads; tf->head_dim = hidden / heads;
    tf->mlp = (int)(hidden * mlp_ratio); tf->n_double = n_double; tf->n_single = n_single;
    tf->text_dim = text_dim; tf->latent_ch = latent_ch; tf->theta = rope_theta;
    tf->axis_dim = tf->head_dim / 4;
    if (check_dims(tf)) { free(tf); return NULL; }
    source_t s = {NULL, seed, NULL, 0};
    return finish_load(tf, &s);
}

int iris_transformer_hidden_size(iris_transformer_t *tf) { return tf->hidden; }
int iris_transformer_num_double_layers(iris_transformer_t *tf) { return tf->n_double; }
int iris_transformer_num_single_layers(iris_transformer_t *tf) { return tf->n_single; }
int iris_transformer_text_dim(iris_transformer_t *tf) { return tf->text_dim; }

/* -------------------------------------------------------------- workspace */

static void work_free(work_t *w) {
    iris_hip_graph_destroy(w->graph);
    void *bufs[] = {w->x, w->a, w->qkv, w->q, w->k, w->vt, w->cat, w->tok, w->txtb, w->txtf, w->lat, w->vel,
                    w->rope_cos, w->rope_sin, w->rp_cos, w->rp_sin, w->rp_pos, w->rp_axis, w->krope_cos, w->krope_sin,
                    w->tsin, w->tmp,
                    w->temb, w->mod, w->attn_ws, w->fill_ws};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++) iris_hip_free(bufs[i]);
    free(w->tsin_host);
    memset(w, 0, sizeof(*w));
}

/* The Q prologue's pair tables in factored form: every row's axis positions
 * (text row t: (0, 0, 0, t); image row (y, x) of a latent with T-offset o:
 * (o, y, x, 0), iris_transformer_flux.c:896-1087) and one table of the four
 * axes' shared frequencies per position. Kept only when it reproduces the
 * [S][64] tables bit for bit (pc, ps); otherwise the prologue reads those. */
static int factored_rope(work_t *w, const float *pc, const float *ps, int T, int ih, int iw, const iris_ref_t *refs,
                         int n_refs, int axis_dim, float theta) {
    if (axis_dim != 32) return 0;   /* four axes of 16 pairs */
    const size_t S = w->S;
    int len = T > ih ? T : ih;
    if (iw > len) len = iw;
    for (int r = 0; r < n_refs; r++) {
        if (refs[r].t_offset < 0) return 0;
        if (refs[r].h > len) len = refs[r].h;
        if (refs[r].w > len) len = refs[r].w;
        if (refs[r].t_offset + 1 > len) len = refs[r].t_offset + 1;
    }
    if (len > (1 << 15)) return 0;
    int16_t *pos = (int16_t *)calloc(S * 4, sizeof(int16_t));
    float *tab = (float *)malloc((size_t)len * 32 * sizeof(float));
    if (!pos || !tab) { free(pos); free(tab); return -1; }
    size_t row = 0;
    for (int t = 0; t < T; t++, row++) pos[row * 4 + 3] = (int16_t)t;
    for (int r = -1; r < n_refs; r++) {
        const int hh = r < 0 ? ih : refs[r].h, ww = r < 0 ? iw : refs[r].w, to = r < 0 ? 0 : refs[r].t_offset;
        for (int y = 0; y < hh; y++)
            for (int x = 0; x < ww; x++, row++) {
                pos[row * 4] = (int16_t)to;
                pos[row * 4 + 1] = (int16_t)y;
                pos[row * 4 + 2] = (int16_t)x;
            }
    }
    iris_rope_axis(tab, tab + (size_t)len * 16, len, axis_dim, theta);
    int same = row == S;
    for (size_t q = 0; same && q < S; q++)
        for (int i = 0; i < 64 && same; i++) {
            const int p = pos[q * 4 + i / 16];
            same = !memcmp(&pc[q * 64 + i], &tab[p * 16 + i % 16], 4) &&
                   !memcmp(&ps[q * 64 + i], &tab[((size_t)len + p) * 16 + i % 16], 4);
        }
    int rc = 0;
    if (same) {
        w->rp_pos = (int16_t *)iris_hip_malloc(S * 4 * sizeof(int16_t));
        w->rp_axis = (float *)iris_hip_malloc((size_t)len * 32 * sizeof(float));
        w->rp_axis_len = len;
        rc = !w->rp_pos || !w->rp_axis || iris_hip_memcpy_h2d(w->rp_pos, pos, S * 4 * sizeof(int16_t)) ||
             iris_hip_memcpy_h2d(w->rp_axis, tab, (size_t)len * 32 * sizeof(float)) || iris_hip_sync();
    }
    free(pos);
    free(tab);
    return rc ? -1 : 0;
}

static int same_geometry(const work_t *w, int ih, int iw, const iris_ref_t *refs, int n, int T, int B) {
    if (!w->valid || w->ih != ih || w->iw != iw || w->n_refs != n || w->T != T || w->B != B) return 0;
    for (int r = 0; r < n; r++)
        if (w->ref_h[r] != refs[r].h || w->ref_w[r] != refs[r].w || w->ref_t[r] != refs[r].t_offset) return 0;
    return 1;
}

static int enqueue_forward(iris_transformer_t *tf);

/* K-side RoPE tables: the Q tables with the H and W bands of the reference
 * rows [T + I0, S) scaled by s(d) = shf + (slf - shf) (d / 15)^2 per rotation
 * pair d (band_scale_ref_krope, iris_transformer_flux.c:1255-1280; a scalar
 * per pair commutes with the rotation, so it scales that band's share of
 * q . k). Text and target rows are unchanged. */
static int fill_ktables(iris_transformer_t *tf, const float *c, const float *s) {
    work_t *w = &tf->w;
    const size_t n = (size_t)w->S * 128;
    float *kc = (float *)malloc(n * sizeof(float)), *ks = (float *)malloc(n * sizeof(float));
    if (!kc || !ks) { free(kc); free(ks); return -1; }
    memcpy(kc, c, n * sizeof(float));
    memcpy(ks, s, n * sizeof(float));
    const float shf = tf->sref_shf, slf = tf->sref_slf;
    const int ad = tf->axis_dim, half = ad / 2;
    if (w->n_refs > 0 && (shf != 1.0f || slf != 1.0f)) {
        float sd[64];
        for (int d = 0; d < half && d < 64; d++) {
            const float dn = half > 1 ? (float)d / (float)(half - 1) : 0.0f;
            sd[d] = shf + (slf - shf) * dn * dn;
        }
        for (int pos = w->T + w->I0; pos < w->S; pos++) {
            float *cr = kc + (size_t)pos * 128, *sr = ks + (size_t)pos * 128;
            for (int d = 0; d < half; d++) {
                const int hh = ad + d * 2, ww = ad * 2 + d * 2;
                cr[hh] *= sd[d]; cr[hh + 1] *= sd[d]; sr[hh] *= sd[d]; sr[hh + 1] *= sd[d];
                cr[ww] *= sd[d]; cr[ww + 1] *= sd[d]; sr[ww] *= sd[d]; sr[ww + 1] *= sd[d];
            }
        }
    }
    const int rc = iris_hip_memcpy_h2d(w->krope_cos, kc, n * 4) || iris_hip_memcpy_h2d(w->krope_sin, ks, n * 4) ||
                   iris_hip_sync();
    free(kc);
    free(ks);
    if (rc) return -1;
    w->kshf = shf;
    w->kslf = slf;
    return 0;
}

/* (re)capture one forward into the step graph */
static int capture(iris_transformer_t *tf) {
    work_t *w = &tf->w;
    if (w->graph) { iris_hip_graph_destroy(w->graph); w->graph = NULL; }
    w->kgamma = tf->sref_strength;
    w->csd_on = tf->csd_delta != NULL;
    w->lora_gen = tf->lora_gen;
    if (w->csd_on && !tf->d_csd && !(tf->d_csd = (float *)iris_hip_malloc((size_t)tf->hidden * 4))) return -1;
    if (iris_hip_graph_begin()) return -1;
    if (enqueue_forward(tf)) {
        void *g = iris_hip_graph_end();
        iris_hip_graph_destroy(g);
        return -1;
    }
    w->graph = iris_hip_graph_end();
    return w->graph ? 0 : -1;
}

int iris_flux_prepare(iris_transformer_t *tf, int ih, int iw, const iris_ref_t *refs, int n_refs, int T, int B) {
    work_t *w = &tf->w;
    if (n_refs < 0 || n_refs > MAX_REFS) { fprintf(stderr, "iris_hip: %d references (max %d)\n", n_refs, MAX_REFS); return -1; }
    if (B < 1 || B > 2) { fprintf(stderr, "iris_hip: batch %d (1 or 2)\n", B); return -1; }
    if (ih <= 0 || iw <= 0 || T <= 0) { fprintf(stderr, "iris_hip: empty geometry\n"); return -1; }
    if (same_geometry(w, ih, iw, refs, n_refs, T, B)) return 0;
    if (same_geometry(&tf->w_alt, ih, iw, refs, n_refs, T, B)) {
        const work_t t = tf->w;
        tf->w = tf->w_alt;
        tf->w_alt = t;
        return 0;
    }
    /* the current workspace becomes the alternate one */
    work_free(&tf->w_alt);
    tf->w_alt = tf->w;
    memset(w, 0, sizeof(*w));
    int h = tf->hidden, mlp = tf->mlp, C = tf->latent_ch, td = tf->text_dim, H = tf->heads;
    w->ih = ih; w->iw = iw; w->n_refs = n_refs; w->T = T; w->B = B;
    w->I0 = ih * iw;
    w->I = w->I0;
    for (int r = 0; r < n_refs; r++) {
        w->ref_h[r] = refs[r].h; w->ref_w[r] = refs[r].w; w->ref_t[r] = refs[r].t_offset;
        w->I += refs[r].h * refs[r].w;
    }
    w->S = w->I + T;
    w->S_pad = (w->S + 63) / 64 * 64;
    size_t S = w->S, BS = (size_t)B * S;
#define DA(dst, bytes) do { if (!((dst) = iris_hip_malloc(bytes))) goto fail; } while (0)
    DA(w->x, BS * h * 4);
    DA(w->a, BS * h * 2);
    DA(w->qkv, BS * 3 * h * 2);
    DA(w->q, BS * h * 2);
    DA(w->k, BS * h * 2);
    DA(w->vt, (size_t)B * H * 128 * w->S_pad * 2);
    DA(w->cat, BS * (h + mlp) * 2);
    DA(w->tok, (size_t)w->I * C * 2);
    DA(w->txtb, (size_t)B * T * td * 2);
    DA(w->txtf, (size_t)B * T * td * 4);
    DA(w->lat, (size_t)w->I * C * 4);
    DA(w->vel, (size_t)B * C * w->I0 * 4);
    DA(w->rope_cos, S * 128 * 4);
    DA(w->krope_cos, S * 128 * 4);
    DA(w->krope_sin, S * 128 * 4);
    DA(w->rope_sin, S * 128 * 4);
    DA(w->rp_cos, S * 64 * 4);
    DA(w->rp_sin, S * 64 * 4);
    DA(w->tsin, 256 * 4);
    DA(w->tmp, (size_t)h * 4);
    DA(w->temb, (size_t)h * 4);
    DA(w->mod, (size_t)17 * h * 4);
    w->attn_ws_bytes = iris_hip_attention_workspace_bytes();
    DA(w->attn_ws, w->attn_ws_bytes);
    DA(w->fill_ws, FILL_WS_BYTES);
    if (iris_hip_memset(w->attn_ws, 0, w->attn_ws_bytes) || iris_hip_sync()) goto fail;
#undef DA
    w->tsin_host = (float *)malloc(256 * sizeof(float));
    if (!w->tsin_host) goto fail;
    /* RoPE tables in sequence order: txt rows, target, references (:4634-4657) */
    {
        float *c = (float *)malloc(S * 128 * sizeof(float)), *s = (float *)malloc(S * 128 * sizeof(float));
        if (!c || !s) { free(c); free(s); goto fail; }
        iris_rope_txt(c, s, T, tf->axis_dim, tf->theta);
        size_t off = (size_t)T * 128;
        iris_rope_img(c + off, s + off, ih, iw, tf->axis_dim, tf->theta, 0);
        off += (size_t)w->I0 * 128;
        for (int r = 0; r < n_refs; r++) {
            iris_rope_img(c + off, s + off, refs[r].h, refs[r].w, tf->axis_dim, tf->theta, refs[r].t_offset);
            off += (size_t)refs[r].h * refs[r].w * 128;
        }
        float *pc = (float *)malloc(S * 64 * sizeof(float)), *ps = (float *)malloc(S * 64 * sizeof(float));
        int rc = !pc || !ps;
        if (!rc) iris_rope_pairs(pc, ps, c, s, S);
        if (!rc) rc = factored_rope(w, pc, ps, T, ih, iw, refs, n_refs, tf->axis_dim, tf->theta);
        rc = rc || iris_hip_memcpy_h2d(w->rope_cos, c, S * 128 * 4) || iris_hip_memcpy_h2d(w->rope_sin, s, S * 128 * 4) ||
             iris_hip_memcpy_h2d(w->rp_cos, pc, S * 64 * 4) || iris_hip_memcpy_h2d(w->rp_sin, ps, S * 64 * 4) ||
             iris_hip_sync() || fill_ktables(tf, c, s);
        free(c); free(s); free(pc); free(ps);
        if (rc) goto fail;
    }
    w->valid = 1;
    if (lora_work(tf) < 0 || capture(tf)) goto fail;
    return 0;
fail:
    fprintf(stderr, "iris_flux_prepare: %s\n", iris_hip_last_error());
    work_free(w);
    return -1;
}

/* ------------------------------------------------------------- the forward */

#define CK(x) do { if ((x) != 0) return -1; } while (0)

static int gemm(const iris_gemm_problem_t *p, int n) { return iris_hip_gemm(p, n); }
/* products on few rows (one launch of n problems): split-K through the
 * forward's workspace when their tiles leave most of the chip idle */
static int gemm_fill(iris_transformer_t *tf, const iris_gemm_problem_t *p, int n) {
    return iris_hip_gemm_fill_n(p, n, tf->w.fill_ws, FILL_WS_BYTES);
}

static iris_gemm_problem_t prob(const void *A, int lda, const uint16_t *W, int ldw, void *out, int ldo,
                                const float *vec, int M, int N, int K, int epi) {
    iris_gemm_problem_t p;
    memset(&p, 0, sizeof(p));
    p.A = (const uint16_t *)A; p.lda = lda; p.W = W; p.ldw = ldw; p.out = out; p.ldo = ldo;
    p.vec = vec; p.M = M; p.N = N; p.K = K; p.epi = epi;
    return p;
}

/* K-RMSNorm + RoPE of each stream and V^T for every batch slot (the Q half
 * runs in the attention kernel's prologue). kside: K rotates with the K-side
 * tables (the SREF band control), which the reference applies in
 * single-stream blocks only (iris_transformer_flux.c:3866-3873); its double
 * blocks rotate K with the plain tables (:2449-2450). */
static int kv_prepare(iris_transformer_t *tf, const float *wkA, const float *wkB, int split, int kside) {
    work_t *w = &tf->w;
    int h = tf->hidden;
    for (int b = 0; b < w->B; b++) {
        iris_qkprep_args_t a;
        memset(&a, 0, sizeof(a));
        a.qkv = w->qkv + (size_t)b * w->S * 3 * h;
        a.ld_qkv = 3 * h; a.col_k = h; a.col_v = 2 * h;
        a.k_out = w->k + (size_t)b * w->S * h;
        a.vt_out = w->vt + (size_t)b * tf->heads * 128 * w->S_pad;
        a.ld_vt = w->S_pad;
        a.rows = w->S; a.heads = tf->heads;
        a.wkA = wkA; a.wkB = wkB; a.split = split;
        a.cos_t = w->rope_cos; a.sin_t = w->rope_sin;
        if (kside) { a.kcos_t = w->krope_cos; a.ksin_t = w->krope_sin; }
        a.eps = 1e-6f;
        CK(iris_hip_kv_prepare(&a));
    }
    return 0;
}

/* joint attention over the resident sequence; Q (columns [0, h) of qkv) is
 * QK-normalised (wqA for rows < split, else wqB) and rotated in the kernel's
 * prologue */
static int attention(iris_transformer_t *tf, const float *wqA, const float *wqB, int split, uint16_t *o, int ld_o) {
    work_t *w = &tf->w;
    int h = tf->hidden;
    iris_attn_args_t a;
    memset(&a, 0, sizeof(a));
    a.q = w->qkv; a.k = w->k; a.vt = w->vt; a.o = o;
    a.ld_q = 3 * h; a.ld_k = h; a.ld_vt = w->S_pad; a.ld_o = ld_o;
    a.sq = w->S; a.sk = w->S; a.heads = tf->heads; a.batch = w->B;
    a.q_bstride = (long long)w->S * 3 * h; a.k_bstride = (long long)w->S * h;
    a.vt_bstride = (long long)tf->heads * 128 * w->S_pad; a.o_bstride = (long long)w->S * ld_o;
    a.scale = 1.0f / sqrtf(128.0f);
    a.kv_lo0 = 0; a.kv_hi0 = w->S;
    a.qn_wA = wqA; a.qn_wB = wqB; a.qn_split = split; a.qn_eps = 1e-6f;
    a.rope_cos = w->rp_cos; a.rope_sin = w->rp_sin;
    if (w->rp_pos) { a.rope_pos = w->rp_pos; a.rope_axis = w->rp_axis; a.rope_axis_len = w->rp_axis_len; }
    a.ws = w->attn_ws; a.ws_bytes = w->attn_ws_bytes;
    /* SREF strength (sref_set_strength_bias, iris_transformer_flux.c:1328-1338):
     * log gamma on the logits of the reference keys, the trailing I - I0 tokens */
    if (w->n_refs > 0 && tf->sref_strength != 1.0f) {
        a.bias_from = w->S - (w->I - w->I0);
        a.key_bias = logf(tf->sref_strength);
    }
    return iris_hip_attention(&a);
}

static int adaln(iris_transformer_t *tf, const float *shA, const float *scA, const float *shB, const float *scB,
                 int split) {
    work_t *w = &tf->w;
    iris_norm_args_t a;
    memset(&a, 0, sizeof(a));
    a.x = w->x; a.ldx = tf->hidden; a.out = w->a; a.ldo = tf->hidden; a.out_bf16 = 1;
    a.rows = w->B * w->S; a.cols = tf->hidden; a.mode = IRIS_NORM_LN_MOD; a.eps = 1e-6f;
    a.split = split; a.period = w->S;
    a.shiftA = shA; a.scaleA = scA; a.shiftB = shB; a.scaleB = scB;
    return iris_hip_rownorm(&a);
}

/* double_block_forward, iris_transformer_flux.c:2366-2614: per batch slot,
 * txt rows [0, T) use the txt weights/modulation, img rows [T, S) the img ones. */
static int double_block_forward(iris_transformer_t *tf, int i) {
    work_t *w = &tf->w;
    const dev_double_t *bw = &tf->dbl[i];
    int h = tf->hidden, mlp = tf->mlp, T = w->T, I = w->I, S = w->S, B = w->B, hm = h + mlp;
    const float *mi = w->mod, *mt = w->mod + 6 * h;      /* shift1 scale1 gate1 shift2 scale2 gate2 */
    iris_gemm_problem_t p[4];
    int n;
    const lora_dev_t *l_iq = lora_at(tf, 4 * i), *l_ip = lora_at(tf, 4 * i + 1);
    const lora_dev_t *l_tq = lora_at(tf, 4 * i + 2), *l_tp = lora_at(tf, 4 * i + 3);
    /* AdaLN (shift1, scale1) -> Q, K, V per stream */
    CK(adaln(tf, mt, mt + h, mi, mi + h, T));
    n = 0;
    for (int b = 0; b < B; b++) {
        size_t r0 = (size_t)b * S;
        CK(lora_down(tf, l_tq, w->a + r0 * h, h, r0, T));
        CK(lora_down(tf, l_iq, w->a + (r0 + T) * h, h, r0 + T, I));
        p[n] = prob(w->a + r0 * h, h, bw->txt_qkv, h, w->qkv + r0 * 3 * h, 3 * h, NULL, T, 3 * h, h, IRIS_EPI_BF16);
        lora_seg(tf, &p[n++], l_tq, r0, 0);
        p[n] = prob(w->a + (r0 + T) * h, h, bw->img_qkv, h, w->qkv + (r0 + T) * 3 * h, 3 * h, NULL, I, 3 * h, h,
                    IRIS_EPI_BF16);
        lora_seg(tf, &p[n++], l_iq, r0 + T, 0);
    }
    CK(gemm(p, n));
    CK(kv_prepare(tf, bw->txt_nk, bw->img_nk, T, 0));
    /* joint attention over [txt, img] -> cat[:, 0:h] */
    CK(attention(tf, bw->txt_nq, bw->img_nq, T, w->cat, hm));
    /* output projections, gated residual (gate1) */
    n = 0;
    for (int b = 0; b < B; b++) {
        size_t r0 = (size_t)b * S;
        CK(lora_down(tf, l_tp, w->cat + r0 * hm, hm, r0, T));
        CK(lora_down(tf, l_ip, w->cat + (r0 + T) * hm, hm, r0 + T, I));
        p[n] = prob(w->cat + r0 * hm, hm, bw->txt_o, h, w->x + r0 * h, h, mt + 2 * h, T, h, h, IRIS_EPI_GATED_ADD);
        lora_seg(tf, &p[n++], l_tp, r0, 0);
        p[n] = prob(w->cat + (r0 + T) * hm, hm, bw->img_o, h, w->x + (r0 + T) * h, h, mi + 2 * h, I, h, h,
                    IRIS_EPI_GATED_ADD);
        lora_seg(tf, &p[n++], l_ip, r0 + T, 0);
    }
    CK(gemm_fill(tf, p, n));
    /* AdaLN (shift2, scale2) -> SwiGLU FFN -> gated residual (gate2) */
    CK(adaln(tf, mt + 3 * h, mt + 4 * h, mi + 3 * h, mi + 4 * h, T));
    n = 0;
    for (int b = 0; b < B; b++) {
        size_t r0 = (size_t)b * S;
        p[n++] = prob(w->a + r0 * h, h, bw->txt_ffin, h, w->cat + r0 * hm + h, hm, NULL, T, 2 * mlp, h, IRIS_EPI_SWIGLU);
        p[n++] = prob(w->a + (r0 + T) * h, h, bw->img_ffin, h, w->cat + (r0 + T) * hm + h, hm, NULL, I, 2 * mlp, h,
                      IRIS_EPI_SWIGLU);
    }
    CK(gemm(p, n));
    n = 0;
    for (int b = 0; b < B; b++) {
        size_t r0 = (size_t)b * S;
        p[n++] = prob(w->cat + r0 * hm + h, hm, bw->txt_down, mlp, w->x + r0 * h, h, mt + 5 * h, T, h, mlp,
                      IRIS_EPI_GATED_ADD);
        p[n++] = prob(w->cat + (r0 + T) * hm + h, hm, bw->img_down, mlp, w->x + (r0 + T) * h, h, mi + 5 * h, I, h, mlp,
                      IRIS_EPI_GATED_ADD);
    }
    CK(gemm_fill(tf, p, n));
    return 0;
}

/* single_block_forward, iris_transformer_flux.c:3761-3928 */
static int single_block_forward(iris_transformer_t *tf, int i) {
    work_t *w = &tf->w;
    const dev_single_t *bw = &tf->sgl[i];
    int h = tf->hidden, mlp = tf->mlp, hm = h + mlp, BS = w->B * w->S;
    const float *ms = w->mod + 12 * h;                   /* shift scale gate */
    const lora_dev_t *l1 = lora_at(tf, 4 * tf->n_double + 2 * i), *l2 = lora_at(tf, 4 * tf->n_double + 2 * i + 1);
    CK(adaln(tf, ms, ms + h, ms, ms + h, w->S));
    /* the first linear's two parts: Q,K,V rows -> qkv; gate/up rows -> SwiGLU
     * -> cat[:, h:] */
    iris_gemm_problem_t p[2];
    CK(lora_down(tf, l1, w->a, h, 0, BS));
    p[0] = prob(w->a, h, bw->qkv_mlp, h, w->qkv, 3 * h, NULL, BS, 3 * h, h, IRIS_EPI_BF16);
    lora_seg(tf, &p[0], l1, 0, 0);
    p[1] = prob(w->a, h, bw->qkv_mlp + (size_t)3 * h * h, h, w->cat + h, hm, NULL, BS, 2 * mlp, h, IRIS_EPI_SWIGLU);
    lora_seg(tf, &p[1], l1, 0, 3 * h);
    /* The gate/up product feeds only the output projection: it runs on the
     * side stream beside the QKV product, the K/V preparation and the
     * attention (it fills the attention's part-empty second round of blocks
     * and the products' store bursts). With the per-kernel profile on, the
     * same launches run one after the other so each is timed alone. The two
     * write disjoint 128-byte-aligned column ranges of cat. */
    const int side = !iris_hip_profile_enabled();
    if (side) {
        CK(iris_hip_fork());
        iris_hip_side(1);
    }
    /* once forked, the side stream is joined whatever fails after the fork
     * (an unjoined fork would leave a graph capture unable to end) */
    int rc = gemm(&p[1], 1);
    iris_hip_side(0);
    if (!rc) rc = gemm(&p[0], 1);
    if (!rc) rc = kv_prepare(tf, bw->nk, bw->nk, w->S, 1);
    if (!rc) rc = attention(tf, bw->nq, bw->nq, w->S, w->cat, hm);
    if (side && iris_hip_join() && !rc) rc = -1;
    CK(rc);
    /* [attn | mlp] . W_out^T, gated residual */
    CK(lora_down(tf, l2, w->cat, hm, 0, BS));
    p[0] = prob(w->cat, hm, bw->out, hm, w->x, h, ms + 2 * h, BS, h, hm, IRIS_EPI_GATED_ADD);
    lora_seg(tf, &p[0], l2, 0, 0);
    CK(gemm_fill(tf, p, 1));
    return 0;
}

static int enqueue_forward(iris_transformer_t *tf) {
    work_t *w = &tf->w;
    int h = tf->hidden, C = tf->latent_ch, td = tf->text_dim, T = w->T, I0 = w->I0, S = w->S, B = w->B;
    /* timestep MLP (:1366-1379) and the modulation GEMVs on SiLU(t_emb) (:4059-4069,
     * :3787-3797, :4270-4277); the single-block modulation is the same for all
     * 20 blocks and is computed once */
    /* The embedders below and the GEMV chain here are independent (token
     * rows and residual stream vs the time embedding and modulation vector):
     * the embedders run on the side stream beside the GEMVs, joined before
     * the first block; one after the other while profiling. */
    const int side = !iris_hip_profile_enabled();
    if (side) CK(iris_hip_fork());
    int rc = iris_hip_gemv(w->tmp, tf->t_fc1, w->tsin, NULL, h, 256, 0);
    /* the CSD style delta is added to temb before its SiLU (iris_transformer_flux.c:3969-3972):
     * the bias of the second time-MLP linear */
    if (!rc) rc = iris_hip_gemv(w->temb, tf->t_fc2, w->tmp, w->csd_on ? tf->d_csd : NULL, h, h, 1);
    /* the four modulation linears in one GEMV over their stacked rows:
     * mod = dimg 6h | dtxt 6h | single 3h | final 2h */
    if (!rc) rc = iris_hip_gemv(w->mod, tf->mod_all, w->temb, NULL, 17 * h, h, 1);
    iris_hip_side(side);
    /* NCHW -> token rows for the target and each reference (:3986-3993, :4667-4689) */
    size_t off = 0;
    if (!rc) rc = iris_hip_nchw_to_tokens(w->tok, w->lat, C, I0);
    off = I0;
    for (int r = 0; r < w->n_refs && !rc; r++) {
        int rs = w->ref_h[r] * w->ref_w[r];
        rc = iris_hip_nchw_to_tokens(w->tok + off * C, w->lat + off * C, C, rs);
        off += rs;
    }
    if (!rc) rc = iris_hip_f32_to_bf16(w->txtb, w->txtf, (size_t)B * T * td);
    /* img_in / txt_in into the residual stream rows [T, S) and [0, T) (:4022-4031):
     * the image rows (K = latent channels) in one launch, then each text
     * stream (K = text_dim, few rows) split over K */
    iris_gemm_problem_t p[4];
    int n = 0;
    for (int b = 0; b < B; b++)
        p[n++] = prob(w->tok, C, tf->img_in, C, w->x + ((size_t)b * S + T) * h, h, NULL, w->I, h, C, IRIS_EPI_F32);
    if (!rc) rc = gemm(p, n);
    for (int b = 0; b < B && !rc; b++) {
        p[0] = prob(w->txtb + (size_t)b * T * td, td, tf->txt_in, td, w->x + (size_t)b * S * h, h, NULL, T, h, td,
                    IRIS_EPI_F32);
        rc = gemm_fill(tf, p, 1);
    }
    iris_hip_side(0);
    /* once forked, the side stream is joined whatever failed after the fork */
    if (side && iris_hip_join() && !rc) rc = -1;
    CK(rc);
    for (int i = 0; i < tf->n_double; i++) CK(double_block_forward(tf, i));
    for (int i = 0; i < tf->n_single; i++) CK(single_block_forward(tf, i));
    /* final layer on the target rows: AdaLN with (scale, shift) order, proj_out,
     * written transposed to NCHW (:4254-4301) */
    const float *fm = w->mod + 15 * h;
    for (int b = 0; b < B; b++) {
        iris_norm_args_t a;
        memset(&a, 0, sizeof(a));
        a.x = w->x + ((size_t)b * S + T) * h; a.ldx = h;
        a.out = w->a + (size_t)b * I0 * h; a.ldo = h; a.out_bf16 = 1;
        a.rows = I0; a.cols = h; a.mode = IRIS_NORM_LN_MOD; a.eps = 1e-6f;
        a.split = I0; a.shiftA = fm + h; a.scaleA = fm;
        CK(iris_hip_rownorm(&a));
        p[0] = prob(w->a + (size_t)b * I0 * h, h, tf->proj_out, h, w->vel + (size_t)b * C * I0, I0, NULL, I0, C, h,
                    IRIS_EPI_F32_T);
        CK(gemm_fill(tf, p, 1));
    }
    return 0;
}

/* One block on the resident stream (x, modulation, RoPE tables as uploaded),
 * outside the captured graph: the block functions of the reference
 * (double_block_forward :2366, single_block_forward :3761) as C entry points. */
int iris_flux_double_block_forward(iris_transformer_t *tf, int idx) {
    if (!tf->w.valid || idx < 0 || idx >= tf->n_double) return -1;
    if (lora_sync(tf) < 0 || lora_work(tf) < 0) return -1;
    if (double_block_forward(tf, idx)) return -1;
    return iris_hip_sync();
}

int iris_flux_single_block_forward(iris_transformer_t *tf, int idx) {
    if (!tf->w.valid || idx < 0 || idx >= tf->n_single) return -1;
    if (lora_sync(tf) < 0 || lora_work(tf) < 0) return -1;
    if (single_block_forward(tf, idx)) return -1;
    return iris_hip_sync();
}

/* -------------------------------------------------------- step entry points */

int iris_flux_upload(iris_transformer_t *tf, const float *latent, const iris_ref_t *refs, const float *txt) {
    work_t *w = &tf->w;
    if (!w->valid) return -1;
    int C = tf->latent_ch;
    if (latent && iris_hip_memcpy_h2d(w->lat, latent, (size_t)C * w->I0 * 4)) return -1;
    size_t off = w->I0;
    for (int r = 0; refs && r < w->n_refs; r++) {
        size_t rs = (size_t)w->ref_h[r] * w->ref_w[r];
        if (iris_hip_memcpy_h2d(w->lat + off * C, refs[r].latent, C * rs * 4)) return -1;
        off += rs;
    }
    if (txt && iris_hip_memcpy_h2d(w->txtf, txt, (size_t)w->B * w->T * tf->text_dim * 4)) return -1;
    return iris_hip_sync();
}

int iris_flux_velocity(iris_transformer_t *tf, float t) {
    work_t *w = &tf->w;
    if (!w->valid) return -1;
    if (adapter_active(tf)) return -1;
    if (lora_sync(tf) || lora_work(tf) < 0) return -1;
    /* SREF settings changed since the graph was captured */
    if (w->kshf != tf->sref_shf || w->kslf != tf->sref_slf) {
        const size_t n = (size_t)w->S * 128;
        float *c = (float *)malloc(n * 4), *s = (float *)malloc(n * 4);
        const int rc = !c || !s || iris_hip_memcpy_d2h(c, w->rope_cos, n * 4) ||
                       iris_hip_memcpy_d2h(s, w->rope_sin, n * 4) || fill_ktables(tf, c, s);
        free(c);
        free(s);
        if (rc) return -1;
    }
    /* adapters rebuilt (the graph holds the old GEMM problems), SREF strength
     * changed, or a CSD delta attached / removed. Skipping the CSD delta
     * (csd_skip, flipped before every forward by the style-CFG sampler)
     * uploads zeros instead: acc + 0 is the plain forward bit for bit, and
     * the graph is kept. */
    const int csd_on = tf->csd_delta != NULL;
    if ((w->lora_gen != tf->lora_gen || w->kgamma != tf->sref_strength || w->csd_on != csd_on) && capture(tf))
        return -1;
    if (csd_on) {
        const size_t nb = (size_t)tf->hidden * 4;
        if (tf->csd_skip) {
            if (!tf->csd_zero && !(tf->csd_zero = (float *)calloc(tf->hidden, sizeof(float)))) return -1;
            if (iris_hip_memcpy_h2d(tf->d_csd, tf->csd_zero, nb) || iris_hip_sync()) return -1;
        } else if (iris_hip_memcpy_h2d(tf->d_csd, tf->csd_delta, nb) || iris_hip_sync()) {
            return -1;
        }
    }
    /* get_timestep_embedding(t * 1000), :3967 */
    iris_timestep_sincos(w->tsin_host, t * 1000.0f, 256, 10000.0f);
    if (iris_hip_memcpy_h2d(w->tsin, w->tsin_host, 256 * 4)) return -1;
    /* profiled: the same launches one by one, each timed */
    if (iris_hip_profile_enabled() ? enqueue_forward(tf) : iris_hip_graph_launch(w->graph)) return -1;
    /* per-block progress (iris_transformer_flux.c:4085-4086, :4185-4186,
     * :4315-4316); the blocks run inside one graph, so these fire once the
     * step has been enqueued */
    if (iris_substep_callback) {
        for (int i = 0; i < tf->n_double; i++) iris_substep_callback(IRIS_SUBSTEP_DOUBLE_BLOCK, i, tf->n_double);
        for (int i = 0; i < tf->n_single; i++) iris_substep_callback(IRIS_SUBSTEP_SINGLE_BLOCK, i, tf->n_single);
        iris_substep_callback(IRIS_SUBSTEP_FINAL_LAYER, 0, 1);
    }
    return 0;
}

int iris_flux_step(iris_transformer_t *tf, float t_curr, float t_next, float guidance) {
    work_t *w = &tf->w;
    if (iris_flux_velocity(tf, t_curr)) return -1;
    size_t n = (size_t)tf->latent_ch * w->I0;
    /* Euler (iris_sample.c:359) or CFG combine (:768-771): slot 0 uncond, 1 cond */
    if (w->B == 2) return iris_hip_euler(w->lat, w->vel, w->vel + n, guidance, t_next - t_curr, 1.0f, n);
    return iris_hip_euler(w->lat, w->vel, NULL, 0.0f, t_next - t_curr, 1.0f, n);
}

int iris_flux_download_latent(iris_transformer_t *tf, float *latent) {
    return iris_hip_memcpy_d2h(latent, tf->w.lat, (size_t)tf->latent_ch * tf->w.I0 * 4);
}

int iris_flux_download_velocity(iris_transformer_t *tf, float *v) {
    return iris_hip_memcpy_d2h(v, tf->w.vel, (size_t)tf->w.B * tf->latent_ch * tf->w.I0 * 4);
}

void *iris_flux_device_buffer(iris_transformer_t *tf, const char *name) {
    work_t *w = &tf->w;
    if (!strcmp(name, "x")) return w->x;
    if (!strcmp(name, "latent")) return w->lat;
    if (!strcmp(name, "velocity")) return w->vel;
    if (!strcmp(name, "tokens")) return w->tok;
    if (!strcmp(name, "rope_cos")) return w->rope_cos;
    if (!strcmp(name, "krope_cos")) return w->krope_cos;
    if (!strcmp(name, "krope_sin")) return w->krope_sin;
    if (!strcmp(name, "rope_sin")) return w->rope_sin;
    if (!strcmp(name, "rope_pair_cos")) return w->rp_cos;
    if (!strcmp(name, "rope_pair_sin")) return w->rp_sin;
    if (!strcmp(name, "rope_pos")) return w->rp_pos;
    if (!strcmp(name, "rope_axis")) return w->rp_axis;
    if (!strcmp(name, "t_emb")) return w->temb;
    if (!strcmp(name, "mod")) return w->mod;
    if (!strcmp(name, "a")) return w->a;
    if (!strcmp(name, "cat")) return w->cat;
    if (!strcmp(name, "qkv")) return w->qkv;
    if (!strcmp(name, "q")) return w->q;
    if (!strcmp(name, "k")) return w->k;
    if (!strcmp(name, "vt")) return w->vt;
    if (!strcmp(name, "txt")) return w->txtf;
    return NULL;
}

/* ------------------------------------------------------------- adapters */

/* ------------------------------------------------------------------ LoRA */

/* The reference adds scale * B (A x) in f32 to the output of each adapted
 * linear (lora_apply, iris_lora.c:43-90; call sites iris_transformer_flux.c:
 * 2429-2434, :2482-2487, :2529-2532, :3818-3819, :3909-3910). Here each
 * adapted linear runs as one GEMM over the concatenated K axis,
 *     [x | u] [W | scale B]^T,   u = x A^T (bf16 [rows][rp]),
 * so the low-rank term is accumulated in f32 with the product itself, before
 * the epilogue (bf16 store, SwiGLU, gated residual), and the weights stay
 * untouched. The adapters of one fused linear (Q, K, V of a stream) share u:
 * their A rows are stacked in dn and each B fills its own columns of up.
 * u is formed by a split-K GEMM per adapted linear and call. */
static void lora_dev_free(iris_transformer_t *tf) {
    const int n = 4 * tf->n_double + 2 * tf->n_single;
    if (tf->ldev || tf->lu || tf->lws) tf->lora_gen++;
    for (int i = 0; tf->ldev && i < n; i++) {
        iris_hip_free(tf->ldev[i].dn);
        iris_hip_free(tf->ldev[i].up);
    }
    free(tf->ldev);
    tf->ldev = NULL;
    tf->lrp_max = 0;
    iris_hip_free(tf->lu);
    iris_hip_free(tf->lws);
    tf->lu = NULL;
    tf->lws = NULL;
    tf->lu_rows = tf->lws_floats = 0;
    tf->lora_built = NULL;
}

/* one adapter of a fused linear: rows row0 .. row0 + out of the logical
 * output (before the SwiGLU interleave) */
typedef struct {
    const lora_adapter_t *ad;
    int row0, out;
} lora_part_t;

static int lora_valid(const lora_adapter_t *ad) { return ad && ad->lora_A && ad->lora_B && ad->rank > 0; }

/* Build one adapted linear (in inputs, rows outputs; logical rows >= il_from
 * are the SwiGLU gate / up halves, il_len each, interleaved in groups of
 * SWIGLU_GROUP in the weight). Adapters whose in_dim or out_dim does not match
 * the linear are rejected (-1), as the reference's loader skips them
 * (iris_lora.c:151-164). */
static int lora_build(lora_dev_t *d, const lora_part_t *parts, int n, int in, int rows, int il_from, int il_len,
                      float scale, const char *what, int blk) {
    memset(d, 0, sizeof(*d));
    int rsum = 0;
    for (int j = 0; j < n; j++) {
        const lora_adapter_t *ad = parts[j].ad;
        if (!lora_valid(ad)) continue;
        if (ad->in_dim != in || ad->out_dim != parts[j].out) {
            fprintf(stderr, "iris_hip: LoRA %s of block %d: adapter %d x %d (in x out), the linear takes %d x %d\n",
                    what, blk, ad->in_dim, ad->out_dim, in, parts[j].out);
            return -1;
        }
        rsum += ad->rank;
    }
    if (!rsum) return 0;
    const int rp = (rsum + 63) / 64 * 64;
    uint16_t *hdn = (uint16_t *)calloc((size_t)rp * in, 2), *hup = (uint16_t *)calloc((size_t)rows * rp, 2);
    int rc = -1;
    if (!hdn || !hup) goto out;
    for (int j = 0, c0 = 0; j < n; j++) {
        const lora_adapter_t *ad = parts[j].ad;
        if (!lora_valid(ad)) continue;
        const int r = ad->rank;
        for (size_t e = 0; e < (size_t)r * in; e++) hdn[(size_t)c0 * in + e] = iris_f32_to_bf16(ad->lora_A[e]);
        for (int o = 0; o < ad->out_dim; o++) {
            const int q = parts[j].row0 + o;
            int m = q;
            if (il_len > 0 && q >= il_from) {
                const int g = q - il_from, up = g >= il_len, gi = up ? g - il_len : g;
                m = il_from + (gi / SWIGLU_GROUP) * 2 * SWIGLU_GROUP + up * SWIGLU_GROUP + gi % SWIGLU_GROUP;
            }
            if (m < 0 || m >= rows) {
                fprintf(stderr, "iris_hip: LoRA %s of block %d: output row %d outside 0..%d\n", what, blk, m, rows - 1);
                goto out;
            }
            for (int k = 0; k < r; k++)
                hup[(size_t)m * rp + c0 + k] = iris_f32_to_bf16(scale * ad->lora_B[(size_t)o * r + k]);
        }
        c0 += r;
    }
    d->dn = (uint16_t *)iris_hip_malloc((size_t)rp * in * 2);
    d->up = (uint16_t *)iris_hip_malloc((size_t)rows * rp * 2);
    if (!d->dn || !d->up || iris_hip_memcpy_h2d(d->dn, hdn, (size_t)rp * in * 2) ||
        iris_hip_memcpy_h2d(d->up, hup, (size_t)rows * rp * 2) || iris_hip_sync())
        goto out;
    d->in = in;
    d->rows = rows;
    d->rp = rp;
    rc = 0;
out:
    if (rc) {
        iris_hip_free(d->dn);
        iris_hip_free(d->up);
        memset(d, 0, sizeof(*d));
    }
    free(hdn);
    free(hup);
    return rc;
}

/* split count for u = x dn^T: enough 256-row tiles x K chunks for the chip */
static int lora_splits(int M, int K) {
    const int tm = (M + 255) / 256, nk = K / 64;
    int s = 256 / tm;
    if (s > nk) s = nk;
    return s < 1 ? 1 : s;
}

/* u and split-K buffers for the prepared geometry; 1 if reallocated (a
 * captured graph holds the old addresses: lora_gen moves on), 0 if
 * unchanged, -1 on error */
static int lora_work(iris_transformer_t *tf) {
    if (!tf->ldev || !tf->lrp_max || !tf->w.valid) return 0;
    const size_t rows = (size_t)tf->w.B * tf->w.S;
    /* chunks * M <= 256 x 256 whenever the product is split (lora_splits) */
    const size_t wsf = (size_t)65536 * tf->lrp_max;
    if (rows <= tf->lu_rows && wsf <= tf->lws_floats) return 0;
    tf->lora_gen++;
    iris_hip_free(tf->lu);
    iris_hip_free(tf->lws);
    tf->lu = (uint16_t *)iris_hip_malloc(rows * tf->lrp_max * 2);
    tf->lws = (float *)iris_hip_malloc(wsf * 4);
    if (!tf->lu || !tf->lws) {
        iris_hip_free(tf->lu);
        iris_hip_free(tf->lws);
        tf->lu = NULL;
        tf->lws = NULL;
        tf->lu_rows = tf->lws_floats = 0;
        return -1;
    }
    tf->lu_rows = rows;
    tf->lws_floats = wsf;
    return 1;
}

/* Device adapters for tf->lora; 0 when they match it, -1 on error (none are
 * applied then and the next forward tries again). Any change of the device
 * state moves lora_gen on: a step graph captured before must be captured
 * again before its next launch, also after a failed build freed the
 * previous adapters. */
static int lora_sync(iris_transformer_t *tf) {
    if (!tf->lora_dirty && tf->lora == tf->lora_built) return 0;
    tf->lora_dirty = 0;
    lora_dev_free(tf);
    const lora_state_t *L = (const lora_state_t *)tf->lora;
    if (!L || L->scale == 0.0f) {
        tf->lora_built = tf->lora;
        return 0;
    }
    const int h = tf->hidden, mlp = tf->mlp, nd = tf->n_double, ns = tf->n_single;
    const float sc = L->scale;
    tf->ldev = (lora_dev_t *)calloc((size_t)4 * nd + 2 * ns, sizeof(lora_dev_t));
    if (!tf->ldev) return -1;
#define AD(arr, n, i) ((arr) && (i) < (n) ? &(arr)[i] : NULL)
    for (int i = 0; i < nd; i++) {
        const int n = L->num_double_blocks;
        lora_part_t iq[3] = {{AD(L->double_img_q, n, i), 0, h}, {AD(L->double_img_k, n, i), h, h},
                             {AD(L->double_img_v, n, i), 2 * h, h}};
        lora_part_t tq[3] = {{AD(L->double_txt_q, n, i), 0, h}, {AD(L->double_txt_k, n, i), h, h},
                             {AD(L->double_txt_v, n, i), 2 * h, h}};
        lora_part_t ip = {AD(L->double_img_proj, n, i), 0, h}, tp = {AD(L->double_txt_proj, n, i), 0, h};
        lora_dev_t *d = &tf->ldev[4 * i];
        if (lora_build(d + 0, iq, 3, h, 3 * h, 0, 0, sc, "img qkv", i) ||
            lora_build(d + 1, &ip, 1, h, h, 0, 0, sc, "img proj", i) ||
            lora_build(d + 2, tq, 3, h, 3 * h, 0, 0, sc, "txt qkv", i) ||
            lora_build(d + 3, &tp, 1, h, h, 0, 0, sc, "txt proj", i))
            goto fail;
    }
    for (int i = 0; i < ns; i++) {
        const int n = L->num_single_blocks;
        lora_part_t l1 = {AD(L->single_linear1, n, i), 0, 3 * h + 2 * mlp}, l2 = {AD(L->single_linear2, n, i), 0, h};
        lora_dev_t *d = &tf->ldev[4 * nd + 2 * i];
        if (lora_build(d + 0, &l1, 1, h, 3 * h + 2 * mlp, 3 * h, mlp, sc, "linear1", i) ||
            lora_build(d + 1, &l2, 1, h + mlp, h, 0, 0, sc, "linear2", i))
            goto fail;
    }
#undef AD
    for (int i = 0; i < 4 * nd + 2 * ns; i++)
        if (tf->ldev[i].rp > tf->lrp_max) tf->lrp_max = tf->ldev[i].rp;
    if (!tf->lrp_max) {
        free(tf->ldev);
        tf->ldev = NULL;
    }
    if (lora_work(tf) < 0) goto fail;
    tf->lora_built = tf->lora;
    tf->lora_gen++;
    return 0;
fail:
    lora_dev_free(tf);
    tf->lora_dirty = 1;   /* try again (and fail loudly again) at the next forward */
    return -1;
}

/* u rows [r0, r0 + M) = x dn^T for the adapted linear d (x bf16, row stride
 * ldx); no-op without an adapter */
static int lora_down(iris_transformer_t *tf, const lora_dev_t *d, const uint16_t *x, int ldx, size_t r0, int M) {
    if (!d || !d->rp || M <= 0) return 0;
    iris_gemm_problem_t p;
    memset(&p, 0, sizeof(p));
    p.A = x; p.lda = ldx; p.W = d->dn; p.ldw = d->in;
    p.out = tf->lu + r0 * tf->lrp_max; p.ldo = tf->lrp_max;
    p.M = M; p.N = d->rp; p.K = d->in; p.epi = IRIS_EPI_BF16;
    return iris_hip_gemm_splitk(&p, lora_splits(M, d->in), tf->lws, tf->lws_floats * 4);
}

/* add the adapter's second K segment (u rows from r0, up rows from row0) */
static void lora_seg(const iris_transformer_t *tf, iris_gemm_problem_t *p, const lora_dev_t *d, size_t r0, int row0) {
    if (!d || !d->rp) return;
    p->A2 = tf->lu + r0 * tf->lrp_max; p->lda2 = tf->lrp_max;
    p->W2 = d->up + (size_t)row0 * d->rp; p->ldw2 = d->rp;
    p->K2 = d->rp;
}

static const lora_dev_t *lora_at(const iris_transformer_t *tf, int idx) {
    return tf->ldev && tf->ldev[idx].rp ? &tf->ldev[idx] : NULL;
}

/* The reference's adapter setters (iris_transformer_flux.c:5131-5201), kept
 * so a caller links unchanged. LoRA, the CSD style delta and the SREF
 * controls are applied; while an IP-Adapter is attached every forward fails
 * with a message instead of silently ignoring it. Ownership follows the
 * reference: the transformer takes what it is given and releases it on
 * replacement or free through the reference's own release functions when
 * those are linked in. */
void lora_free(void *lora) __attribute__((weak));
void iris_ip_adapter_free(void *ip) __attribute__((weak));
int iris_ip_adapter_set_schedule(void *ip, const char *spec) __attribute__((weak));
void iris_ip_adapter_set_step(void *ip, int step, int num_steps) __attribute__((weak));

static void release_adapters(iris_transformer_t *tf) {
    if (tf->lora && lora_free) lora_free(tf->lora);
    if (tf->ip && iris_ip_adapter_free) iris_ip_adapter_free(tf->ip);
    free(tf->ip_embeds);
    free(tf->csd_delta);
    tf->lora = tf->ip = tf->ip_embeds = NULL;
    tf->csd_delta = NULL;
}

static int adapter_active(const iris_transformer_t *tf) {
    const char *what = tf->ip ? "IP-Adapter" : NULL;
    if (what) fprintf(stderr, "iris_hip: %s is attached; the HIP denoiser does not apply adapters\n", what);
    return what != NULL;
}

void iris_transformer_set_lora(iris_transformer_t *tf, void *lora) {
    if (!tf) return;
    if (tf->lora && tf->lora != lora && lora_free) lora_free(tf->lora);
    tf->lora = lora;
    tf->lora_dirty = 1;   /* built at the next forward (a freed state's address may come back) */
}

void iris_transformer_set_csd_delta(iris_transformer_t *tf, float *delta) {
    if (!tf) return;
    if (tf->csd_delta != delta) free(tf->csd_delta);
    tf->csd_delta = delta;
}

void iris_transformer_set_csd_skip(iris_transformer_t *tf, int skip) {
    if (tf) tf->csd_skip = skip;
}

int iris_transformer_csd_active(iris_transformer_t *tf) { return tf && tf->csd_delta != NULL; }

void iris_transformer_set_sref_bands(iris_transformer_t *tf, float shf, float slf) {
    if (!tf) return;
    tf->sref_shf = (shf >= 0.0f && shf <= 1.0f) ? shf : 1.0f;
    tf->sref_slf = (slf >= 1.0f) ? slf : 1.0f;
}

void iris_transformer_set_sref_strength(iris_transformer_t *tf, float gamma) {
    if (!tf) return;
    if (!(gamma > 0.0f) || gamma == 1.0f) { tf->sref_strength = 1.0f; return; }
    tf->sref_strength = gamma < 1e-3f ? 1e-3f : gamma > 8.0f ? 8.0f : gamma;
}

int iris_transformer_set_ip_adapter(iris_transformer_t *tf, void *ip, float *ip_embeds) {
    if (!tf) return -1;
    if (tf->ip && iris_ip_adapter_free) iris_ip_adapter_free(tf->ip);
    free(tf->ip_embeds);
    tf->ip = ip;
    tf->ip_embeds = ip ? ip_embeds : NULL;
    if (!ip) free(ip_embeds);
    return 0;
}

int iris_transformer_set_ip_schedule(iris_transformer_t *tf, const char *spec) {
    if (!tf || !tf->ip || !iris_ip_adapter_set_schedule) return -1;
    return iris_ip_adapter_set_schedule(tf->ip, spec);
}

void iris_transformer_set_ip_step(iris_transformer_t *tf, int step, int num_steps) {
    if (tf && tf->ip && iris_ip_adapter_set_step) iris_ip_adapter_set_step(tf->ip, step, num_steps);
}

/* Legacy single-file loader (iris_transformer_flux.c:4845): the HIP build
 * reads safetensors directories only. */
iris_transformer_t *iris_transformer_load(FILE *f) {
    (void)f;
    fprintf(stderr, "iris_transformer_load: the HIP build loads safetensors directories "
                    "(iris_transformer_load_safetensors)\n");
    return NULL;
}

/* The reference's profile counters (:55-80): its cumulative single-block
 * breakdown becomes the per-kernel table of the library's profile (eager
 * steps with an event pair around every launch). reset starts a profile,
 * print writes the table to stderr and leaves the profile running. */
/* The reference zeroes its cumulative counters here
 * (iris_transformer_flux.c:73-77). Here the counters are the per-kernel
 * records of iris_hip_profile_enable, which is also what turns them on (and
 * makes the forward run launch by launch instead of replaying its graph);
 * this call only clears them, and leaves the execution mode as it is. With
 * IRIS_PROFILE=1 in the environment the library starts with the profile on,
 * for callers written against the reference's interface. */
void iris_reset_blas_profile(void) {
    if (iris_hip_profile_enabled()) iris_hip_profile_enable(1);
}

void iris_print_blas_profile(void) {
    if (!iris_hip_profile_enabled()) return;
    iris_kernel_time_t k[128];
    const int n = iris_hip_profile_read(k, 128);
    double total = 0.0;
    for (int i = 0; i < n; i++) total += k[i].total_ms;
    if (n <= 0 || total <= 0.0) return;
    fprintf(stderr, "\nKernel breakdown (cumulative, %d kernel shapes):\n", n);
    for (int i = 0; i < n; i++)
        fprintf(stderr, "  %-44s grid %8lld  %5d x %8.3f ms = %8.1f ms (%4.1f%%)\n", k[i].kernel, k[i].grid, k[i].calls,
                k[i].total_ms / k[i].calls, k[i].total_ms, 100.0 * k[i].total_ms / total);
    fprintf(stderr, "  Total:  %8.1f ms\n", total);
}

/* ------------------------------------------------------ reference entries */

static float *forward_host(iris_transformer_t *tf, const float *latent, int ih, int iw, const iris_ref_t *refs,
                           int n_refs, const float *txt, int T, float t) {
    if (!tf || !latent || !txt) return NULL;
    if (iris_flux_prepare(tf, ih, iw, refs, n_refs, T, 1)) return NULL;
    if (iris_flux_upload(tf, latent, refs, txt)) return NULL;
    if (iris_flux_velocity(tf, t)) return NULL;
    size_t n = (size_t)tf->latent_ch * ih * iw;
    float *out = (float *)malloc(n * sizeof(float));
    if (!out) return NULL;
    if (iris_hip_memcpy_d2h(out, tf->w.vel, n * sizeof(float))) {
        fprintf(stderr, "iris_transformer_forward: %s\n", iris_hip_last_error());
        free(out);
        return NULL;
    }
    return out;
}

float *iris_transformer_forward(iris_transformer_t *tf, const float *img_latent, int img_h, int img_w,
                                const float *txt_emb, int txt_seq, float timestep) {
    return forward_host(tf, img_latent, img_h, img_w, NULL, 0, txt_emb, txt_seq, timestep);
}

float *iris_transformer_forward_with_refs(iris_transformer_t *tf, const float *img_latent, int img_h, int img_w,
                                          const float *ref_latent, int ref_h, int ref_w, int t_offset,
                                          const float *txt_emb, int txt_seq, float timestep) {
    if (!ref_latent) return iris_transformer_forward(tf, img_latent, img_h, img_w, txt_emb, txt_seq, timestep);
    iris_ref_t r = {ref_latent, ref_h, ref_w, t_offset};
    return forward_host(tf, img_latent, img_h, img_w, &r, 1, txt_emb, txt_seq, timestep);
}

float *iris_transformer_forward_with_multi_refs(iris_transformer_t *tf, const float *img_latent, int img_h,
                                                int img_w, const iris_ref_t *refs, int num_refs,
                                                const float *txt_emb, int txt_seq, float timestep) {
    if (!refs || num_refs == 0)
        return iris_transformer_forward(tf, img_latent, img_h, img_w, txt_emb, txt_seq, timestep);
    return forward_host(tf, img_latent, img_h, img_w, refs, num_refs, txt_emb, txt_seq, timestep);
}
