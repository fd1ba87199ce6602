/*
 * iris_qwen3.c - Qwen3 text encoder forward on the HIP layer.
 *
 * The reference's f32 CPU forward (iris_qwen3.c): embedding lookup
 * (:1080-1091); per layer (:496-538) RMSNorm (:191-210) -> Q, K, V
 * projections -> per-head RMSNorm of Q and K (:214-236) -> split-half rotary
 * embedding (:258-320) -> attention with causal and padding masks, GQA
 * (:331-467) -> output projection + residual -> RMSNorm -> SwiGLU MLP
 * (:470-488) + residual; hidden states captured after layers 8, 17, 26
 * (Flux) or num_layers-2 (Z-Image) (:1159-1200).
 *
 * Here every linear is the bf16 MFMA GEMM (fused epilogues: the residual adds
 * are IRIS_EPI_GATED_ADD without a gate, silu(gate)*up is IRIS_EPI_SWIGLU
 * over gate/up rows interleaved in 32-row groups), Q/K norm + rotary
 * embedding is iris_hip_kv_prepare for K and the attention kernel's prologue
 * for Q, and attention is the flash kernel with
 * its causal and grouped-query modes. The split-half rotation pairs dims d
 * and d+64 of a head; the upload permutes each head's Q and K rows (and the
 * Q/K norm weights) to the order 0, 64, 1, 65, ... so those pairs are
 * adjacent, which is the kernel's pairing. Q.K is unchanged by a common
 * permutation of the dims and V is not permuted, so the attention output is
 * the reference's.
 */
#include "../../include/iris_qwen3.h"
#include "../../include/iris_hip.h"
#include "../../include/iris_synth.h"
#include "iris_st.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define SWIGLU_GROUP 32
#define HD 128

typedef struct {
    uint16_t *qkv;       /* [(Hq + 2 Hkv) * 128][h]: Q rows, K rows (head dims permuted), V rows */
    uint16_t *o;         /* [h][Hq * 128] */
    uint16_t *gate_up;   /* [2 I][h], gate and up rows interleaved in 32-row groups */
    uint16_t *down;      /* [h][I] */
    float *ln1, *ln2;    /* [h] */
    float *q_norm, *k_norm;   /* [128], permuted like the Q / K rows */
} qlayer_t;

struct qwen3_model {
    int hidden, inter, heads, kv_heads, vocab, layers;
    float rope_theta;
    int mode;                 /* 0 Flux, 1 Z-Image */
    uint16_t *embed;          /* [vocab][h] */
    qlayer_t *L;
    /* work buffers for QWEN3_MAX_SEQ_LEN tokens */
    int *ids;
    float *x, *out;           /* x [S][h] residual stream; out [S][3h] */
    uint16_t *a, *qkv, *q, *k, *vt, *attn, *mlp;
    float *rope_cos, *rope_sin;   /* [S][128], value of pair p at 2p and 2p+1 */
    float *rp_cos, *rp_sin;       /* [S][64], value of pair p at p (the attention's Q prologue) */
    float *ws;                    /* split-K partial products */
    size_t ws_bytes;
};

/* position of permuted dim j in the reference's head layout */
static int head_perm(int j) { return (j & 1) ? (j >> 1) + HD / 2 : (j >> 1); }

static int fail(const char *what) {
    fprintf(stderr, "qwen3: %s: %s\n", what, iris_hip_last_error());
    return -1;
}

/* ------------------------------------------------------------ weight upload */

typedef struct {
    iris_st_set_t st;
    int have_st;
    uint64_t seed;
    uint16_t *stage;
    size_t stage_n;
} qsrc_t;

static const uint16_t *qsrc_get(qsrc_t *s, const char *name, size_t n, int is_norm) {
    if (s->stage_n < n) {
        free(s->stage);
        s->stage = (uint16_t *)malloc(n * sizeof(uint16_t));
        s->stage_n = s->stage ? n : 0;
        if (!s->stage) return NULL;
    }
    if (s->have_st) {
        const iris_st_file_t *f;
        const iris_st_tensor_t *t = iris_st_set_find(&s->st, name, &f);
        if (!t) { fprintf(stderr, "qwen3: tensor %s not found\n", name); return NULL; }
        if ((size_t)iris_st_numel(t) != n) {
            fprintf(stderr, "qwen3: tensor %s has %lld elements, expected %zu\n", name, (long long)iris_st_numel(t), n);
            return NULL;
        }
        if (t->dtype == IRIS_ST_BF16) return (const uint16_t *)iris_st_ptr(f, t);
        if (iris_st_read_bf16(f, t, s->stage)) return NULL;
        return s->stage;
    }
    iris_synth_fill_bf16(s->stage, n, iris_synth_seed(s->seed, name), 0, is_norm ? 1.0f : 0.0f, 0.02f);
    return s->stage;
}

/* f32 copy of a 1-D tensor (norm weights), optionally permuted per head */
static float *upload_vec(qsrc_t *s, const char *name, size_t n, int permute) {
    float *h = (float *)malloc(n * sizeof(float));
    float *d = NULL;
    if (!h) return NULL;
    const iris_st_file_t *f = NULL;
    const iris_st_tensor_t *t = s->have_st ? iris_st_set_find(&s->st, name, &f) : NULL;
    if (t && (size_t)iris_st_numel(t) == n && t->dtype != IRIS_ST_BF16) {
        if (iris_st_read_f32(f, t, h)) goto out;
    } else {
        const uint16_t *b = qsrc_get(s, name, n, 1);
        if (!b) goto out;
        for (size_t i = 0; i < n; i++) h[i] = iris_bf16_to_f32(b[i]);
    }
    if (permute) {
        float tmp[HD];
        for (size_t base = 0; base + HD <= n; base += HD) {
            for (int j = 0; j < HD; j++) tmp[j] = h[base + head_perm(j)];
            memcpy(h + base, tmp, sizeof(tmp));
        }
    }
    d = (float *)iris_hip_malloc(n * sizeof(float));
    if (!d || iris_hip_memcpy_h2d(d, h, n * sizeof(float)) || iris_hip_sync()) { iris_hip_free(d); d = NULL; }
out:
    free(h);
    return d;
}

/* rows [rows][cols] of a named tensor into dst (device), head rows permuted if asked */
static int upload_rows(qsrc_t *s, const char *name, uint16_t *dst, size_t rows, size_t cols, int permute) {
    const uint16_t *h = qsrc_get(s, name, rows * cols, 0);
    if (!h) return -1;
    if (!permute) {
        if (iris_hip_memcpy_h2d(dst, h, rows * cols * 2)) return -1;
        return iris_hip_sync();
    }
    uint16_t *t = (uint16_t *)malloc(rows * cols * 2);
    if (!t) return -1;
    for (size_t r = 0; r < rows; r++)
        memcpy(t + r * cols, h + ((r / HD) * HD + head_perm((int)(r % HD))) * cols, cols * 2);
    int rc = iris_hip_memcpy_h2d(dst, t, rows * cols * 2) || iris_hip_sync();
    free(t);
    return rc;
}

/* gate rows g*32.. and up rows g*32.. -> interleaved groups of 32 */
static int upload_gate_up(qsrc_t *s, const char *gate, const char *up, uint16_t *dst, size_t inter, size_t cols) {
    const size_t G = SWIGLU_GROUP;
    uint16_t *t = (uint16_t *)malloc(2 * inter * cols * 2);
    if (!t) return -1;
    int rc = -1;
    for (int which = 0; which < 2; which++) {
        const uint16_t *h = qsrc_get(s, which ? up : gate, inter * cols, 0);
        if (!h) goto out;
        for (size_t g = 0; g < inter / G; g++)
            memcpy(t + (2 * g + which) * G * cols, h + g * G * cols, G * cols * 2);
    }
    rc = iris_hip_memcpy_h2d(dst, t, 2 * inter * cols * 2) || iris_hip_sync();
out:
    free(t);
    return rc;
}

static void free_model(qwen3_model_t *m) {
    if (!m) return;
    if (m->L) {
        for (int i = 0; i < m->layers; i++) {
            qlayer_t *l = &m->L[i];
            iris_hip_free(l->qkv); iris_hip_free(l->o); iris_hip_free(l->gate_up); iris_hip_free(l->down);
            iris_hip_free(l->ln1); iris_hip_free(l->ln2); iris_hip_free(l->q_norm); iris_hip_free(l->k_norm);
        }
        free(m->L);
    }
    iris_hip_free(m->embed);
    iris_hip_free(m->ids); iris_hip_free(m->x); iris_hip_free(m->out);
    iris_hip_free(m->a); iris_hip_free(m->qkv); iris_hip_free(m->q); iris_hip_free(m->k); iris_hip_free(m->vt);
    iris_hip_free(m->attn); iris_hip_free(m->mlp);
    iris_hip_free(m->rope_cos); iris_hip_free(m->rope_sin); iris_hip_free(m->rp_cos); iris_hip_free(m->rp_sin); iris_hip_free(m->ws);
    free(m);
}

void qwen3_model_free(qwen3_model_t *m) { free_model(m); }

static int check_arch(const qwen3_model_t *m) {
    if (m->hidden <= 0 || m->hidden % 64 || m->inter <= 0 || m->inter % 64 || m->heads <= 0 || m->kv_heads <= 0 ||
        m->heads % m->kv_heads || m->vocab <= 0 || m->layers < 1) {
        fprintf(stderr, "qwen3: unsupported architecture (hidden %d, intermediate %d, heads %d/%d, vocab %d, layers %d)"
                        "; hidden and intermediate must be multiples of 64, heads a multiple of kv_heads\n",
                m->hidden, m->inter, m->heads, m->kv_heads, m->vocab, m->layers);
        return -1;
    }
    return 0;
}

/* compute_rope_freqs (iris_qwen3.c:258-270) in the adjacent-pair layout */
static int build_rope(qwen3_model_t *m) {
    const int S = QWEN3_MAX_SEQ_LEN;
    float *c = (float *)malloc((size_t)S * HD * sizeof(float)), *sn = (float *)malloc((size_t)S * HD * sizeof(float));
    int rc = -1;
    if (!c || !sn) goto out;
    for (int pos = 0; pos < S; pos++)
        for (int i = 0; i < HD / 2; i++) {
            const float freq = 1.0f / powf(m->rope_theta, (float)(2 * i) / HD);
            const float angle = pos * freq;
            c[(size_t)pos * HD + 2 * i] = c[(size_t)pos * HD + 2 * i + 1] = cosf(angle);
            sn[(size_t)pos * HD + 2 * i] = sn[(size_t)pos * HD + 2 * i + 1] = sinf(angle);
        }
    m->rope_cos = (float *)iris_hip_malloc((size_t)S * HD * sizeof(float));
    m->rope_sin = (float *)iris_hip_malloc((size_t)S * HD * sizeof(float));
    m->rp_cos = (float *)iris_hip_malloc((size_t)S * (HD / 2) * sizeof(float));
    m->rp_sin = (float *)iris_hip_malloc((size_t)S * (HD / 2) * sizeof(float));
    if (!m->rope_cos || !m->rope_sin || !m->rp_cos || !m->rp_sin) goto out;
    if (iris_hip_memcpy_h2d(m->rope_cos, c, (size_t)S * HD * 4) || iris_hip_memcpy_h2d(m->rope_sin, sn, (size_t)S * HD * 4))
        goto out;
    /* the pair tables: entry i = column 2i */
    for (int pos = 0; pos < S; pos++)
        for (int i = 0; i < HD / 2; i++) {
            c[(size_t)pos * (HD / 2) + i] = c[(size_t)pos * HD + 2 * i];
            sn[(size_t)pos * (HD / 2) + i] = sn[(size_t)pos * HD + 2 * i];
        }
    if (iris_hip_memcpy_h2d(m->rp_cos, c, (size_t)S * (HD / 2) * 4) ||
        iris_hip_memcpy_h2d(m->rp_sin, sn, (size_t)S * (HD / 2) * 4) || iris_hip_sync())
        goto out;
    rc = 0;
out:
    free(c); free(sn);
    return rc;
}

static int alloc_work(qwen3_model_t *m) {
    const size_t S = QWEN3_MAX_SEQ_LEN, h = m->hidden, qd = (size_t)m->heads * HD, kd = (size_t)m->kv_heads * HD;
#define QA(dst, bytes) do { if (!((dst) = iris_hip_malloc(bytes))) return -1; } while (0)
    QA(m->ids, S * sizeof(int));
    QA(m->x, S * h * 4);
    QA(m->out, S * 3 * h * 4);
    QA(m->a, S * h * 2);
    QA(m->qkv, S * (qd + 2 * kd) * 2);
    QA(m->q, S * qd * 2);
    QA(m->k, S * kd * 2);
    QA(m->vt, kd * S * 2);
    QA(m->attn, S * qd * 2);
    QA(m->mlp, S * (size_t)m->inter * 2);
    m->ws_bytes = (size_t)64 << 20;
    QA(m->ws, m->ws_bytes);
#undef QA
    return 0;
}

static int load_weights(qwen3_model_t *m, qsrc_t *s) {
    const size_t h = m->hidden, I = m->inter, qd = (size_t)m->heads * HD, kd = (size_t)m->kv_heads * HD;
    char nm[256];
    m->embed = (uint16_t *)iris_hip_malloc((size_t)m->vocab * h * 2);
    if (!m->embed || upload_rows(s, "model.embed_tokens.weight", m->embed, m->vocab, h, 0)) return -1;
    m->L = (qlayer_t *)calloc((size_t)m->layers, sizeof(qlayer_t));
    if (!m->L) return -1;
    /* tensor names: iris_qwen3.c:1254-1300 */
    for (int i = 0; i < m->layers; i++) {
        qlayer_t *l = &m->L[i];
        l->qkv = (uint16_t *)iris_hip_malloc((qd + 2 * kd) * h * 2);
        l->o = (uint16_t *)iris_hip_malloc(h * qd * 2);
        l->gate_up = (uint16_t *)iris_hip_malloc(2 * I * h * 2);
        l->down = (uint16_t *)iris_hip_malloc(h * I * 2);
        if (!l->qkv || !l->o || !l->gate_up || !l->down) return -1;
#define NM(fmt) (snprintf(nm, sizeof(nm), "model.layers.%d." fmt, i), nm)
        if (upload_rows(s, NM("self_attn.q_proj.weight"), l->qkv, qd, h, 1)) return -1;
        if (upload_rows(s, NM("self_attn.k_proj.weight"), l->qkv + qd * h, kd, h, 1)) return -1;
        if (upload_rows(s, NM("self_attn.v_proj.weight"), l->qkv + (qd + kd) * h, kd, h, 0)) return -1;
        if (upload_rows(s, NM("self_attn.o_proj.weight"), l->o, h, qd, 0)) return -1;
        char up[256];
        snprintf(up, sizeof(up), "model.layers.%d.mlp.up_proj.weight", i);
        if (upload_gate_up(s, NM("mlp.gate_proj.weight"), up, l->gate_up, I, h)) return -1;
        if (upload_rows(s, NM("mlp.down_proj.weight"), l->down, h, I, 0)) return -1;
        if (!(l->ln1 = upload_vec(s, NM("input_layernorm.weight"), h, 0))) return -1;
        if (!(l->ln2 = upload_vec(s, NM("post_attention_layernorm.weight"), h, 0))) return -1;
        if (!(l->q_norm = upload_vec(s, NM("self_attn.q_norm.weight"), HD, 1))) return -1;
        if (!(l->k_norm = upload_vec(s, NM("self_attn.k_norm.weight"), HD, 1))) return -1;
#undef NM
    }
    return 0;
}

static qwen3_model_t *finish(qwen3_model_t *m, qsrc_t *s) {
    int rc = check_arch(m) || load_weights(m, s) || build_rope(m) || alloc_work(m);
    free(s->stage);
    if (s->have_st) iris_st_set_close(&s->st);
    if (rc) {
        fail("model setup");
        free_model(m);
        return NULL;
    }
    return m;
}

/* config.json keys as parse_qwen3_config reads them (iris_qwen3.c:1380-1440),
 * with its defaults (qwen3_set_defaults) for missing keys */
static void parse_config(const char *dir, qwen3_model_t *m) {
    m->hidden = 2560; m->inter = 9728; m->heads = 32; m->kv_heads = 8;
    m->vocab = QWEN3_VOCAB_SIZE; m->layers = 36; m->rope_theta = QWEN3_ROPE_THETA;
    char path[2048];
    snprintf(path, sizeof(path), "%s/config.json", dir);
    FILE *f = fopen(path, "r");
    if (!f) return;
    char buf[16384];
    size_t n = fread(buf, 1, sizeof(buf) - 1, f);
    fclose(f);
    buf[n] = 0;
    struct { const char *key; int *dst; } ik[] = {
        {"\"hidden_size\"", &m->hidden}, {"\"intermediate_size\"", &m->inter},
        {"\"num_attention_heads\"", &m->heads}, {"\"num_key_value_heads\"", &m->kv_heads},
        {"\"vocab_size\"", &m->vocab}, {"\"num_hidden_layers\"", &m->layers}};
    for (size_t i = 0; i < sizeof(ik) / sizeof(ik[0]); i++) {
        const char *p = strstr(buf, ik[i].key);
        if (p && (p = strchr(p, ':'))) {
            const int v = atoi(p + 1);
            if (v > 0) *ik[i].dst = v;
        }
    }
    const char *p = strstr(buf, "\"rope_theta\"");
    if (p && (p = strchr(p, ':'))) {
        const float v = (float)atof(p + 1);
        if (v > 0) m->rope_theta = v;
    }
    p = strstr(buf, "\"head_dim\"");
    if (p && (p = strchr(p, ':')) && atoi(p + 1) != HD) {
        fprintf(stderr, "qwen3: head_dim %d unsupported (128)\n", atoi(p + 1));
        m->layers = 0;   /* rejected by check_arch */
    }
}

qwen3_model_t *qwen3_model_load(const char *model_dir) {
    if (!model_dir || iris_hip_init(0)) return NULL;
    qwen3_model_t *m = (qwen3_model_t *)calloc(1, sizeof(*m));
    if (!m) return NULL;
    parse_config(model_dir, m);
    qsrc_t s;
    memset(&s, 0, sizeof(s));
    /* shard discovery as open_safetensors_shards (iris_qwen3.c:1450-1527),
     * plus a single model.safetensors */
    static const char *const fb[] = {"model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors", NULL,
                                     "model.safetensors"};
    if (iris_st_set_open_files(&s.st, model_dir, "model.safetensors.index.json", fb, 4)) {
        fprintf(stderr, "qwen3_model_load: no safetensors shards in %s\n", model_dir);
        free(m);
        return NULL;
    }
    s.have_st = 1;
    return finish(m, &s);
}

qwen3_model_t *qwen3_model_create_synthetic(int hidden, int intermediate, int heads, int kv_heads, int layers,
                                            int vocab, uint64_t seed) {
    if (iris_hip_init(0)) return NULL;
    qwen3_model_t *m = (qwen3_model_t *)calloc(1, sizeof(*m));
    if (!m) return NULL;
    m->hidden = hidden; m->inter = intermediate; m->heads = heads; m->kv_heads = kv_heads;
    m->layers = layers; m->vocab = vocab; m->rope_theta = QWEN3_ROPE_THETA;
    qsrc_t s;
    memset(&s, 0, sizeof(s));
    s.seed = seed;
    return finish(m, &s);
}

void qwen3_model_set_extraction_mode(qwen3_model_t *m, int mode) {
    if (m) m->mode = mode ? 1 : 0;
}

int qwen3_model_text_dim(const qwen3_model_t *m) { return m ? (m->mode ? 1 : 3) * m->hidden : 0; }

/* ------------------------------------------------------------------ forward */

#define CK(x) do { if (x) return fail(#x); } while (0)

static iris_gemm_problem_t prob(const uint16_t *A, int lda, const uint16_t *W, int ldw, void *out, int ldo, int M,
                                int N, int K, int epi) {
    iris_gemm_problem_t p;
    memset(&p, 0, sizeof(p));
    p.A = A; p.lda = lda; p.W = W; p.ldw = ldw; p.out = out; p.ldo = ldo;
    p.M = M; p.N = N; p.K = K; p.epi = epi;
    return p;
}

/* At 512 tokens the N 2560 products are 20 tiles of 256x256 and the QKV
 * product 48: iris_hip_gemm_fill splits K (on 128-row tiles where that is
 * faster) up to what the workspace holds; the gate/up product (152 tiles)
 * runs as one launch. */
static int gemm(qwen3_model_t *m, const iris_gemm_problem_t *p) {
    return iris_hip_gemm_fill(p, m->ws, m->ws_bytes);
}

static int rms(const qwen3_model_t *m, const float *w, int S) {
    iris_norm_args_t a;
    memset(&a, 0, sizeof(a));
    a.x = m->x; a.ldx = m->hidden; a.out = m->a; a.ldo = m->hidden; a.out_bf16 = 1;
    a.rows = S; a.cols = m->hidden; a.mode = IRIS_NORM_RMS; a.eps = QWEN3_RMS_NORM_EPS;
    a.split = S; a.wA = w; a.wB = w;
    return iris_hip_rownorm(&a);
}

/* qwen3_layer_forward (iris_qwen3.c:496-538) */
static int layer_forward(qwen3_model_t *m, const qlayer_t *l, int S, int n_real) {
    const int h = m->hidden, qd = m->heads * HD, kd = m->kv_heads * HD, I = m->inter;
    const int S_pad = (S + 63) / 64 * 64;
    iris_gemm_problem_t p;
    CK(rms(m, l->ln1, S));
    p = prob(m->a, h, l->qkv, h, m->qkv, qd + 2 * kd, S, qd + 2 * kd, h, IRIS_EPI_BF16);
    CK(gemm(m, &p));
    iris_qkprep_args_t q;
    memset(&q, 0, sizeof(q));
    q.qkv = m->qkv; q.ld_qkv = qd + 2 * kd; q.col_k = qd; q.col_v = qd + kd;
    q.k_out = m->k; q.vt_out = m->vt; q.ld_vt = S_pad;
    q.rows = S; q.heads = m->heads; q.kv_heads = m->kv_heads;
    q.wkA = q.wkB = l->k_norm; q.split = S;
    q.cos_t = m->rope_cos; q.sin_t = m->rope_sin; q.eps = QWEN3_RMS_NORM_EPS;
    CK(iris_hip_kv_prepare(&q));
    /* Q: RMSNorm + rotary in the attention kernel's prologue */
    iris_attn_args_t at;
    memset(&at, 0, sizeof(at));
    at.q = m->qkv; at.k = m->k; at.vt = m->vt; at.o = m->attn;
    at.ld_q = qd + 2 * kd; at.ld_k = kd; at.ld_vt = S_pad; at.ld_o = qd;
    at.qn_wA = at.qn_wB = l->q_norm; at.qn_split = S; at.qn_eps = QWEN3_RMS_NORM_EPS;
    at.rope_cos = m->rp_cos; at.rope_sin = m->rp_sin;
    at.sq = S; at.sk = S; at.heads = m->heads; at.batch = 1;
    at.scale = 1.0f / sqrtf((float)HD);
    at.kv_lo0 = 0; at.kv_hi0 = n_real;          /* padding keys (:408-414) */
    at.causal = 1; at.kv_group = m->heads / m->kv_heads;
    CK(iris_hip_attention(&at));
    /* o_proj + residual (:461-466, :514-517) */
    p = prob(m->attn, qd, l->o, qd, m->x, h, S, h, qd, IRIS_EPI_GATED_ADD);
    CK(gemm(m, &p));
    CK(rms(m, l->ln2, S));
    p = prob(m->a, h, l->gate_up, h, m->mlp, I, S, 2 * I, h, IRIS_EPI_SWIGLU);
    CK(gemm(m, &p));
    p = prob(m->mlp, I, l->down, I, m->x, h, S, h, I, IRIS_EPI_GATED_ADD);
    CK(gemm(m, &p));
    return 0;
}

float *qwen3_forward(qwen3_model_t *m, const int *input_ids, const int *attention_mask, int seq_len) {
    if (!m || !input_ids || seq_len < 1 || seq_len > QWEN3_MAX_SEQ_LEN) {
        fprintf(stderr, "qwen3_forward: seq_len %d outside [1, %d]\n", seq_len, QWEN3_MAX_SEQ_LEN);
        return NULL;
    }
    const int S = seq_len, h = m->hidden;
    int n_real = S;
    if (attention_mask) {
        n_real = 0;
        while (n_real < S && attention_mask[n_real]) n_real++;
        for (int i = n_real; i < S; i++)
            if (attention_mask[i]) {
                fprintf(stderr, "qwen3_forward: attention_mask must be ones followed by zeros\n");
                return NULL;
            }
        if (n_real == 0) {
            fprintf(stderr, "qwen3_forward: attention_mask has no real token\n");
            return NULL;
        }
    }
    const int last = m->mode ? m->layers - 2 : QWEN3_OUTPUT_LAYER_3;
    if (last < 0 || last >= m->layers) {
        fprintf(stderr, "qwen3_forward: %d layers, extraction needs layer %d\n", m->layers, last);
        return NULL;
    }
    const int text_dim = qwen3_model_text_dim(m);
    if (iris_hip_memcpy_h2d(m->ids, input_ids, (size_t)S * sizeof(int)) ||
        iris_hip_embed_rows(m->x, m->embed, m->ids, S, h, m->vocab)) {
        fail("embedding");
        return NULL;
    }
    for (int i = 0; i <= last; i++) {
        if (layer_forward(m, &m->L[i], S, n_real)) return NULL;
        int slot = -1;
        if (m->mode) slot = i == last ? 0 : -1;
        else slot = i == QWEN3_OUTPUT_LAYER_1 ? 0 : i == QWEN3_OUTPUT_LAYER_2 ? 1 : i == QWEN3_OUTPUT_LAYER_3 ? 2 : -1;
        if (slot >= 0 && iris_hip_copy_rows(m->out + (size_t)slot * h, text_dim, m->x, h, S, h)) {
            fail("layer output");
            return NULL;
        }
    }
    float *out = (float *)malloc((size_t)S * text_dim * sizeof(float));
    if (!out) return NULL;
    if (iris_hip_memcpy_d2h(out, m->out, (size_t)S * text_dim * sizeof(float))) {
        fail("download");
        free(out);
        return NULL;
    }
    return out;
}
