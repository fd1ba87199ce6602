/*
 * orc_qwen3.c - CPU f32 restatement of the reference's Qwen3 text encoder
 * forward (TEST INFRASTRUCTURE ONLY; see iris_oracle.h).
 *
 * Follows iris_qwen3.c: config keys and defaults (:1380-1440, :1442-1449),
 * tensor names (:1254-1300), RoPE tables (:258-270), RMSNorm (:191-210),
 * per-head Q/K RMSNorm (:214-236), split-half rotation (:277-320), attention
 * with causal and padding masks at -1e9 and GQA (:331-467), SwiGLU MLP
 * (:470-488), the layer (:496-538) and the forward with layer extraction
 * (:1072-1200). Weights are widened bf16 -> f32 as the reference's load_tensor
 * does; the softmax and SiLU use fast_expf like the reference.
 */
#include "orc_internal.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define Q_MAX_SEQ 512

typedef struct {
    float *q, *k, *v, *o, *qn, *kn, *gate, *up, *down, *ln1, *ln2;
} orc_qlayer_t;

struct orc_qwen3 {
    int hidden, inter, heads, kv_heads, head_dim, vocab, layers;
    float theta;
    int mode;
    float *embed;
    orc_qlayer_t *L;
};

static void q_defaults(orc_qwen3_t *m) {
    m->hidden = 2560; m->inter = 9728; m->heads = 32; m->kv_heads = 8; m->head_dim = 128;
    m->vocab = 151936; m->layers = 36; m->theta = 1000000.0f;
}

/* parse_qwen3_config, iris_qwen3.c:1380-1440 */
static void q_config(orc_qwen3_t *m, const char *dir) {
    q_defaults(m);
    char path[2048];
    snprintf(path, sizeof(path), "%s/config.json", dir);
    FILE *f = fopen(path, "r");
    if (!f) return;
    char buf[8192];
    size_t n = fread(buf, 1, sizeof(buf) - 1, f);
    fclose(f);
    buf[n] = 0;
    const char *keys[] = {"\"hidden_size\"", "\"intermediate_size\"", "\"num_attention_heads\"",
                          "\"num_key_value_heads\"", "\"head_dim\"", "\"vocab_size\"", "\"num_hidden_layers\""};
    int *dst[] = {&m->hidden, &m->inter, &m->heads, &m->kv_heads, &m->head_dim, &m->vocab, &m->layers};
    for (int i = 0; i < 7; i++) {
        const char *p = strstr(buf, keys[i]);
        if (p && (p = strchr(p, ':')) && atoi(p + 1) > 0) *dst[i] = atoi(p + 1);
    }
    const char *p = strstr(buf, "\"rope_theta\"");
    if (p && (p = strchr(p, ':')) && atof(p + 1) > 0) m->theta = (float)atof(p + 1);
}

void orc_qwen3_free(orc_qwen3_t *m) {
    if (!m) return;
    if (m->L)
        for (int i = 0; i < m->layers; i++) {
            orc_qlayer_t *l = &m->L[i];
            float *all[] = {l->q, l->k, l->v, l->o, l->qn, l->kn, l->gate, l->up, l->down, l->ln1, l->ln2};
            for (int j = 0; j < 11; j++) free(all[j]);
        }
    free(m->L);
    free(m->embed);
    free(m);
}

typedef float *(*q_get_fn)(void *ctx, const char *name, size_t n, int is_norm);

static float *q_get_st(void *ctx, const char *name, size_t n, int is_norm) {
    float *d = orc_load_f32((const iris_st_set_t *)ctx, name);
    (void)n; (void)is_norm;
    return d;
}

static float *q_get_synth(void *ctx, const char *name, size_t n, int is_norm) {
    return orc_synth_f32(*(const uint64_t *)ctx, name, n, is_norm ? 1.0f : 0.0f, 0.02f);
}

static orc_qwen3_t *q_fill(orc_qwen3_t *m, q_get_fn get, void *ctx) {
    const size_t h = m->hidden, I = m->inter, qd = (size_t)m->heads * m->head_dim, kd = (size_t)m->kv_heads * m->head_dim;
    char nm[256];
    m->L = (orc_qlayer_t *)calloc((size_t)m->layers, sizeof(orc_qlayer_t));
    if (!m->L || !(m->embed = get(ctx, "model.embed_tokens.weight", (size_t)m->vocab * h, 0))) goto fail;
    for (int i = 0; i < m->layers; i++) {
        orc_qlayer_t *l = &m->L[i];
#define G(dst, fmt, n, norm) \
        do { snprintf(nm, sizeof(nm), "model.layers.%d." fmt, i); if (!((dst) = get(ctx, nm, (n), (norm)))) goto fail; } while (0)
        G(l->ln1, "input_layernorm.weight", h, 1);
        G(l->ln2, "post_attention_layernorm.weight", h, 1);
        G(l->q, "self_attn.q_proj.weight", qd * h, 0);
        G(l->k, "self_attn.k_proj.weight", kd * h, 0);
        G(l->v, "self_attn.v_proj.weight", kd * h, 0);
        G(l->o, "self_attn.o_proj.weight", h * qd, 0);
        G(l->qn, "self_attn.q_norm.weight", (size_t)m->head_dim, 1);
        G(l->kn, "self_attn.k_norm.weight", (size_t)m->head_dim, 1);
        G(l->gate, "mlp.gate_proj.weight", I * h, 0);
        G(l->up, "mlp.up_proj.weight", I * h, 0);
        G(l->down, "mlp.down_proj.weight", h * I, 0);
#undef G
    }
    return m;
fail:
    orc_qwen3_free(m);
    return NULL;
}

orc_qwen3_t *orc_qwen3_load(const char *dir) {
    orc_qwen3_t *m = (orc_qwen3_t *)calloc(1, sizeof(*m));
    if (!m) return NULL;
    q_config(m, dir);
    iris_st_set_t st;
    static const char *const fb[] = {"model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors", NULL,
                                     "model.safetensors"};
    if (iris_st_set_open_files(&st, dir, "model.safetensors.index.json", fb, 4)) { free(m); return NULL; }
    orc_qwen3_t *r = q_fill(m, q_get_st, &st);
    iris_st_set_close(&st);
    return r;
}

orc_qwen3_t *orc_qwen3_create_synth(int hidden, int inter, int heads, int kv_heads, int layers, int vocab,
                                    uint64_t seed) {
    orc_qwen3_t *m = (orc_qwen3_t *)calloc(1, sizeof(*m));
    if (!m) return NULL;
    q_defaults(m);
    m->hidden = hidden; m->inter = inter; m->heads = heads; m->kv_heads = kv_heads; m->layers = layers;
    m->vocab = vocab;
    return q_fill(m, q_get_synth, &seed);
}

void orc_qwen3_set_mode(orc_qwen3_t *m, int mode) { m->mode = mode ? 1 : 0; }

int orc_qwen3_dims(const orc_qwen3_t *m, int *out4) {
    out4[0] = m->hidden; out4[1] = m->layers; out4[2] = (m->mode ? 1 : 3) * m->hidden; out4[3] = m->head_dim;
    return 0;
}

/* per-head RMSNorm, iris_qwen3.c:214-236 */
static void q_head_rms(float *x, const float *w, int seq, int nh, int hd) {
    for (int s = 0; s < seq; s++)
        for (int h = 0; h < nh; h++) {
            float *v = x + ((size_t)s * nh + h) * hd;
            float ss = 0.0f;
            for (int i = 0; i < hd; i++) ss += v[i] * v[i];
            const float inv = 1.0f / sqrtf(ss / hd + 1e-6f);
            for (int i = 0; i < hd; i++) v[i] = v[i] * inv * w[i];
        }
}

/* apply_rope on one [seq][nh][hd] tensor, iris_qwen3.c:277-320 */
static void q_rope(float *x, const float *c, const float *sn, int seq, int nh, int hd) {
    const int half = hd / 2;
    for (int s = 0; s < seq; s++)
        for (int h = 0; h < nh; h++) {
            float *v = x + ((size_t)s * nh + h) * hd;
            for (int i = 0; i < half; i++) {
                const float x0 = v[i], x1 = v[i + half], cc = c[s * half + i], ss = sn[s * half + i];
                v[i] = x0 * cc - x1 * ss;
                v[i + half] = x0 * ss + x1 * cc;
            }
        }
}

/* layers up to last_limit (or the mode's last extraction layer if < 0) */
float *orc_qwen3_forward(orc_qwen3_t *m, const int *ids, const int *mask, int seq, int last_limit) {
    if (seq < 1 || seq > Q_MAX_SEQ) return NULL;
    const int h = m->hidden, hd = m->head_dim, nh = m->heads, nkv = m->kv_heads, I = m->inter;
    const int qd = nh * hd, kd = nkv * hd, half = hd / 2, group = nh / nkv;
    const int last = m->mode ? m->layers - 2 : 26;
    const int stop = last_limit >= 0 && last_limit < last ? last_limit : last;
    if (stop < 0 || stop >= m->layers) return NULL;
    const int text_dim = (m->mode ? 1 : 3) * h;
    float *x = calloc((size_t)seq * h, 4), *res = malloc((size_t)seq * h * 4), *nrm = malloc((size_t)seq * h * 4);
    float *q = malloc((size_t)seq * qd * 4), *k = malloc((size_t)seq * kd * 4), *v = malloc((size_t)seq * kd * 4);
    float *ao = malloc((size_t)seq * qd * 4), *g = malloc((size_t)seq * I * 4), *u = malloc((size_t)seq * I * 4);
    float *mo = malloc((size_t)seq * h * 4), *out = calloc((size_t)seq * text_dim, 4);
    float *rc = malloc((size_t)seq * half * 4), *rs = malloc((size_t)seq * half * 4);
    float *sc = malloc((size_t)nh * seq * seq * 4);
    if (!x || !res || !nrm || !q || !k || !v || !ao || !g || !u || !mo || !out || !rc || !rs || !sc) goto fail;
    /* compute_rope_freqs: 1 / powf(theta, 2i / hd) in the reference's
     * -ffast-math build is libmvec powf(theta, -2i / hd) (as for the Flux tables) */
    {
        float base[64];
        orc_rope_bases(base, half, hd, m->theta);
        for (int pos = 0; pos < seq; pos++)
            for (int i = 0; i < half; i++) {
                const float angle = pos * base[i];
                rc[pos * half + i] = cosf(angle);
                rs[pos * half + i] = sinf(angle);
            }
    }
    for (int s = 0; s < seq; s++)
        if (ids[s] >= 0 && ids[s] < m->vocab) memcpy(x + (size_t)s * h, m->embed + (size_t)ids[s] * h, h * 4);
    const float scale = 1.0f / sqrtf((float)hd);
    for (int li = 0; li <= stop; li++) {
        const orc_qlayer_t *l = &m->L[li];
        memcpy(res, x, (size_t)seq * h * 4);
        orc_rms_norm(nrm, x, l->ln1, seq, h, 1e-6f);
        orc_linear(q, nrm, l->q, NULL, seq, h, qd);
        orc_linear(k, nrm, l->k, NULL, seq, h, kd);
        orc_linear(v, nrm, l->v, NULL, seq, h, kd);
        q_head_rms(q, l->qn, seq, nh, hd);
        q_head_rms(k, l->kn, seq, nkv, hd);
        q_rope(q, rc, rs, seq, nh, hd);
        q_rope(k, rc, rs, seq, nkv, hd);
#pragma omp parallel for schedule(dynamic)
        for (int hh = 0; hh < nh; hh++) {
            const int kvh = hh / group;
            float *S = sc + (size_t)hh * seq * seq;
            orc_sgemm_nt(seq, seq, hd, scale, q + hh * hd, qd, k + kvh * hd, kd, 0.0f, S, seq);
            for (int i = 0; i < seq; i++) {
                for (int j = 0; j < seq; j++) {
                    if (j > i) S[(size_t)i * seq + j] = -1e9f;
                    if (mask && mask[j] == 0) S[(size_t)i * seq + j] = -1e9f;
                }
                orc_softmax(S + (size_t)i * seq, 1, seq);
            }
            orc_sgemm_nn(seq, hd, seq, 1.0f, S, seq, v + kvh * hd, kd, 0.0f, ao + hh * hd, qd);
        }
        orc_linear(x, ao, l->o, NULL, seq, qd, h);
        for (size_t i = 0; i < (size_t)seq * h; i++) x[i] += res[i];
        memcpy(res, x, (size_t)seq * h * 4);
        orc_rms_norm(nrm, x, l->ln2, seq, h, 1e-6f);
        orc_linear(g, nrm, l->gate, NULL, seq, h, I);
        orc_linear(u, nrm, l->up, NULL, seq, h, I);
        orc_silu_mul(g, u, (size_t)seq * I);
        orc_linear(mo, g, l->down, NULL, seq, I, h);
        for (size_t i = 0; i < (size_t)seq * h; i++) x[i] = res[i] + mo[i];
        int slot = -1;
        if (m->mode) slot = li == last ? 0 : -1;
        else slot = li == 8 ? 0 : li == 17 ? 1 : li == 26 ? 2 : -1;
        if (slot >= 0)
            for (int s = 0; s < seq; s++) memcpy(out + (size_t)s * text_dim + slot * h, x + (size_t)s * h, h * 4);
    }
    /* a truncated run (last_limit) returns the hidden state it stopped at */
    if (stop < last) {
        free(out);
        out = x;
        x = NULL;
    }
    free(x); free(res); free(nrm); free(q); free(k); free(v); free(ao); free(g); free(u); free(mo);
    free(rc); free(rs); free(sc);
    return out;
fail:
    free(x); free(res); free(nrm); free(q); free(k); free(v); free(ao); free(g); free(u); free(mo);
    free(out); free(rc); free(rs); free(sc);
    return NULL;
}
