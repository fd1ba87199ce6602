/*
 * iris_st.c - memory-mapped safetensors reader (see iris_st.h).
 *
 * Reads the same files the reference loader reads (iris_safetensors.c:233-456,
 * shard discovery iris_transformer_flux.c:470-570); written for the HIP build:
 * the map is kept read-only and tensors are widened/narrowed only on request.
 */
#include "iris_st.h"

#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* ---- minimal JSON walker for the safetensors header ---- */

typedef struct { const char *p, *end; } jcur_t;

static void jws(jcur_t *c) {
    while (c->p < c->end && (*c->p == ' ' || *c->p == '\n' || *c->p == '\r' || *c->p == '\t')) c->p++;
}

static int jstr(jcur_t *c, char *out, size_t cap) {
    jws(c);
    if (c->p >= c->end || *c->p != '"') return -1;
    c->p++;
    size_t n = 0;
    while (c->p < c->end && *c->p != '"') {
        char ch = *c->p++;
        if (ch == '\\' && c->p < c->end) ch = *c->p++;
        if (out && n + 1 < cap) out[n] = ch;
        n++;
    }
    if (c->p >= c->end) return -1;
    c->p++;
    if (out) out[n < cap ? n : cap - 1] = 0;
    return 0;
}

static int jint(jcur_t *c, int64_t *v) {
    jws(c);
    char *e;
    long long x = strtoll(c->p, &e, 10);
    if (e == c->p) return -1;
    c->p = e;
    *v = x;
    return 0;
}

static int jexpect(jcur_t *c, char ch) {
    jws(c);
    if (c->p >= c->end || *c->p != ch) return -1;
    c->p++;
    return 0;
}

/* Skips any JSON value (used for __metadata__ and unknown fields). */
static int jskip(jcur_t *c) {
    jws(c);
    if (c->p >= c->end) return -1;
    char ch = *c->p;
    if (ch == '"') return jstr(c, NULL, 0);
    if (ch == '{' || ch == '[') {
        int depth = 0;
        while (c->p < c->end) {
            char d = *c->p;
            if (d == '"') { if (jstr(c, NULL, 0)) return -1; continue; }
            if (d == '{' || d == '[') depth++;
            if (d == '}' || d == ']') { depth--; if (depth == 0) { c->p++; return 0; } }
            c->p++;
        }
        return -1;
    }
    while (c->p < c->end && *c->p != ',' && *c->p != '}' && *c->p != ']') c->p++;
    return 0;
}

static int jarray_ints(jcur_t *c, int64_t *v, int cap) {
    if (jexpect(c, '[')) return -1;
    int n = 0;
    jws(c);
    if (c->p < c->end && *c->p == ']') { c->p++; return 0; }
    for (;;) {
        int64_t x;
        if (jint(c, &x)) return -1;
        if (n < cap) v[n] = x;
        n++;
        jws(c);
        if (c->p < c->end && *c->p == ',') { c->p++; continue; }
        if (jexpect(c, ']')) return -1;
        return n;
    }
}

static iris_st_dtype_t parse_dtype(const char *s) {
    if (!strcmp(s, "F32")) return IRIS_ST_F32;
    if (!strcmp(s, "F16")) return IRIS_ST_F16;
    if (!strcmp(s, "BF16")) return IRIS_ST_BF16;
    return IRIS_ST_OTHER;
}

static int parse_header(iris_st_file_t *f, const char *json, size_t len, size_t data_len) {
    jcur_t c = { json, json + len };
    if (jexpect(&c, '{')) return -1;
    int cap = 256;
    f->t = (iris_st_tensor_t *)calloc((size_t)cap, sizeof(iris_st_tensor_t));
    if (!f->t) return -1;
    f->n = 0;
    for (;;) {
        jws(&c);
        if (c.p < c.end && *c.p == '}') break;
        char key[200];
        if (jstr(&c, key, sizeof(key))) return -1;
        if (jexpect(&c, ':')) return -1;
        if (!strcmp(key, "__metadata__")) {
            if (jskip(&c)) return -1;
        } else {
            if (f->n == cap) {
                cap *= 2;
                iris_st_tensor_t *nt = (iris_st_tensor_t *)realloc(f->t, (size_t)cap * sizeof(*nt));
                if (!nt) return -1;
                f->t = nt;
            }
            iris_st_tensor_t *t = &f->t[f->n];
            memset(t, 0, sizeof(*t));
            snprintf(t->name, sizeof(t->name), "%s", key);
            if (jexpect(&c, '{')) return -1;
            int64_t offs[2] = {0, 0};
            for (;;) {
                jws(&c);
                if (c.p < c.end && *c.p == '}') { c.p++; break; }
                char fk[32];
                if (jstr(&c, fk, sizeof(fk))) return -1;
                if (jexpect(&c, ':')) return -1;
                if (!strcmp(fk, "dtype")) {
                    char dt[16];
                    if (jstr(&c, dt, sizeof(dt))) return -1;
                    t->dtype = parse_dtype(dt);
                } else if (!strcmp(fk, "shape")) {
                    int nd = jarray_ints(&c, t->shape, 6);
                    if (nd < 0 || nd > 6) return -1;
                    t->ndim = nd;
                } else if (!strcmp(fk, "data_offsets")) {
                    if (jarray_ints(&c, offs, 2) != 2) return -1;
                } else {
                    if (jskip(&c)) return -1;
                }
                jws(&c);
                if (c.p < c.end && *c.p == ',') c.p++;
            }
            if (offs[0] < 0 || offs[1] < offs[0] || (size_t)offs[1] > data_len) return -1;
            t->offset = (size_t)offs[0];
            t->nbytes = (size_t)(offs[1] - offs[0]);
            f->n++;
        }
        jws(&c);
        if (c.p < c.end && *c.p == ',') { c.p++; continue; }
        if (jexpect(&c, '}')) return -1;
        break;
    }
    return 0;
}

iris_st_file_t *iris_st_open(const char *path) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) return NULL;
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 8) { close(fd); return NULL; }
    void *map = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return NULL;
    iris_st_file_t *f = (iris_st_file_t *)calloc(1, sizeof(*f));
    if (!f) { munmap(map, (size_t)st.st_size); return NULL; }
    f->map = map;
    f->map_size = (size_t)st.st_size;
    uint64_t hlen;
    memcpy(&hlen, map, 8);
    if (hlen > f->map_size - 8) { iris_st_close(f); return NULL; }
    f->data = (const uint8_t *)map + 8 + hlen;
    if (parse_header(f, (const char *)map + 8, (size_t)hlen, f->map_size - 8 - (size_t)hlen)) {
        fprintf(stderr, "iris_st_open: bad safetensors header in %s\n", path);
        iris_st_close(f);
        return NULL;
    }
    return f;
}

void iris_st_close(iris_st_file_t *f) {
    if (!f) return;
    if (f->map) munmap(f->map, f->map_size);
    free(f->t);
    free(f);
}

const iris_st_tensor_t *iris_st_find(const iris_st_file_t *f, const char *name) {
    for (int i = 0; i < f->n; i++)
        if (!strcmp(f->t[i].name, name)) return &f->t[i];
    return NULL;
}

const void *iris_st_ptr(const iris_st_file_t *f, const iris_st_tensor_t *t) {
    return f->data + t->offset;
}

int64_t iris_st_numel(const iris_st_tensor_t *t) {
    int64_t n = 1;
    for (int i = 0; i < t->ndim; i++) n *= t->shape[i];
    return n;
}

static float f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff, u;
    if (e == 0) {
        if (m == 0) u = s;
        else {            /* subnormal */
            e = 127 - 15 + 1;
            while (!(m & 0x400)) { m <<= 1; e--; }
            m &= 0x3ff;
            u = s | (e << 23) | (m << 13);
        }
    } else if (e == 31) u = s | 0x7f800000u | (m << 13);
    else u = s | ((e + 127 - 15) << 23) | (m << 13);
    union { uint32_t u; float f; } v = { u };
    return v.f;
}

int iris_st_read_f32(const iris_st_file_t *f, const iris_st_tensor_t *t, float *dst) {
    int64_t n = iris_st_numel(t);
    const uint8_t *src = (const uint8_t *)iris_st_ptr(f, t);
    switch (t->dtype) {
    case IRIS_ST_F32:
        if (t->nbytes != (size_t)n * 4) return -1;
        memcpy(dst, src, (size_t)n * 4);
        return 0;
    case IRIS_ST_BF16:
        if (t->nbytes != (size_t)n * 2) return -1;
        for (int64_t i = 0; i < n; i++) {
            uint16_t b; memcpy(&b, src + 2 * i, 2);
            dst[i] = iris_bf16_to_f32(b);
        }
        return 0;
    case IRIS_ST_F16:
        if (t->nbytes != (size_t)n * 2) return -1;
        for (int64_t i = 0; i < n; i++) {
            uint16_t b; memcpy(&b, src + 2 * i, 2);
            dst[i] = f16_to_f32(b);
        }
        return 0;
    default:
        return -1;
    }
}

int iris_st_read_bf16(const iris_st_file_t *f, const iris_st_tensor_t *t, uint16_t *dst) {
    int64_t n = iris_st_numel(t);
    const uint8_t *src = (const uint8_t *)iris_st_ptr(f, t);
    switch (t->dtype) {
    case IRIS_ST_BF16:
        if (t->nbytes != (size_t)n * 2) return -1;
        memcpy(dst, src, (size_t)n * 2);
        return 0;
    case IRIS_ST_F32:
        if (t->nbytes != (size_t)n * 4) return -1;
        for (int64_t i = 0; i < n; i++) {
            float x; memcpy(&x, src + 4 * i, 4);
            dst[i] = iris_f32_to_bf16(x);
        }
        return 0;
    case IRIS_ST_F16:
        if (t->nbytes != (size_t)n * 2) return -1;
        for (int64_t i = 0; i < n; i++) {
            uint16_t b; memcpy(&b, src + 2 * i, 2);
            dst[i] = iris_f32_to_bf16(f16_to_f32(b));
        }
        return 0;
    default:
        return -1;
    }
}

/* Shard discovery: the index json's weight_map values name the shard files
 * (iris_transformer_flux.c:473-557); otherwise a single file. */
int iris_st_set_open_files(iris_st_set_t *s, const char *dir, const char *index_name, const char *const *fallback,
                           int n_fallback) {
    memset(s, 0, sizeof(*s));
    char path[4096];
    snprintf(path, sizeof(path), "%.2047s/%.1023s", dir, index_name);
    FILE *fp = fopen(path, "rb");
    if (fp) {
        fseek(fp, 0, SEEK_END);
        long len = ftell(fp);
        fseek(fp, 0, SEEK_SET);
        char *json = (char *)malloc((size_t)len + 1);
        if (!json) { fclose(fp); return -1; }
        size_t got = fread(json, 1, (size_t)len, fp);
        fclose(fp);
        json[got] = 0;
        char names[IRIS_ST_MAX_SHARDS][1024];
        int nn = 0;
        const char *p = strstr(json, "\"weight_map\"");
        if (p) p = strchr(p, '{');
        jcur_t c = { p ? p + 1 : json, json + got };
        while (p) {
            jws(&c);
            if (c.p >= c.end || *c.p == '}') break;
            char k[256], v[256];
            if (jstr(&c, k, sizeof(k)) || jexpect(&c, ':') || jstr(&c, v, sizeof(v))) break;
            int dup = 0;
            for (int i = 0; i < nn; i++) if (!strcmp(names[i], v)) dup = 1;
            if (!dup && nn < IRIS_ST_MAX_SHARDS) snprintf(names[nn++], 1024, "%s", v);
            jws(&c);
            if (c.p < c.end && *c.p == ',') c.p++;
        }
        free(json);
        for (int i = 0; i < nn; i++) {
            snprintf(path, sizeof(path), "%.2047s/%.1023s", dir, names[i]);
            s->f[s->n] = iris_st_open(path);
            if (!s->f[s->n]) {
                fprintf(stderr, "iris_st: failed to open shard %s\n", path);
                iris_st_set_close(s);
                return -1;
            }
            s->n++;
        }
        if (s->n > 0) return 0;
    }
    /* no index: the fallback names, all of one group present; groups are
     * separated by NULL entries */
    for (int i = 0; i < n_fallback; i++) {
        int j = i, ok = 1;
        while (j < n_fallback && fallback[j]) {
            snprintf(path, sizeof(path), "%.2047s/%.1023s", dir, fallback[j]);
            if (ok && s->n < IRIS_ST_MAX_SHARDS && (s->f[s->n] = iris_st_open(path))) s->n++;
            else ok = 0;
            j++;
        }
        if (ok && s->n > 0) return 0;
        iris_st_set_close(s);
        i = j;
    }
    return -1;
}

int iris_st_set_open(iris_st_set_t *s, const char *model_dir) {
    char dir[2048];
    snprintf(dir, sizeof(dir), "%s/transformer", model_dir);
    static const char *const fb[] = {"diffusion_pytorch_model.safetensors"};
    return iris_st_set_open_files(s, dir, "diffusion_pytorch_model.safetensors.index.json", fb, 1);
}

void iris_st_set_close(iris_st_set_t *s) {
    for (int i = 0; i < s->n; i++) iris_st_close(s->f[i]);
    s->n = 0;
}

const iris_st_tensor_t *iris_st_set_find(const iris_st_set_t *s, const char *name,
                                         const iris_st_file_t **owner) {
    for (int i = 0; i < s->n; i++) {
        const iris_st_tensor_t *t = iris_st_find(s->f[i], name);
        if (t) { if (owner) *owner = s->f[i]; return t; }
    }
    return NULL;
}
