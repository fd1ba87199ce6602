/*
 * iris_st.h - memory-mapped safetensors reader for the HIP build.
 *
 * Role: the source of the one-time device weight upload. A file is mapped
 * read-only; tensors are located by name and their bytes are handed to the
 * device upload without an intermediate host copy (bf16 stays bf16).
 *
 * Format (same on-disk format the reference reads, iris_safetensors.c:233):
 *   u64 little-endian header length N, N bytes of JSON
 *   {"name": {"dtype": "BF16", "shape": [..], "data_offsets": [b, e]}, ...}
 *   followed by the raw tensor bytes; offsets are relative to the data start.
 */
#ifndef IRIS_ST_H
#define IRIS_ST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    IRIS_ST_F32 = 0,
    IRIS_ST_F16 = 1,
    IRIS_ST_BF16 = 2,
    IRIS_ST_OTHER = 3
} iris_st_dtype_t;

typedef struct {
    char name[200];
    iris_st_dtype_t dtype;
    int ndim;
    int64_t shape[6];
    size_t offset;      /* from start of the data section */
    size_t nbytes;
} iris_st_tensor_t;

typedef struct {
    void *map;
    size_t map_size;
    const uint8_t *data;   /* start of the data section */
    int n;
    iris_st_tensor_t *t;
} iris_st_file_t;

iris_st_file_t *iris_st_open(const char *path);
void iris_st_close(iris_st_file_t *f);
const iris_st_tensor_t *iris_st_find(const iris_st_file_t *f, const char *name);
const void *iris_st_ptr(const iris_st_file_t *f, const iris_st_tensor_t *t);
int64_t iris_st_numel(const iris_st_tensor_t *t);
/* Widen any float dtype to a caller-provided f32 array (n = numel). */
int iris_st_read_f32(const iris_st_file_t *f, const iris_st_tensor_t *t, float *dst);
/* Narrow/copy any float dtype to bf16 (RNE for f32 sources, exact for bf16). */
int iris_st_read_bf16(const iris_st_file_t *f, const iris_st_tensor_t *t, uint16_t *dst);

/* A set of shards opened from a model's transformer/ directory. */
#define IRIS_ST_MAX_SHARDS 32
typedef struct {
    iris_st_file_t *f[IRIS_ST_MAX_SHARDS];
    int n;
} iris_st_set_t;

/* Opens <dir>/transformer/diffusion_pytorch_model.safetensors[.index.json]
 * (the shard discovery of iris_transformer_flux.c:470-570). Returns 0 on success. */
int iris_st_set_open(iris_st_set_t *s, const char *model_dir);
/* Opens the shards that <dir>/<index_name> lists in its weight_map, or, with
 * no index, the first group of fallback names (groups separated by NULL)
 * whose files all open. Returns 0 on success. */
int iris_st_set_open_files(iris_st_set_t *s, const char *dir, const char *index_name, const char *const *fallback,
                           int n_fallback);
void iris_st_set_close(iris_st_set_t *s);
const iris_st_tensor_t *iris_st_set_find(const iris_st_set_t *s, const char *name,
                                         const iris_st_file_t **owner);

static inline float iris_bf16_to_f32(uint16_t b) {
    union { uint32_t u; float f; } v;
    v.u = (uint32_t)b << 16;
    return v.f;
}
static inline uint16_t iris_f32_to_bf16(float f) {
    union { float f; uint32_t u; } v;
    v.f = f;
    if ((v.u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;   /* NaN */
    v.u += 0x7fffu + ((v.u >> 16) & 1u);                    /* round to nearest even */
    return (uint16_t)(v.u >> 16);
}

#ifdef __cplusplus
}
#endif
#endif
