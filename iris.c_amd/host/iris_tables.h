/* iris_tables.h - host-built RoPE and timestep tables (see iris_tables.c). */
#ifndef IRIS_TABLES_H
#define IRIS_TABLES_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif
void iris_rope_img(float *cos_out, float *sin_out, int ph, int pw, int axis_dim, float theta, int t_offset);
void iris_rope_txt(float *cos_out, float *sin_out, int txt_seq, int axis_dim, float theta);
void iris_rope_zimage(float *cos_out, float *sin_out, const int *pos, int seq, const int *axes,
                      const int *lens, float theta);
void iris_timestep_sincos(float *out, float t, int dim, float max_period);
void iris_rope_pairs(float *pc, float *ps, const float *c, const float *s, size_t rows);
void iris_rope_axis(float *cos_out, float *sin_out, int len, int axis_dim, float theta);
#ifdef __cplusplus
}
#endif
#endif
