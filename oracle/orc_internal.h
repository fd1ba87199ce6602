/* orc_internal.h - shared declarations of the oracle (TEST INFRASTRUCTURE ONLY). */
#ifndef ORC_INTERNAL_H
#define ORC_INTERNAL_H
#include "iris_oracle.h"
#include "../iris.c_amd/host/iris_st.h"
#include "../include/iris_synth.h"

void orc_sgemm_nt(int M, int N, int K, float alpha, const float *A, int lda,
                  const float *B, int ldb, float beta, float *C, int ldc);
void orc_sgemm_nn(int M, int N, int K, float alpha, const float *A, int lda,
                  const float *B, int ldb, float beta, float *C, int ldc);
void orc_linear(float *y, const float *x, const float *W, const float *b,
                int seq, int in_dim, int out_dim);
void orc_silu(float *x, int n);
void orc_silu_mul(float *gate, const float *up, size_t n);
void orc_softmax(float *x, int rows, int cols);
void orc_rms_norm(float *out, const float *x, const float *w, int rows, int dim, float eps);
void orc_vpowf(float *out, const float *x, const float *y, int n);
void orc_vexpf(float *out, const float *x, int n);
void orc_rope_bases(float *base, int half, int axis_dim, float theta);
float *orc_load_f32(const iris_st_set_t *s, const char *name);
float *orc_synth_f32(uint64_t seed, const char *name, size_t n, float mean, float std);
#endif
