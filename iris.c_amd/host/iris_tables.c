/*
 * iris_tables.c - host-built position and timestep tables, uploaded once per
 * geometry (RoPE) or per step (timestep sinusoid).
 *
 * Bit-exactness: the reference is compiled with -O3 -march=native -ffast-math
 * (Makefile:5); gcc then evaluates the RoPE base frequencies
 * `1.0f / powf(theta, 2d/axis)` (iris_transformer_flux.c:903-906,
 * iris_transformer_zimage.c:603) as glibc libmvec's vector powf(theta, -2d/axis)
 * while cosf/sinf and the timestep expf stay scalar libm calls. This file calls
 * the same libmvec entry point explicitly and is compiled without -ffast-math,
 * so the tables carry the reference build's bits independent of flags.
 */
#include "iris_tables.h"

#include <immintrin.h>
#include <math.h>
#include <string.h>

__m128 _ZGVbN4vv_powf(__m128, __m128);

static void rope_bases(float *base, int half, int axis_dim, float theta) {
    for (int d = 0; d < half; d += 4) {
        float x[4], y[4], o[4];
        for (int j = 0; j < 4; j++) {
            x[j] = theta;
            y[j] = d + j < half ? -((float)(2 * (d + j)) / (float)axis_dim) : 0.0f;
        }
        _mm_storeu_ps(o, _ZGVbN4vv_powf(_mm_loadu_ps(x), _mm_loadu_ps(y)));
        for (int j = 0; j < 4 && d + j < half; j++) base[d + j] = o[j];
    }
}

/* one axis of 2*half dims: each frequency's cos/sin duplicated into the pair */
static void axis_fill(float *c, float *s, int pos, const float *base, int half) {
    for (int d = 0; d < half; d++) {
        float a = (float)pos * base[d];
        float cv = cosf(a), sv = sinf(a);
        c[2 * d] = cv; c[2 * d + 1] = cv;
        s[2 * d] = sv; s[2 * d + 1] = sv;
    }
}

static void axis_identity(float *c, float *s, int n) {
    for (int d = 0; d < n; d++) { c[d] = 1.0f; s[d] = 0.0f; }
}

/* compute_rope_2d / _with_t_offset (iris_transformer_flux.c:896-1018):
 * axes T (t_offset, identity when 0), H = y, W = x, L = 0. Rows of 4*axis_dim. */
void iris_rope_img(float *cos_out, float *sin_out, int ph, int pw, int axis_dim, float theta, int t_offset) {
    int half = axis_dim / 2, hd = 4 * axis_dim;
    float base[64];
    rope_bases(base, half, axis_dim, theta);
    for (int y = 0; y < ph; y++)
        for (int x = 0; x < pw; x++) {
            float *c = cos_out + (size_t)(y * pw + x) * hd, *s = sin_out + (size_t)(y * pw + x) * hd;
            if (t_offset == 0) axis_identity(c, s, axis_dim);
            else axis_fill(c, s, t_offset, base, half);
            axis_fill(c + axis_dim, s + axis_dim, y, base, half);
            axis_fill(c + 2 * axis_dim, s + 2 * axis_dim, x, base, half);
            axis_identity(c + 3 * axis_dim, s + 3 * axis_dim, axis_dim);
        }
}

/* One axis's per-pair values at positions 0 .. len-1: [len][axis_dim / 2],
 * through axis_fill (entry d of position p = column 2d of that axis's rows). */
void iris_rope_axis(float *cos_out, float *sin_out, int len, int axis_dim, float theta) {
    int half = axis_dim / 2;
    float base[64], c[128], s[128];
    rope_bases(base, half, axis_dim, theta);
    for (int p = 0; p < len; p++) {
        axis_fill(c, s, p, base, half);
        for (int d = 0; d < half; d++) {
            cos_out[(size_t)p * half + d] = c[2 * d];
            sin_out[(size_t)p * half + d] = s[2 * d];
        }
    }
}

/* compute_rope_text (iris_transformer_flux.c:1055-1087): only axis L = s rotates */
void iris_rope_txt(float *cos_out, float *sin_out, int txt_seq, int axis_dim, float theta) {
    int half = axis_dim / 2, hd = 4 * axis_dim;
    float base[64];
    rope_bases(base, half, axis_dim, theta);
    for (int t = 0; t < txt_seq; t++) {
        float *c = cos_out + (size_t)t * hd, *s = sin_out + (size_t)t * hd;
        axis_identity(c, s, 3 * axis_dim);
        axis_fill(c + 3 * axis_dim, s + 3 * axis_dim, t, base, half);
    }
}

/* zi_precompute_rope (iris_transformer_zimage.c:595-613) expanded per token:
 * axis `ax` of the token's (T, H, W) ids rotates dims [off_ax, off_ax + d_ax);
 * ids outside [0, len) leave the axis unrotated (zi_apply_rope :631), which the
 * identity rows reproduce exactly. */
void iris_rope_zimage(float *cos_out, float *sin_out, const int *pos, int seq, const int *axes,
                      const int *lens, float theta) {
    float base[3][64];
    for (int ax = 0; ax < 3; ax++) rope_bases(base[ax], axes[ax] / 2, axes[ax], theta);
    int hd = axes[0] + axes[1] + axes[2];
    for (int s = 0; s < seq; s++) {
        float *c = cos_out + (size_t)s * hd, *sn = sin_out + (size_t)s * hd;
        int off = 0;
        for (int ax = 0; ax < 3; ax++) {
            int p = pos[s * 3 + ax];
            if (p < 0 || p >= lens[ax]) axis_identity(c + off, sn + off, axes[ax]);
            else axis_fill(c + off, sn + off, p, base[ax], axes[ax] / 2);
            off += axes[ax];
        }
    }
}

/* get_timestep_embedding (iris_transformer_flux.c:1349-1360) and
 * zi_sinusoidal_embedding (iris_transformer_zimage.c:548-557): [cos | sin] */
void iris_timestep_sincos(float *out, float t, int dim, float max_period) {
    int half = dim / 2;
    float lm = logf(max_period);
    for (int i = 0; i < half; i++) {
        float a = t * expf(-lm * (float)i / (float)half);
        out[i] = cosf(a);
        out[i + half] = sinf(a);
    }
}

/* Per-pair copies of [rows][128] tables whose pairs (2i, 2i+1) hold one
 * value: [rows][64], entry i = column 2i (the attention kernel's Q prologue
 * reads one value per rotation pair). */
void iris_rope_pairs(float *pc, float *ps, const float *c, const float *s, size_t rows) {
    for (size_t r = 0; r < rows; r++)
        for (int i = 0; i < 64; i++) {
            pc[r * 64 + i] = c[r * 128 + 2 * i];
            ps[r * 64 + i] = s[r * 128 + 2 * i];
        }
}
