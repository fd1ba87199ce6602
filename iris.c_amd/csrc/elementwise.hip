/*
 * elementwise.hip - HBM-bound kernels of the denoiser step on gfx950.
 *
 *   rownorm        apply_adaln (iris_transformer_flux.c:1391-1460), the final
 *                  layer's LayerNorm (:4280-4285), Z-Image RMSNorm / final
 *                  LayerNorm (iris_transformer_zimage.c:657-668, :1590-1606)
 *   rms_gated_add  Z-Image x += gate * RMSNorm(y) (:818-836)
 *   qk_prepare     apply_qk_norm + apply_rope_2d (:1464-1518, :1026-1048),
 *                  zi_qk_norm + zi_apply_rope (zimage :620-682), and the
 *                  transposed V layout the attention kernel reads
 *   gemv           timestep MLP and modulation (:1366-1379, :4059-4069)
 *   layout         NCHW -> tokens (:3986-3993), patchify (zimage :1634-1684),
 *                  f32 <-> bf16, Euler update (iris_sample.c:359, :472-474)
 * One block of 256 threads per row for the row kernels; float4 / 16-byte
 * accesses throughout.
 */
#include "iris_internal.h"

namespace {

constexpr int NT = 256;
constexpr int MAXV = 4;      /* float4 per thread: cols <= 4096 */

__global__ __launch_bounds__(NT) void rownorm_kernel(const iris_norm_args_t a) {
    __shared__ float red[NT / IRIS_WAVE];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *x = a.x + (size_t)row * a.ldx;
    const int nv = a.cols >> 2;
    float4 v[MAXV];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXV; i++) {
        const int c = tid + i * NT;
        v[i] = c < nv ? ((const float4 *)x)[c] : make_float4(0, 0, 0, 0);
        s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
    const bool use_b = (a.period ? row % a.period : row) >= a.split;
    const float *shift = use_b ? a.shiftB : a.shiftA;
    const float *scale = use_b ? a.scaleB : a.scaleA;
    const float *w = use_b ? a.wB : a.wA;
    float mean = 0.0f, inv;
    if (a.mode == IRIS_NORM_RMS) {
        float q = 0.0f;
#pragma unroll
        for (int i = 0; i < MAXV; i++) q += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
        q = block_sum<NT / IRIS_WAVE>(q, red);
        inv = 1.0f / sqrtf(q / a.cols + a.eps);
    } else {
        mean = block_sum<NT / IRIS_WAVE>(s, red) / a.cols;
        float q = 0.0f;
#pragma unroll
        for (int i = 0; i < MAXV; i++) {
            const int c = tid + i * NT;
            if (c < nv) {
                float d0 = v[i].x - mean, d1 = v[i].y - mean, d2 = v[i].z - mean, d3 = v[i].w - mean;
                q += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
            }
        }
        q = block_sum<NT / IRIS_WAVE>(q, red);
        inv = 1.0f / sqrtf(q / a.cols + a.eps);
    }
#pragma unroll
    for (int i = 0; i < MAXV; i++) {
        const int c = tid + i * NT;
        if (c >= nv) continue;
        float e[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        float y[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int col = 4 * c + j;
            if (a.mode == IRIS_NORM_LN_MOD) {
                const float n = (e[j] - mean) * inv;
                y[j] = (1.0f + scale[col]) * n + shift[col];
            } else if (a.mode == IRIS_NORM_LN_SCALE) {
                y[j] = (e[j] - mean) * inv * scale[col];
            } else {
                float t = e[j] * inv * w[col];
                if (scale) t *= scale[col];
                y[j] = t;
            }
        }
        if (a.out_bf16) {
            u16x4 o = {f2bf(y[0]), f2bf(y[1]), f2bf(y[2]), f2bf(y[3])};
            *(u16x4 *)((uint16_t *)a.out + (size_t)row * a.ldo + 4 * c) = o;
        } else {
            *(float4 *)((float *)a.out + (size_t)row * a.ldo + 4 * c) = make_float4(y[0], y[1], y[2], y[3]);
        }
    }
}

__global__ __launch_bounds__(NT) void rms_gated_add_kernel(float *x, const float *y, const float *w,
                                                           const float *gate, int cols, float eps, int gate_tanh) {
    __shared__ float red[NT / IRIS_WAVE];
    const int row = blockIdx.x, tid = threadIdx.x, nv = cols >> 2;
    const float *yr = y + (size_t)row * cols;
    float *xr = x + (size_t)row * cols;
    float4 v[MAXV];
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXV; i++) {
        const int c = tid + i * NT;
        v[i] = c < nv ? ((const float4 *)yr)[c] : make_float4(0, 0, 0, 0);
        q += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
    }
    q = block_sum<NT / IRIS_WAVE>(q, red);
    const float inv = 1.0f / sqrtf(q / cols + eps);
#pragma unroll
    for (int i = 0; i < MAXV; i++) {
        const int c = tid + i * NT;
        if (c >= nv) continue;
        float4 xo = ((float4 *)xr)[c];
        float e[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        float *xp = &xo.x;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int col = 4 * c + j;
            const float g = gate ? (gate_tanh ? tanhf(gate[col]) : gate[col]) : 1.0f;
            xp[j] += g * (e[j] * inv * w[col]);
        }
        ((float4 *)xr)[c] = xo;
    }
}

/* one wave per (row, head): lane i owns the rotation pair (2i, 2i+1) */
__global__ __launch_bounds__(NT) void qk_norm_rope_kernel(const iris_qkprep_args_t a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * (NT / IRIS_WAVE) + wave, head = blockIdx.y;
    if (row >= a.rows) return;
    const int prow = a.period ? row % a.period : row;
    const bool use_b = prow >= a.split;
    const float *wq = use_b ? a.wqB : a.wqA;
    const float *wk = use_b ? a.wkB : a.wkA;
    const int d = 2 * lane;
    float c = 1.0f, s = 0.0f;
    if (a.cos_t) {
        c = a.cos_t[(size_t)prow * 128 + d];
        s = a.sin_t[(size_t)prow * 128 + d];
    }
    const size_t out_off = (size_t)row * a.heads * 128 + head * 128 + d;
#pragma unroll
    for (int which = 0; which < 2; which++) {
        const uint16_t *src = a.qkv + (size_t)row * a.ld_qkv + (which ? a.col_k : 0) + head * 128 + d;
        const uint32_t pr = *(const uint32_t *)src;
        float x0 = bf2f((uint16_t)(pr & 0xffff)), x1 = bf2f((uint16_t)(pr >> 16));
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float inv = 1.0f / sqrtf(ss / 128.0f + a.eps);
        const float *w = which ? wk : wq;
        x0 = x0 * inv * w[d];
        x1 = x1 * inv * w[d + 1];
        const float y0 = x0 * c - x1 * s, y1 = x1 * c + x0 * s;
        uint16_t *dst = (which ? a.k_out : a.q_out) + out_off;
        *(uint32_t *)dst = (uint32_t)f2bf(y0) | ((uint32_t)f2bf(y1) << 16);
    }
}

/* V [rows][128] (head slice of qkv) -> V^T [head][128][ld_vt], 64 rows per block */
__global__ __launch_bounds__(NT) void v_transpose_kernel(const iris_qkprep_args_t a) {
    __shared__ uint16_t t[128][64 + 2];
    const int r0 = blockIdx.x * 64, head = blockIdx.y, tid = threadIdx.x;
    for (int i = tid; i < 64 * 64; i += NT) {              /* 64 rows x 64 pairs */
        const int r = i >> 6, p = i & 63;
        uint32_t pr = 0;
        if (r0 + r < a.rows)
            pr = *(const uint32_t *)(a.qkv + (size_t)(r0 + r) * a.ld_qkv + a.col_v + head * 128 + 2 * p);
        t[2 * p][r] = (uint16_t)(pr & 0xffff);
        t[2 * p + 1][r] = (uint16_t)(pr >> 16);
    }
    __syncthreads();
    uint16_t *dst = a.vt_out + (size_t)head * 128 * a.ld_vt + r0;
    for (int i = tid; i < 128 * 32; i += NT) {             /* 128 d x 32 pairs of rows */
        const int d = i >> 5, p = i & 31;
        if (r0 + 2 * p < a.ld_vt)
            *(uint32_t *)(dst + (size_t)d * a.ld_vt + 2 * p) = (uint32_t)t[d][2 * p] | ((uint32_t)t[d][2 * p + 1] << 16);
    }
}

/* one wave per output row */
__global__ __launch_bounds__(NT) void gemv_kernel(float *y, const uint16_t *W, const float *x, const float *bias,
                                                  int N, int K, int act_in) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n = blockIdx.x * (NT / IRIS_WAVE) + wave;
    if (n >= N) return;
    const uint16_t *w = W + (size_t)n * K;
    float acc = 0.0f;
    for (int k = lane * 8; k < K; k += 64 * 8) {
        const u16x8 wv = *(const u16x8 *)(w + k);
        const float4 xa = *(const float4 *)(x + k), xb = *(const float4 *)(x + k + 4);
        float xs[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float xv = xs[e];
            if (act_in == 1) xv = xv / (1.0f + __expf(-xv));
            acc += bf2f(wv[e]) * xv;
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) y[n] = acc + (bias ? bias[n] : 0.0f);
}

__global__ void nchw_to_tokens_kernel(uint16_t *out, const float *lat, int C, int hw) {
    __shared__ float t[64][65];
    const int p0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
    for (int i = threadIdx.x; i < 64 * 64; i += NT) {
        const int c = i >> 6, p = i & 63;
        t[c][p] = (c0 + c < C && p0 + p < hw) ? lat[(size_t)(c0 + c) * hw + p0 + p] : 0.0f;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 64; i += NT) {
        const int p = i >> 6, c = i & 63;
        if (c0 + c < C && p0 + p < hw) out[(size_t)(p0 + p) * C + c0 + c] = f2bf(t[c][p]);
    }
}

__global__ void f32_to_bf16_kernel(uint16_t *o, const float *x, size_t n) {
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) o[i] = f2bf(x[i]);
}

__global__ void bf16_to_f32_kernel(float *o, const uint16_t *x, size_t n) {
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) o[i] = bf2f(x[i]);
}

__global__ void euler_kernel(float *z, const float *v, const float *v2, float g, float dt, float sign, size_t n) {
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) {
        float vv = v[i];
        if (v2) vv = vv + g * (v2[i] - vv);
        z[i] += dt * (sign * vv);
    }
}

__global__ void patchify_kernel(uint16_t *out, const float *lat, int C, int H, int W, int ps) {
    const int Wt = W / ps, pf = ps * ps * C;
    const size_t n = (size_t)(H / ps) * Wt * pf;
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) {
        const int patch = (int)(i / pf), e = (int)(i % pf);
        const int h = patch / Wt, w = patch % Wt;
        const int py = e / (ps * C), px = (e / C) % ps, c = e % C;
        out[i] = f2bf(lat[(size_t)c * H * W + (size_t)(h * ps + py) * W + (w * ps + px)]);
    }
}

__global__ void unpatchify_kernel(float *lat, const float *pt, int C, int H, int W, int ps) {
    const int Wt = W / ps, pf = ps * ps * C;
    const size_t n = (size_t)(H / ps) * Wt * pf;
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) {
        const int patch = (int)(i / pf), e = (int)(i % pf);
        const int h = patch / Wt, w = patch % Wt;
        const int py = e / (ps * C), px = (e / C) % ps, c = e % C;
        lat[(size_t)c * H * W + (size_t)(h * ps + py) * W + (w * ps + px)] = pt[i];
    }
}

__global__ void fill_rows_kernel(float *x, const float *row, int r0, int r1, int cols) {
    const size_t n = (size_t)(r1 - r0) * cols;
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT)
        x[(size_t)r0 * cols + i] = row[i % cols];
}

int grid1d(size_t n) {
    size_t b = (n + NT - 1) / NT;
    return (int)(b < 8192 ? (b ? b : 1) : 8192);
}

}  // namespace

extern "C" {

int iris_hip_rownorm(const iris_norm_args_t *a) {
    if (a->rows <= 0) return 0;
    if (a->cols % 4 || a->cols > NT * 4 * MAXV) return iris_set_error("rownorm: cols=%d", a->cols);
    if (a->ldx % 4 || a->ldo % 4) return iris_set_error("rownorm: ld must be multiple of 4");
    hipLaunchKernelGGL(rownorm_kernel, dim3(a->rows), dim3(NT), 0, iris_stream(), *a);
    return iris_launch_check("rownorm_kernel");
}

int iris_hip_rms_gated_add(float *x, const float *y, const float *w, const float *gate, int rows, int cols,
                           float eps, int gate_tanh) {
    if (rows <= 0) return 0;
    if (cols % 4 || cols > NT * 4 * MAXV) return iris_set_error("rms_gated_add: cols=%d", cols);
    hipLaunchKernelGGL(rms_gated_add_kernel, dim3(rows), dim3(NT), 0, iris_stream(), x, y, w, gate, cols, eps,
                       gate_tanh);
    return iris_launch_check("rms_gated_add_kernel");
}

int iris_hip_qk_prepare(const iris_qkprep_args_t *a) {
    if (a->rows <= 0) return 0;
    if (a->ld_qkv % 2 || a->col_k % 2 || a->col_v % 2) return iris_set_error("qk_prepare: odd layout");
    if (a->ld_vt < a->rows || a->ld_vt % 64) return iris_set_error("qk_prepare: ld_vt=%d", a->ld_vt);
    hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((a->rows + 3) / 4, a->heads), dim3(NT), 0, iris_stream(), *a);
    if (iris_launch_check("qk_norm_rope_kernel")) return -1;
    hipLaunchKernelGGL(v_transpose_kernel, dim3(a->ld_vt / 64, a->heads), dim3(NT), 0, iris_stream(), *a);
    return iris_launch_check("v_transpose_kernel");
}

int iris_hip_gemv(float *y, const uint16_t *W, const float *x, const float *bias, int N, int K, int act_in) {
    if (N <= 0) return 0;
    if (K % 8) return iris_set_error("gemv: K=%d must be a multiple of 8", K);
    hipLaunchKernelGGL(gemv_kernel, dim3((N + 3) / 4), dim3(NT), 0, iris_stream(), y, W, x, bias, N, K, act_in);
    return iris_launch_check("gemv_kernel");
}

int iris_hip_nchw_to_tokens(uint16_t *out, const float *lat, int C, int hw) {
    if (hw <= 0) return 0;
    hipLaunchKernelGGL(nchw_to_tokens_kernel, dim3((hw + 63) / 64, (C + 63) / 64), dim3(NT), 0, iris_stream(), out,
                       lat, C, hw);
    return iris_launch_check("nchw_to_tokens_kernel");
}

int iris_hip_f32_to_bf16(uint16_t *o, const float *x, size_t n) {
    if (!n) return 0;
    hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), o, x, n);
    return iris_launch_check("f32_to_bf16_kernel");
}

int iris_hip_bf16_to_f32(float *o, const uint16_t *x, size_t n) {
    if (!n) return 0;
    hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), o, x, n);
    return iris_launch_check("bf16_to_f32_kernel");
}

int iris_hip_euler(float *z, const float *v, const float *v2, float g, float dt, float sign, size_t n) {
    if (!n) return 0;
    hipLaunchKernelGGL(euler_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), z, v, v2, g, dt, sign, n);
    return iris_launch_check("euler_kernel");
}

int iris_hip_patchify(uint16_t *o, const float *lat, int C, int H, int W, int ps) {
    size_t n = (size_t)(H / ps) * (W / ps) * ps * ps * C;
    if (!n) return 0;
    hipLaunchKernelGGL(patchify_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), o, lat, C, H, W, ps);
    return iris_launch_check("patchify_kernel");
}

int iris_hip_unpatchify(float *lat, const float *pt, int C, int H, int W, int ps) {
    size_t n = (size_t)(H / ps) * (W / ps) * ps * ps * C;
    if (!n) return 0;
    hipLaunchKernelGGL(unpatchify_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), lat, pt, C, H, W, ps);
    return iris_launch_check("unpatchify_kernel");
}

int iris_hip_fill_rows(float *x, const float *row, int r0, int r1, int cols) {
    if (r1 <= r0) return 0;
    size_t n = (size_t)(r1 - r0) * cols;
    hipLaunchKernelGGL(fill_rows_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), x, row, r0, r1, cols);
    return iris_launch_check("fill_rows_kernel");
}

}  /* extern "C" */
