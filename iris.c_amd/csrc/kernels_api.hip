/*
 * kernels_api.hip - device kernels behind the host-pointer kernel API
 * (iris_kernels.h): f32 elementwise ops, normalisations, layout ops, im2col,
 * generic-head-size attention, and the f32 -> (hi, lo) bf16 splits that let the
 * MFMA GEMM reproduce f32 products.
 *
 * A float x is split as hi = bf16(x), lo = bf16(x - hi); then
 * A.B ~= Ahi.Bhi + Ahi.Blo + Alo.Bhi, each product error bounded near 2^-16
 * relative, which keeps the f32 contract of the reference's sgemm calls
 * (iris_kernels.c:220-336) to about 1e-5.
 */
#include "iris_internal.h"

namespace {

constexpr int NT = 256;

int grid_for(size_t n) {
    size_t b = (n + NT - 1) / NT;
    return (int)(b < 16384 ? (b ? b : 1) : 16384);
}

/* The split operands are written as nseg segments of K_pad columns side by
 * side (row stride nseg * K_pad): segment s holds lo(x) when bit s of lo_mask
 * is set, else hi(x). With A = [hi | hi | lo] and W = [hi | lo | hi] a single
 * GEMM over 3 * K_pad accumulates the three cross products in f32. */
__device__ __forceinline__ void put_split(uint16_t *dst, size_t row_off, int k, int K_pad, int nseg, int lo_mask,
                                          float x) {
    const uint16_t hi = f2bf(x);
    const uint16_t lo = f2bf(x - bf2f(hi));
    for (int s = 0; s < nseg; s++) dst[row_off + (size_t)s * K_pad + k] = ((lo_mask >> s) & 1) ? lo : hi;
}

/* src f32 [rows][ld_src] (cols used) -> split segments [rows][nseg * K_pad], zero padded */
__global__ void split_rows_kernel(uint16_t *dst, const float *src, int rows, int cols, int ld_src, int K_pad,
                                  int nseg, int lo_mask) {
    const size_t n = (size_t)rows * K_pad;
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) {
        const int r = (int)(i / K_pad), c = (int)(i % K_pad);
        const float x = c < cols ? src[(size_t)r * ld_src + c] : 0.0f;
        put_split(dst, (size_t)r * nseg * K_pad, c, K_pad, nseg, lo_mask, x);
    }
}

/* src f32 [K][N] -> split segments [N][nseg * K_pad] (transposed, zero padded),
 * 32x32 tiles through LDS */
__global__ void split_transpose_kernel(uint16_t *dst, const float *src, int K, int N, int K_pad, int nseg,
                                       int lo_mask) {
    __shared__ float t[32][33];
    const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   /* 32 x 8 */
    for (int j = ty; j < 32; j += 8) {
        const int k = k0 + j, n = n0 + tx;
        t[j][tx] = (k < K && n < N) ? src[(size_t)k * N + n] : 0.0f;
    }
    __syncthreads();
    for (int j = ty; j < 32; j += 8) {
        const int n = n0 + j, k = k0 + tx;
        if (n < N && k < K_pad) put_split(dst, (size_t)n * nseg * K_pad, k, K_pad, nseg, lo_mask, t[tx][j]);
    }
}

/* bf16 [rows][cols] -> nseg copies side by side in [rows][nseg * K_pad], zero padded */
__global__ void pad_bf16_kernel(uint16_t *dst, const uint16_t *src, int rows, int cols, int K_pad, int nseg) {
    const size_t n = (size_t)rows * K_pad;
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) {
        const int r = (int)(i / K_pad), c = (int)(i % K_pad);
        const uint16_t x = c < cols ? src[(size_t)r * cols + c] : (uint16_t)0;
        for (int s = 0; s < nseg; s++) dst[((size_t)r * nseg + s) * K_pad + c] = x;
    }
}

/* im2col of one image for pixels [pix0, pix0 + npix): row p = output pixel,
 * column k = (ic, kh, kw) in weight order, split into segments [npix][nseg * K_pad] */
__global__ void im2col_split_kernel(uint16_t *dst, const float *in, int C, int H, int W, int kH, int kW,
                                    int stride, int pad, int outW, int pix0, int npix, int K, int K_pad, int nseg,
                                    int lo_mask) {
    const size_t n = (size_t)npix * K_pad;
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) {
        const int p = (int)(i / K_pad), k = (int)(i % K_pad);
        float x = 0.0f;
        if (k < K) {
            const int pix = pix0 + p, oh = pix / outW, ow = pix % outW;
            const int ic = k / (kH * kW), kr = k % (kH * kW), kh = kr / kW, kw = kr % kW;
            const int ih = oh * stride - pad + kh, iw = ow * stride - pad + kw;
            if (ih >= 0 && ih < H && iw >= 0 && iw < W) x = in[((size_t)ic * H + ih) * W + iw];
        }
        put_split(dst, (size_t)p * nseg * K_pad, k, K_pad, nseg, lo_mask, x);
    }
}

/* RMSNorm of each row, one wave per row: out = x * rsqrt(mean(x^2) + eps) * w */
__global__ __launch_bounds__(NT) void rms_rows_kernel(float *out, const float *x, const float *w, int rows, int cols,
                                                      float eps) {
    const int row = blockIdx.x * (NT / IRIS_WAVE) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + (size_t)row * cols;
    float s = 0.0f;
    for (int c = lane; c < cols; c += IRIS_WAVE) s += xr[c] * xr[c];
    const float inv = 1.0f / sqrtf(wave_sum(s) / (float)cols + eps);
    for (int c = lane; c < cols; c += IRIS_WAVE) out[(size_t)row * cols + c] = xr[c] * inv * w[c];
}

__global__ void ew_kernel(int op, float *out, const float *a, const float *b, float s, size_t n) {
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) {
        switch (op) {
        case 0: out[i] = a[i] + b[i]; break;                     /* add */
        case 1: out[i] = a[i] * b[i]; break;                     /* mul */
        case 2: out[i] = a[i] + s * b[i]; break;                 /* axpy */
        case 3: out[i] = a[i] / (1.0f + expf(-a[i])); break;     /* silu */
        default: out[i] = a[i] / (1.0f + expf(-a[i])) * b[i]; break;   /* silu(a) * b */
        }
    }
}

/* out[r][c] += bias[r] */
__global__ void add_row_bias_kernel(float *out, const float *bias, int rows, int cols, int ld) {
    const size_t n = (size_t)rows * cols;
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) {
        const int r = (int)(i / cols), c = (int)(i % cols);
        out[(size_t)r * ld + c] += bias[r];
    }
}

/* softmax over each row, one wave per row */
__global__ __launch_bounds__(NT) void softmax_rows_kernel(float *x, int rows, int cols) {
    const int row = blockIdx.x * (NT / IRIS_WAVE) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    float *r = x + (size_t)row * cols;
    float m = -INFINITY;
    for (int c = lane; c < cols; c += IRIS_WAVE) m = fmaxf(m, r[c]);
    m = wave_max(m);
    float s = 0.0f;
    for (int c = lane; c < cols; c += IRIS_WAVE) {
        const float e = expf(r[c] - m);
        r[c] = e;
        s += e;
    }
    const float inv = 1.0f / wave_sum(s);
    for (int c = lane; c < cols; c += IRIS_WAVE) r[c] *= inv;
}

/* GroupNorm: one block per (batch, group); mean then centred variance */
__global__ __launch_bounds__(NT) void group_norm_kernel(float *out, const float *x, const float *gamma,
                                                        const float *beta, int channels, int spatial, int groups,
                                                        float eps) {
    __shared__ float red[NT / IRIS_WAVE];
    const int b = blockIdx.x / groups, g = blockIdx.x % groups, cpg = channels / groups;
    const size_t base = ((size_t)b * channels + (size_t)g * cpg) * spatial;
    const size_t n = (size_t)cpg * spatial;
    float s = 0.0f;
    for (size_t i = threadIdx.x; i < n; i += NT) s += x[base + i];
    const float mean = block_sum<NT / IRIS_WAVE>(s, red) / (float)n;
    float q = 0.0f;
    for (size_t i = threadIdx.x; i < n; i += NT) {
        const float d = x[base + i] - mean;
        q += d * d;
    }
    const float inv = 1.0f / sqrtf(block_sum<NT / IRIS_WAVE>(q, red) / (float)n + eps);
    for (size_t i = threadIdx.x; i < n; i += NT) {
        const int c = g * cpg + (int)(i / spatial);
        out[base + i] = (x[base + i] - mean) * inv * gamma[c] + beta[c];
    }
}

__global__ void batch_norm_kernel(float *out, const float *x, const float *mean, const float *var,
                                  const float *gamma, const float *beta, int channels, int spatial, size_t n,
                                  float eps) {
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) {
        const int c = (int)((i / spatial) % channels);
        const float g = gamma ? gamma[c] : 1.0f, bb = beta ? beta[c] : 0.0f;
        out[i] = g * (x[i] - mean[c]) * (1.0f / sqrtf(var[c] + eps)) + bb;
    }
}

__global__ void upsample_kernel(float *out, const float *in, int H, int W, int sh, int sw, size_t n) {
    const int oW = W * sw, oHW = H * sh * oW;
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) {
        const size_t plane = i / oHW;
        const int r = (int)(i % oHW), oh = r / oW, ow = r % oW;
        out[i] = in[plane * H * W + (size_t)(oh / sh) * W + ow / sw];
    }
}

/* [B, C, H, W] <-> [B, C*p*p, H/p, W/p]: channel c*p*p + pi*p + pj holds pixel (ph*p + pi, pw*p + pj) */
__global__ void space_to_depth_kernel(float *out, const float *in, int C, int H, int W, int p, int inverse,
                                      size_t n) {
    const int oH = H / p, oW = W / p;
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) {
        /* i indexes the packed [B][C*p*p][oH][oW] tensor */
        const int pw = (int)(i % oW), ph = (int)((i / oW) % oH);
        const size_t oc = (i / ((size_t)oW * oH)) % ((size_t)C * p * p), b = i / ((size_t)oW * oH * C * p * p);
        const int c = (int)(oc / (p * p)), pi = (int)((oc / p) % p), pj = (int)(oc % p);
        const size_t pix = (((b * C + c) * H) + (size_t)(ph * p + pi)) * W + (pw * p + pj);
        if (inverse) out[pix] = in[i];
        else out[i] = in[pix];
    }
}

/* Attention for any head size <= 512 and key count <= 12288, f32 throughout:
 * one block per (sequence, head, query). Row r of q / o of (batch b, head h)
 * starts at b * q_sb + h * q_sh + r * ld, row r of k / v at
 * b * k_sb + h * k_sh + r * ld. */
constexpr int ATT_MAXK = 12288;
__global__ __launch_bounds__(NT) void attention_f32_kernel(float *o, const float *q, const float *k, const float *v,
                                                           int sk, int hd, float scale, long long q_sb,
                                                           long long q_sh, long long k_sb, long long k_sh, int ld) {
    extern __shared__ float sc[];           /* [sk] scores, then [hd] the query */
    __shared__ float red[NT / IRIS_WAVE];
    const int qi = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const size_t qbase = (size_t)b * q_sb + (size_t)h * q_sh;
    const size_t base = (size_t)b * k_sb + (size_t)h * k_sh;
    float *qs = sc + sk;
    for (int d = threadIdx.x; d < hd; d += NT) qs[d] = q[qbase + (size_t)qi * ld + d];
    __syncthreads();
    float m = -INFINITY;
    for (int j = threadIdx.x; j < sk; j += NT) {
        const float *kr = k + base + (size_t)j * ld;
        float acc = 0.0f;
        for (int d = 0; d < hd; d++) acc += qs[d] * kr[d];
        sc[j] = acc * scale;
        m = fmaxf(m, sc[j]);
    }
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < NT / IRIS_WAVE; w++) m = fmaxf(m, red[w]);
    __syncthreads();
    float s = 0.0f;
    for (int j = threadIdx.x; j < sk; j += NT) {
        const float e = expf(sc[j] - m);
        sc[j] = e;
        s += e;
    }
    const float inv = 1.0f / block_sum<NT / IRIS_WAVE>(s, red);
    for (int d = threadIdx.x; d < hd; d += NT) {
        float acc = 0.0f;
        for (int j = 0; j < sk; j++) acc += sc[j] * v[base + (size_t)j * ld + d];
        o[qbase + (size_t)qi * ld + d] = acc * inv;
    }
}

}  // namespace

extern "C" {

int iris_hip_split_rows(uint16_t *dst, const float *src, int rows, int cols, int ld_src, int K_pad, int nseg,
                        int lo_mask) {
    if (rows <= 0 || K_pad <= 0) return 0;
    if (K_pad < cols || nseg < 1 || nseg > 3) return iris_set_error("split_rows: cols %d K_pad %d", cols, K_pad);
    const size_t n = (size_t)rows * K_pad;
    IRIS_LAUNCH(split_rows_kernel, dim3(grid_for(n)), dim3(NT), 0, iris_stream(), dst, src, rows, cols, ld_src,
                       K_pad, nseg, lo_mask);
    return iris_launch_check("split_rows_kernel");
}

int iris_hip_split_transpose(uint16_t *dst, const float *src, int K, int N, int K_pad, int nseg, int lo_mask) {
    if (K <= 0 || N <= 0) return 0;
    if (K_pad < K || nseg < 1 || nseg > 3) return iris_set_error("split_transpose: K %d K_pad %d", K, K_pad);
    IRIS_LAUNCH(split_transpose_kernel, dim3((N + 31) / 32, (K_pad + 31) / 32), dim3(NT), 0, iris_stream(),
                       dst, src, K, N, K_pad, nseg, lo_mask);
    return iris_launch_check("split_transpose_kernel");
}

int iris_hip_pad_bf16(uint16_t *dst, const uint16_t *src, int rows, int cols, int K_pad, int nseg) {
    if (rows <= 0 || K_pad <= 0) return 0;
    if (K_pad < cols || nseg < 1 || nseg > 3) return iris_set_error("pad_bf16: cols %d K_pad %d", cols, K_pad);
    const size_t n = (size_t)rows * K_pad;
    IRIS_LAUNCH(pad_bf16_kernel, dim3(grid_for(n)), dim3(NT), 0, iris_stream(), dst, src, rows, cols, K_pad,
                       nseg);
    return iris_launch_check("pad_bf16_kernel");
}

int iris_hip_im2col_split(uint16_t *dst, const float *in, int C, int H, int W, int kH, int kW, int stride, int pad,
                          int outW, int pix0, int npix, int K_pad, int nseg, int lo_mask) {
    if (npix <= 0) return 0;
    if (K_pad < C * kH * kW || nseg < 1 || nseg > 3) return iris_set_error("im2col: K_pad %d", K_pad);
    const size_t n = (size_t)npix * K_pad;
    IRIS_LAUNCH(im2col_split_kernel, dim3(grid_for(n)), dim3(NT), 0, iris_stream(), dst, in, C, H, W, kH, kW,
                       stride, pad, outW, pix0, npix, C * kH * kW, K_pad, nseg, lo_mask);
    return iris_launch_check("im2col_split_kernel");
}

int iris_hip_rms_rows(float *out, const float *x, const float *w, int rows, int cols, float eps) {
    if (rows <= 0 || cols <= 0) return 0;
    IRIS_LAUNCH(rms_rows_kernel, dim3((rows + NT / IRIS_WAVE - 1) / (NT / IRIS_WAVE)), dim3(NT), 0,
                       iris_stream(), out, x, w, rows, cols, eps);
    return iris_launch_check("rms_rows_kernel");
}

int iris_hip_elementwise(int op, float *out, const float *a, const float *b, float s, size_t n) {
    if (!n) return 0;
    IRIS_LAUNCH(ew_kernel, dim3(grid_for(n)), dim3(NT), 0, iris_stream(), op, out, a, b, s, n);
    return iris_launch_check("ew_kernel");
}

int iris_hip_add_row_bias(float *out, const float *bias, int rows, int cols, int ld) {
    const size_t n = (size_t)rows * cols;
    if (!n) return 0;
    IRIS_LAUNCH(add_row_bias_kernel, dim3(grid_for(n)), dim3(NT), 0, iris_stream(), out, bias, rows, cols, ld);
    return iris_launch_check("add_row_bias_kernel");
}

int iris_hip_softmax_rows(float *x, int rows, int cols) {
    if (rows <= 0 || cols <= 0) return 0;
    IRIS_LAUNCH(softmax_rows_kernel, dim3((rows + NT / IRIS_WAVE - 1) / (NT / IRIS_WAVE)), dim3(NT), 0, iris_stream(), x,
                       rows, cols);
    return iris_launch_check("softmax_rows_kernel");
}

int iris_hip_group_norm(float *out, const float *x, const float *gamma, const float *beta, int batch, int channels,
                        int spatial, int groups, float eps) {
    if (batch <= 0 || groups <= 0 || channels % groups) return iris_set_error("group_norm: channels %% groups");
    IRIS_LAUNCH(group_norm_kernel, dim3(batch * groups), dim3(NT), 0, iris_stream(), out, x, gamma, beta,
                       channels, spatial, groups, eps);
    return iris_launch_check("group_norm_kernel");
}

int iris_hip_batch_norm(float *out, const float *x, const float *mean, const float *var, const float *gamma,
                        const float *beta, int batch, int channels, int spatial, float eps) {
    const size_t n = (size_t)batch * channels * spatial;
    if (!n) return 0;
    IRIS_LAUNCH(batch_norm_kernel, dim3(grid_for(n)), dim3(NT), 0, iris_stream(), out, x, mean, var, gamma,
                       beta, channels, spatial, n, eps);
    return iris_launch_check("batch_norm_kernel");
}

int iris_hip_upsample_nearest(float *out, const float *in, int planes, int H, int W, int sh, int sw) {
    const size_t n = (size_t)planes * H * sh * W * sw;
    if (!n) return 0;
    IRIS_LAUNCH(upsample_kernel, dim3(grid_for(n)), dim3(NT), 0, iris_stream(), out, in, H, W, sh, sw, n);
    return iris_launch_check("upsample_kernel");
}

int iris_hip_space_to_depth(float *out, const float *in, int batch, int C, int H, int W, int p, int inverse) {
    const size_t n = (size_t)batch * C * H * W;
    if (!n) return 0;
    if (p <= 0 || H % p || W % p) return iris_set_error("space_to_depth: %dx%d not divisible by %d", H, W, p);
    IRIS_LAUNCH(space_to_depth_kernel, dim3(grid_for(n)), dim3(NT), 0, iris_stream(), out, in, C, H, W, p,
                       inverse, n);
    return iris_launch_check("space_to_depth_kernel");
}

int iris_hip_attention_f32(float *o, const float *q, const float *k, const float *v, int batch, int heads, int sq,
                           int sk, int hd, float scale, long long q_sb, long long q_sh, long long k_sb,
                           long long k_sh, int ld) {
    if (batch <= 0 || heads <= 0 || sq <= 0 || sk <= 0) return 0;
    if (hd <= 0 || hd > 512 || sk > ATT_MAXK) return iris_set_error("attention_f32: head %d keys %d", hd, sk);
    const size_t smem = (size_t)(sk + hd) * sizeof(float);
    static bool attr = false;
    if (!attr) {
        if (iris_check(hipFuncSetAttribute((const void *)attention_f32_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)((ATT_MAXK + 512) * sizeof(float))),
                       "attention_f32 smem attribute"))
            return -1;
        attr = true;
    }
    IRIS_LAUNCH(attention_f32_kernel, dim3(sq, heads, batch), dim3(NT), smem, iris_stream(), o, q, k, v, sk, hd,
                       scale, q_sb, q_sh, k_sb, k_sh, ld);
    return iris_launch_check("attention_f32_kernel");
}

}  // extern "C"
