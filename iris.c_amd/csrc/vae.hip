/*
 * vae.hip - the VAE decoder's HBM-bound kernels for gfx950, NHWC layout.
 *
 * The decoder (iris_vae_decode, iris_vae.c:835-998) keeps activations
 * channels-last on the device: one pixel's channels are contiguous, so a
 * 3x3 convolution is an implicit GEMM with pixels as rows (iris_hip_conv3x3,
 * gemm.hip) and every kernel here streams whole 16- or 32-byte channel
 * chunks. Replaced reference pieces:
 *   - GroupNorm (iris_group_norm, iris_kernels.c:542-582) + swish
 *     (swish_inplace, iris_vae.c:195): a statistics pass that writes per-block
 *     float64 channel sums, a per-group finalize, and an apply pass that folds
 *     gamma, beta, mean and 1/std into one scale and shift per channel and
 *     writes the bf16 conv input;
 *   - denormalize + unpatchify + post_quant_conv (iris_vae.c:860-897): one
 *     kernel from the NCHW latent to the conv_in input;
 *   - the mid-block attention's softmax and V transpose (iris_vae.c:260-357);
 *   - conv_out 128 -> 3 and the [-1,1] -> uint8 conversion
 *     (iris_vae.c:968-994): one direct kernel.
 */
#include "iris_internal.h"

namespace {

constexpr int NT = 256;

__device__ __forceinline__ void load8(const float *p, float v[8]) {
    const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void load8(const uint16_t *p, float v[8]) {
    const uint4 a = *(const uint4 *)p;
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        v[2 * j] = __uint_as_float(w[j] << 16);
        v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
}
__device__ __forceinline__ uint4 pack8(const float v[8]) {
    uint4 o;
    o.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
    o.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
    o.z = (uint32_t)f2bf(v[4]) | ((uint32_t)f2bf(v[5]) << 16);
    o.w = (uint32_t)f2bf(v[6]) | ((uint32_t)f2bf(v[7]) << 16);
    return o;
}

/* Per-block group sums of x and x^2 over pixels [b*ppb, (b+1)*ppb):
 * part[(b * G + g) * 2 + {0, 1}], float64. Thread t reads channel chunk
 * t % (C/8) of every (256 / (C/8))-th pixel; the block then sums the threads
 * of each chunk, then the channels of each group, in a fixed order, so the
 * result does not depend on timing. */
template <typename T>
__global__ __launch_bounds__(NT) void gn_stats_kernel(const T *x, int pixels, int C, int G, int ppb, double *part) {
    __shared__ double ls[NT][8], lq[NT][8];
    __shared__ double cs[512], cq[512];
    const int cpr = C >> 3, tid = threadIdx.x, ci = tid % cpr, rows = NT / cpr;
    const int p0 = blockIdx.x * ppb, p1 = min(pixels, p0 + ppb);
    double s[8], q[8];
#pragma unroll
    for (int j = 0; j < 8; j++) s[j] = q[j] = 0.0;
#pragma unroll 4
    for (int p = p0 + tid / cpr; p < p1; p += rows) {
        float v[8];
        load8(x + (size_t)p * C + ci * 8, v);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            s[j] += (double)v[j];
            q[j] += (double)v[j] * (double)v[j];
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        ls[tid][j] = s[j];
        lq[tid][j] = q[j];
    }
    __syncthreads();
    for (int c = tid; c < C; c += NT) {
        double a = 0.0, b = 0.0;
        for (int r = 0; r < rows; r++) {
            a += ls[r * cpr + (c >> 3)][c & 7];
            b += lq[r * cpr + (c >> 3)][c & 7];
        }
        cs[c] = a;
        cq[c] = b;
    }
    __syncthreads();
    const int cpg = C / G;
    for (int g = tid; g < G; g += NT) {
        double a = 0.0, b = 0.0;
        for (int c = g * cpg; c < (g + 1) * cpg; c++) {
            a += cs[c];
            b += cq[c];
        }
        part[((size_t)blockIdx.x * G + g) * 2] = a;
        part[((size_t)blockIdx.x * G + g) * 2 + 1] = b;
    }
}

/* One block per group: mean and variance of the group from the per-block
 * partial sums (float64, fixed order), then per channel y = x * a + b with
 * a = gamma / sqrt(var + eps), b = beta - mean * a; ab[c] = a, ab[C + c] = b. */
__global__ __launch_bounds__(NT) void gn_finalize_kernel(const double *part, int nblk, int C, int G,
                                                         const float *gamma, const float *beta, float eps,
                                                         double count, float *ab) {
    __shared__ double rs[NT], rq[NT];
    const int g = blockIdx.x, cpg = C / G, tid = threadIdx.x;
    double s = 0.0, q = 0.0;
    for (int e = tid; e < nblk; e += NT) {
        s += part[((size_t)e * G + g) * 2];
        q += part[((size_t)e * G + g) * 2 + 1];
    }
    rs[tid] = s;
    rq[tid] = q;
    __syncthreads();
    for (int h = NT / 2; h > 0; h >>= 1) {
        if (tid < h) {
            rs[tid] += rs[tid + h];
            rq[tid] += rq[tid + h];
        }
        __syncthreads();
    }
    const double mean = rs[0] / count;
    double var = rq[0] / count - mean * mean;
    if (var < 0.0) var = 0.0;
    const float inv = 1.0f / sqrtf((float)var + eps);
    for (int t = tid; t < cpg; t += NT) {
        const int c = g * cpg + t;
        const float a = inv * gamma[c];
        ab[c] = a;
        ab[C + c] = beta[c] - (float)mean * a;
    }
}

/* y = act(x * ab[c] + ab[C + c]) in bf16, act = swish or identity; raw (if
 * not NULL) receives x itself in bf16 (the input of a 1x1 skip convolution). */
template <typename T>
__global__ __launch_bounds__(NT) void gn_apply_kernel(const T *x, const float *ab, int C, size_t n8, int swish,
                                                      uint16_t *y, uint16_t *raw) {
    const int cpr = C >> 3;
    for (size_t i = (size_t)blockIdx.x * NT + threadIdx.x; i < n8; i += (size_t)gridDim.x * NT) {
        const int c0 = (int)(i % cpr) * 8;
        float v[8];
        load8(x + i * 8, v);
        if (raw) *(uint4 *)(raw + i * 8) = pack8(v);
        const float4 a0 = *(const float4 *)(ab + c0), a1 = *(const float4 *)(ab + c0 + 4);
        const float4 b0 = *(const float4 *)(ab + C + c0), b1 = *(const float4 *)(ab + C + c0 + 4);
        const float a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const float b[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float t = v[j] * a[j] + b[j];
            v[j] = swish ? silu_f(t) : t;
        }
        *(uint4 *)(y + i * 8) = pack8(v);
    }
}

/* Latent [4z][h][w] (NCHW, f32) -> conv_in input [2h][2w][64] bf16:
 * per latent channel x * sc + sh (Flux: sc = sqrt(var + eps), sh = mean) or
 * x / sc + sh (Z-Image: sc = scaling factor, sh = shift); unpatchify 2x2
 * (channel c * 4 + 2 * (oy & 1) + (ox & 1) at (oy / 2, ox / 2) becomes
 * channel c at (oy, ox)); then the 1x1 post_quant_conv when pqw is not NULL;
 * channels z..63 are zero (conv_in's weights are padded to match). */
__global__ __launch_bounds__(NT) void vae_front_kernel(const float *lat, int z, int h, int w, const float *sc,
                                                       const float *sh, int divide, const float *pqw,
                                                       const float *pqb, uint16_t *out) {
    __shared__ float wsh[32 * 32];
    if (pqw)
        for (int i = threadIdx.x; i < z * z; i += NT) wsh[i] = pqw[i];
    __syncthreads();
    const int W2 = 2 * w, npix = 4 * h * w;
    const int p = blockIdx.x * NT + threadIdx.x;
    if (p >= npix) return;
    const int oy = p / W2, ox = p % W2;
    float v[32], o[64];
    for (int c = 0; c < z; c++) {
        const int ic = c * 4 + (oy & 1) * 2 + (ox & 1);
        const float x = lat[((size_t)ic * h + (oy >> 1)) * w + (ox >> 1)];
        v[c] = divide ? x / sc[ic] + sh[ic] : x * sc[ic] + sh[ic];
    }
    for (int j = 0; j < 64; j++) o[j] = 0.0f;
    if (pqw) {
        for (int j = 0; j < z; j++) {
            float a = pqb ? pqb[j] : 0.0f;
            for (int c = 0; c < z; c++) a += wsh[j * z + c] * v[c];
            o[j] = a;
        }
    } else {
        for (int j = 0; j < z; j++) o[j] = v[j];
    }
    uint4 *dst = (uint4 *)(out + (size_t)p * 64);
#pragma unroll
    for (int k = 0; k < 8; k++) dst[k] = pack8(o + 8 * k);
}

/* Encoder input: image [3][H][W] f32 (NCHW) -> bf16 [H][W][64], channels
 * 3..63 zero (conv_in's weights are padded to match). */
__global__ __launch_bounds__(NT) void vae_img_in_kernel(const float *img, int npix, uint16_t *out) {
    const int p = blockIdx.x * NT + threadIdx.x;
    if (p >= npix) return;
    float o[64];
#pragma unroll
    for (int j = 0; j < 64; j++) o[j] = 0.0f;
    o[0] = img[p];
    o[1] = img[(size_t)npix + p];
    o[2] = img[2 * (size_t)npix + p];
    uint4 *dst = (uint4 *)(out + (size_t)p * 64);
#pragma unroll
    for (int k = 0; k < 8; k++) dst[k] = pack8(o + 8 * k);
}

/* Encoder output (iris_vae.c:440-482): moments [h][w][2z] f32 (NHWC) ->
 * optional 1x1 quant_conv (qw [2z][2z]) -> the mean (first z channels) ->
 * patchify 2x2 (channel c at (y, x) becomes channel c * 4 + 2 (y & 1) + (x & 1)
 * at (y / 2, x / 2)) -> per latent channel (x - sh) * sc (Z-Image: scaling,
 * shift; Flux: 1 / sqrt(var + eps), mean) -> latent [4z][h/2][w/2] f32. */
__global__ __launch_bounds__(NT) void vae_enc_out_kernel(const float *mom, int z, int h, int w, const float *qw,
                                                         const float *qb, const float *sc, const float *sh,
                                                         float *lat) {
    const int p = blockIdx.x * NT + threadIdx.x;
    if (p >= h * w) return;
    const int y = p / w, x = p % w, z2 = 2 * z;
    const float *m = mom + (size_t)p * z2;
    const int lh = h / 2, lw = w / 2;
    if ((y >> 1) >= lh || (x >> 1) >= lw) return;
    for (int c = 0; c < z; c++) {
        float v;
        if (qw) {
            v = qb ? qb[c] : 0.0f;
            for (int k = 0; k < z2; k++) v += qw[c * z2 + k] * m[k];
        } else {
            v = m[c];
        }
        const int lc = c * 4 + (y & 1) * 2 + (x & 1);
        lat[((size_t)lc * lh + (y >> 1)) * lw + (x >> 1)] = (v - sh[lc]) * sc[lc];
    }
}

/* Row softmax from f32 scores to bf16 probabilities, one block per row:
 * pass 1 keeps a running (max, sum of exp) per thread and merges them,
 * pass 2 writes exp(x - max) / sum; columns cols..cols_pad-1 get zero. */
__global__ __launch_bounds__(NT) void softmax_bf16_kernel(const float *s, int ld_s, int cols, uint16_t *p, int ld_p,
                                                          int cols_pad) {
    __shared__ float rm[NT / IRIS_WAVE], rl[NT / IRIS_WAVE];
    const float *row = s + (size_t)blockIdx.x * ld_s;
    uint16_t *prow = p + (size_t)blockIdx.x * ld_p;
    float m = -INFINITY, l = 0.0f;
    for (int c = threadIdx.x * 4; c < cols; c += NT * 4) {
        const float4 x = *(const float4 *)(row + c);
        const float mx = fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w));
        const float nm = fmaxf(m, mx);
        l = l * __expf(m - nm) + __expf(x.x - nm) + __expf(x.y - nm) + __expf(x.z - nm) + __expf(x.w - nm);
        m = nm;
    }
    /* merge (m, l) pairs: wave, then block */
    for (int o = 32; o > 0; o >>= 1) {
        const float om = __shfl_xor(m, o), ol = __shfl_xor(l, o);
        const float nm = fmaxf(m, om);
        l = (m == -INFINITY ? 0.0f : l * __expf(m - nm)) + (om == -INFINITY ? 0.0f : ol * __expf(om - nm));
        m = nm;
    }
    const int wv = threadIdx.x / IRIS_WAVE;
    if ((threadIdx.x & (IRIS_WAVE - 1)) == 0) {
        rm[wv] = m;
        rl[wv] = l;
    }
    __syncthreads();
    float M = rm[0];
    for (int i = 1; i < NT / IRIS_WAVE; i++) M = fmaxf(M, rm[i]);
    float Lsum = 0.0f;
    for (int i = 0; i < NT / IRIS_WAVE; i++) Lsum += rm[i] == -INFINITY ? 0.0f : rl[i] * __expf(rm[i] - M);
    const float inv = 1.0f / Lsum;
    for (int c = threadIdx.x * 4; c < cols_pad; c += NT * 4) {
        uint2 o = make_uint2(0u, 0u);
        if (c < cols) {
            const float4 x = *(const float4 *)(row + c);
            o.x = (uint32_t)f2bf(__expf(x.x - M) * inv) | ((uint32_t)f2bf(__expf(x.y - M) * inv) << 16);
            o.y = (uint32_t)f2bf(__expf(x.z - M) * inv) | ((uint32_t)f2bf(__expf(x.w - M) * inv) << 16);
        }
        *(uint2 *)(prow + c) = o;
    }
}

/* dst[c][r] = src[r][c] for r < rows, 0 for rows <= r < rows_pad; 64x64
 * tiles through LDS (stride 65 keeps the transposed reads conflict-free). */
__global__ __launch_bounds__(NT) void transpose_bf16_kernel(const uint16_t *src, int ld_src, int rows, int cols,
                                                            uint16_t *dst, int ld_dst) {
    __shared__ uint16_t t[64][65];
    const int r0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
    for (int i = threadIdx.x; i < 64 * 64; i += NT) {
        const int r = i / 64, c = i % 64;
        t[r][c] = r0 + r < rows && c0 + c < cols ? src[(size_t)(r0 + r) * ld_src + c0 + c] : (uint16_t)0;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 64; i += NT) {
        const int c = i / 64, r = i % 64;
        if (c0 + c < cols) dst[(size_t)(c0 + c) * ld_dst + r0 + r] = t[r][c];
    }
}

/* conv_out (3x3, cin -> 3, zero padding) and the image conversion, one thread
 * per pixel: v = conv + bias; u8 = (uint8)(clamp(((v + 1) * 0.5) * 255, 0,
 * 255) + 0.5) in the reference's order of operations; f32 (if not NULL)
 * receives v as [3][H][W]. Weights wt[tap][cin][4] (4th lane zero) sit in
 * LDS and are read as one broadcast float4 per input channel. */
__global__ __launch_bounds__(NT) void conv_out_kernel(const uint16_t *g, int H, int W, int cin, const float *wt,
                                                      const float *bias, uint8_t *rgb, float *f32) {
    extern __shared__ float4 wl[];
    for (int i = threadIdx.x; i < 9 * cin; i += NT) wl[i] = ((const float4 *)wt)[i];
    __syncthreads();
    const int p = blockIdx.x * NT + threadIdx.x;
    if (p >= H * W) return;
    const int y = p / W, x = p % W;
    float a0 = bias[0], a1 = bias[1], a2 = bias[2];
    for (int tap = 0; tap < 9; tap++) {
        const int yy = y + tap / 3 - 1, xx = x + tap % 3 - 1;
        if ((unsigned)yy >= (unsigned)H || (unsigned)xx >= (unsigned)W) continue;
        const uint16_t *src = g + ((size_t)yy * W + xx) * cin;
        const float4 *wr = wl + tap * cin;
        for (int c = 0; c < cin; c += 8) {
            float v[8];
            load8(src + c, v);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float4 k = wr[c + j];
                a0 += v[j] * k.x;
                a1 += v[j] * k.y;
                a2 += v[j] * k.z;
            }
        }
    }
    const float o[3] = {a0, a1, a2};
#pragma unroll
    for (int ch = 0; ch < 3; ch++) {
        if (f32) f32[(size_t)ch * H * W + p] = o[ch];
        float val = (o[ch] + 1.0f) * 0.5f;
        val = val * 255.0f;
        if (val < 0) val = 0;
        if (val > 255) val = 255;
        rgb[(size_t)p * 3 + ch] = (uint8_t)(val + 0.5f);
    }
}

/* The same convolution over 16 x 16 output tiles: the tile's input pixels
 * and their one-pixel halo are staged in LDS 32 channels at a time (each
 * input row read once per tile instead of once per tap and neighbour), the
 * chunk's weights beside them; one thread per output pixel. The sums run
 * chunk by chunk, tap by tap within a chunk. Rows of 32 channels are padded
 * to 40 elements, so the 16 pixels of a half wave read 16 distinct 4-bank
 * groups. */
constexpr int CO_T = 16, CO_H = CO_T + 2, CO_C = 32, CO_STR = CO_C + 8;
__global__ __launch_bounds__(NT) void conv_out_tiled_kernel(const uint16_t *g, int H, int W, int cin, const float *wt,
                                                            const float *bias, uint8_t *rgb, float *f32) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[CO_H * CO_H * CO_STR];
    __shared__ float4 wl[9 * CO_C];
    const int tx = threadIdx.x & (CO_T - 1), ty = threadIdx.x / CO_T;
    const int x0 = blockIdx.x * CO_T, y0 = blockIdx.y * CO_T;
    float a0 = bias[0], a1 = bias[1], a2 = bias[2];
    for (int c0 = 0; c0 < cin; c0 += CO_C) {
        __syncthreads();   /* the previous chunk's reads are done */
        for (int i = threadIdx.x; i < CO_H * CO_H * (CO_C / 8); i += NT) {
            const int pix = i >> 2, part = i & 3;
            const int gy = y0 + pix / CO_H - 1, gx = x0 + pix % CO_H - 1;
            uint4 v = make_uint4(0, 0, 0, 0);
            if ((unsigned)gy < (unsigned)H && (unsigned)gx < (unsigned)W)
                v = *(const uint4 *)(g + ((size_t)gy * W + gx) * cin + c0 + part * 8);
            *(uint4 *)(xs + pix * CO_STR + part * 8) = v;
        }
        for (int i = threadIdx.x; i < 9 * CO_C; i += NT) wl[i] = ((const float4 *)wt)[(i / CO_C) * cin + c0 + i % CO_C];
        __syncthreads();
        for (int tap = 0; tap < 9; tap++) {
            const uint16_t *src = xs + ((ty + tap / 3) * CO_H + tx + tap % 3) * CO_STR;
            const float4 *wr = wl + tap * CO_C;
#pragma unroll
            for (int c = 0; c < CO_C; c += 8) {
                const u16x8 r = *(const u16x8 *)(src + c);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float v = bf2f(r[j]);
                    const float4 k = wr[c + j];
                    a0 += v * k.x;
                    a1 += v * k.y;
                    a2 += v * k.z;
                }
            }
        }
    }
    const int y = y0 + ty, x = x0 + tx;
    if (y >= H || x >= W) return;
    const int p = y * W + x;
    const float o[3] = {a0, a1, a2};
#pragma unroll
    for (int ch = 0; ch < 3; ch++) {
        if (f32) f32[(size_t)ch * H * W + p] = o[ch];
        float val = (o[ch] + 1.0f) * 0.5f;
        val = val * 255.0f;
        if (val < 0) val = 0;
        if (val > 255) val = 255;
        rgb[(size_t)p * 3 + ch] = (uint8_t)(val + 0.5f);
    }
}

unsigned blocks_for(size_t n) {
    const size_t b = (n + NT - 1) / NT;
    return (unsigned)(b < 65536 ? b : 65536);
}

}  // namespace

extern "C" int iris_hip_gn_stats(const void *x, int is_bf16, int pixels, int C, int groups, double *part, int nblk) {
    if (!x || !part || pixels <= 0 || nblk <= 0) return iris_set_error("gn_stats: bad arguments");
    if (C < 64 || C > 512 || (C & (C - 1))) return iris_set_error("gn_stats: C=%d (a power of two in 64..512)", C);
    if (groups <= 0 || C % groups) return iris_set_error("gn_stats: %d groups of %d channels", groups, C);
    if ((uintptr_t)x & 15) return iris_set_error("gn_stats: x must be 16-byte aligned");
    const int ppb = (pixels + nblk - 1) / nblk;
    const int used = (pixels + ppb - 1) / ppb;
    if (is_bf16)
        IRIS_LAUNCH(gn_stats_kernel<uint16_t>, dim3(used), dim3(NT), 0, iris_stream(), (const uint16_t *)x,
                           pixels, C, groups, ppb, part);
    else
        IRIS_LAUNCH(gn_stats_kernel<float>, dim3(used), dim3(NT), 0, iris_stream(), (const float *)x, pixels,
                           C, groups, ppb, part);
    if (iris_launch_check("gn_stats_kernel")) return -1;
    return used;
}

extern "C" int iris_hip_gn_finalize(const double *part, int nblk, int pixels, int C, int groups, const float *gamma,
                                    const float *beta, float eps, float *ab) {
    if (!part || !gamma || !beta || !ab || nblk <= 0 || groups <= 0 || C % groups)
        return iris_set_error("gn_finalize: bad arguments");
    const double count = (double)pixels * (C / groups);
    IRIS_LAUNCH(gn_finalize_kernel, dim3(groups), dim3(NT), 0, iris_stream(), part, nblk, C, groups, gamma,
                       beta, eps, count, ab);
    return iris_launch_check("gn_finalize_kernel");
}

extern "C" int iris_hip_gn_apply(const void *x, int is_bf16, const float *ab, int pixels, int C, int swish,
                                 uint16_t *y, uint16_t *raw) {
    if (!x || !ab || !y || pixels <= 0 || C % 8 || ((uintptr_t)x & 15) || ((uintptr_t)y & 15) ||
        ((uintptr_t)raw & 15) || ((uintptr_t)ab & 15))
        return iris_set_error("gn_apply: bad arguments");
    const size_t n8 = (size_t)pixels * C / 8;
    if (is_bf16)
        IRIS_LAUNCH(gn_apply_kernel<uint16_t>, dim3(blocks_for(n8)), dim3(NT), 0, iris_stream(),
                           (const uint16_t *)x, ab, C, n8, swish, y, raw);
    else
        IRIS_LAUNCH(gn_apply_kernel<float>, dim3(blocks_for(n8)), dim3(NT), 0, iris_stream(), (const float *)x,
                           ab, C, n8, swish, y, raw);
    return iris_launch_check("gn_apply_kernel");
}

extern "C" int iris_hip_vae_front(uint16_t *out, const float *lat, int z, int h, int w, const float *sc,
                                  const float *sh, int divide, const float *pqw, const float *pqb) {
    if (!out || !lat || !sc || !sh || z <= 0 || z > 32 || h <= 0 || w <= 0 || ((uintptr_t)out & 15))
        return iris_set_error("vae_front: bad arguments (z=%d, %dx%d)", z, h, w);
    const int npix = 4 * h * w;
    IRIS_LAUNCH(vae_front_kernel, dim3((npix + NT - 1) / NT), dim3(NT), 0, iris_stream(), lat, z, h, w, sc, sh,
                       divide, pqw, pqb, out);
    return iris_launch_check("vae_front_kernel");
}

extern "C" int iris_hip_softmax_bf16(uint16_t *p, int ld_p, int cols_pad, const float *s, int ld_s, int rows,
                                     int cols) {
    if (!p || !s || rows <= 0 || cols <= 0 || cols % 4 || ld_s % 4 || ld_p % 4 || cols_pad % 4 || cols_pad < cols ||
        ld_s < cols || ld_p < cols_pad || ((uintptr_t)s & 15) || ((uintptr_t)p & 7))
        return iris_set_error("softmax_bf16: bad shape (rows %d cols %d pad %d ld %d/%d)", rows, cols, cols_pad, ld_s,
                              ld_p);
    IRIS_LAUNCH(softmax_bf16_kernel, dim3(rows), dim3(NT), 0, iris_stream(), s, ld_s, cols, p, ld_p, cols_pad);
    return iris_launch_check("softmax_bf16_kernel");
}

extern "C" int iris_hip_transpose_bf16(uint16_t *dst, int ld_dst, int rows_pad, const uint16_t *src, int ld_src,
                                       int rows, int cols) {
    if (!dst || !src || rows <= 0 || cols <= 0 || rows_pad < rows || rows_pad % 64 || ld_dst < rows_pad ||
        ld_src < cols)
        return iris_set_error("transpose_bf16: bad shape");
    IRIS_LAUNCH(transpose_bf16_kernel, dim3(rows_pad / 64, (cols + 63) / 64), dim3(NT), 0, iris_stream(), src,
                       ld_src, rows, cols, dst, ld_dst);
    return iris_launch_check("transpose_bf16_kernel");
}

extern "C" int iris_hip_vae_conv_out(uint8_t *rgb, float *f32, const uint16_t *g, int H, int W, int cin,
                                     const float *wt, const float *bias) {
    if (!rgb || !g || !wt || !bias || H <= 0 || W <= 0 || H > 32768 || W > 32768 || cin <= 0 || cin > 256 || cin % 8 ||
        ((uintptr_t)g & 15) ||
        ((uintptr_t)wt & 15))
        return iris_set_error("vae_conv_out: bad arguments");
    if (cin % CO_C == 0) {
        IRIS_LAUNCH(conv_out_tiled_kernel, dim3((W + CO_T - 1) / CO_T, (H + CO_T - 1) / CO_T), dim3(NT), 0,
                    iris_stream(), g, H, W, cin, wt, bias, rgb, f32);
        return iris_launch_check("conv_out_tiled_kernel");
    }
    const int npix = H * W;
    IRIS_LAUNCH(conv_out_kernel, dim3((npix + NT - 1) / NT), dim3(NT), 9 * cin * sizeof(float4), iris_stream(),
                       g, H, W, cin, wt, bias, rgb, f32);
    return iris_launch_check("conv_out_kernel");
}

extern "C" int iris_hip_vae_img_in(uint16_t *out, const float *img, int H, int W) {
    if (!out || !img || H <= 0 || W <= 0 || ((uintptr_t)out & 15)) return iris_set_error("vae_img_in: bad arguments");
    const int npix = H * W;
    IRIS_LAUNCH(vae_img_in_kernel, dim3((npix + NT - 1) / NT), dim3(NT), 0, iris_stream(), img, npix, out);
    return iris_launch_check("vae_img_in_kernel");
}

extern "C" int iris_hip_vae_enc_out(float *lat, const float *mom, int z, int h, int w, const float *qw,
                                    const float *qb, const float *sc, const float *sh) {
    if (!lat || !mom || !sc || !sh || z <= 0 || h < 2 || w < 2) return iris_set_error("vae_enc_out: bad arguments");
    IRIS_LAUNCH(vae_enc_out_kernel, dim3((h * w + NT - 1) / NT), dim3(NT), 0, iris_stream(), mom, z, h, w, qw,
                       qb, sc, sh, lat);
    return iris_launch_check("vae_enc_out_kernel");
}
