/*
 * elementwise.hip - HBM-bound kernels of the denoiser step on gfx950.
 *
 *   rownorm        apply_adaln (iris_transformer_flux.c:1391-1460), the final
 *                  layer's LayerNorm (:4280-4285), Z-Image RMSNorm / final
 *                  LayerNorm (iris_transformer_zimage.c:657-668, :1590-1606)
 *   rms_gated_add  Z-Image x += gate * RMSNorm(y) (:818-836)
 *   qk_prepare     apply_qk_norm + apply_rope_2d (:1464-1518, :1026-1048),
 *                  zi_qk_norm + zi_apply_rope (zimage :620-682), and the
 *                  transposed V layout the attention kernel reads; the K
 *                  and V half alone for attention calls that normalise Q in
 *                  their prologue
 *   gemv           timestep MLP and modulation (:1366-1379, :4059-4069)
 *   layout         NCHW -> tokens (:3986-3993), patchify (zimage :1634-1684),
 *                  f32 <-> bf16, Euler update (iris_sample.c:359, :472-474)
 * One block per row for the normalisations, one wave per row for the other
 * row kernels; float4 / 16-byte accesses throughout.
 */
#include "iris_internal.h"

namespace {

constexpr int NT = 256;

/* One block of 256 threads per row: thread t owns float4 columns t, t + 256,
 * ... (V of them); each reduction is a wave shuffle plus a 4-entry LDS sum.
 * A wave per row leaves each wave a long chain (load, two reductions, store)
 * over 12 KB; spreading the row over four waves shortens it and keeps more
 * rows' loads in flight (5.5 TB/s against 4.8 for wave-per-row at
 * 4608 x 3072 f32 -> bf16). */
template <int V, int MODE>
__global__ __launch_bounds__(NT) void rownorm_kernel(const iris_norm_args_t a) {
    __shared__ float red[2][NT / IRIS_WAVE];
    const int row = blockIdx.x, t = threadIdx.x, wv = t >> 6, lane = t & 63;
    const float *x = a.x + (size_t)row * a.ldx;
    const int nv = a.cols >> 2;
    float4 v[V];
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = t + i * NT;
        v[i] = c < nv ? ld_stream((const float4 *)x + c) : make_float4(0, 0, 0, 0);
    }
    const bool use_b = (a.period ? row % a.period : row) >= a.split;
    const float *shift = use_b ? a.shiftB : a.shiftA;
    const float *scale = use_b ? a.scaleB : a.scaleA;
    const float *w = use_b ? a.wB : a.wA;
    auto block_sum = [&](float q, int k) {
        q = wave_sum(q);
        if (lane == 0) red[k][wv] = q;
        __syncthreads();
        return (red[k][0] + red[k][1]) + (red[k][2] + red[k][3]);
    };
    float mean = 0.0f, inv;
    if (MODE == IRIS_NORM_RMS) {
        float q = 0.0f;
#pragma unroll
        for (int i = 0; i < V; i++) q += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
        inv = 1.0f / sqrtf(block_sum(q, 0) / a.cols + a.eps);
    } else {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < V; i++) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
        mean = block_sum(s, 0) / a.cols;
        float q = 0.0f;
#pragma unroll
        for (int i = 0; i < V; i++) {
            const int c = t + i * NT;
            if (c < nv) {
                float d0 = v[i].x - mean, d1 = v[i].y - mean, d2 = v[i].z - mean, d3 = v[i].w - mean;
                q += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
            }
        }
        inv = 1.0f / sqrtf(block_sum(q, 1) / a.cols + a.eps);
    }
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = t + i * NT;
        if (c >= nv) continue;
        float e[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        float y[4];
        float4 sc4 = make_float4(0, 0, 0, 0), sh4 = make_float4(0, 0, 0, 0), w4 = make_float4(1, 1, 1, 1);
        if (MODE == IRIS_NORM_LN_MOD) {
            sc4 = ((const float4 *)scale)[c];
            sh4 = ((const float4 *)shift)[c];
        } else {
            if (scale) sc4 = ((const float4 *)scale)[c];
            if (MODE == IRIS_NORM_RMS) w4 = ((const float4 *)w)[c];
        }
        const float sc[4] = {sc4.x, sc4.y, sc4.z, sc4.w}, sh[4] = {sh4.x, sh4.y, sh4.z, sh4.w};
        const float ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (MODE == IRIS_NORM_LN_MOD) {
                const float n = (e[j] - mean) * inv;
                y[j] = (1.0f + sc[j]) * n + sh[j];
            } else if (MODE == IRIS_NORM_LN_SCALE) {
                y[j] = (e[j] - mean) * inv * sc[j];
            } else {
                float tt = e[j] * inv * ww[j];
                if (scale) tt *= sc[j];
                y[j] = tt;
            }
        }
        if (a.out_bf16) {
            u16x4 o = {f2bf_hw(y[0]), f2bf_hw(y[1]), f2bf_hw(y[2]), f2bf_hw(y[3])};
            *(u16x4 *)((uint16_t *)a.out + (size_t)row * a.ldo + 4 * c) = o;
        } else {
            *(float4 *)((float *)a.out + (size_t)row * a.ldo + 4 * c) = make_float4(y[0], y[1], y[2], y[3]);
        }
    }
}

/* x += g * RMSNorm(y) * w, one block of 256 threads per row (as rownorm). */
template <int V>
__global__ __launch_bounds__(NT) void rms_gated_add_kernel(float *x, const float *y, const float *w,
                                                           const float *gate, int rows, int cols, float eps,
                                                           int gate_tanh) {
    __shared__ float red[NT / IRIS_WAVE];
    const int row = blockIdx.x, t = threadIdx.x, wv = t >> 6, lane = t & 63;
    const int nv = cols >> 2;
    const float *yr = y + (size_t)row * cols;
    float *xr = x + (size_t)row * cols;
    float4 v[V];
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = t + i * NT;
        v[i] = c < nv ? ld_stream((const float4 *)yr + c) : make_float4(0, 0, 0, 0);
        q += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
    }
    q = wave_sum(q);
    if (lane == 0) red[wv] = q;
    __syncthreads();
    const float inv = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / cols + eps);
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = t + i * NT;
        if (c >= nv) continue;
        float4 xo = ld_stream((const float4 *)xr + c);
        const float4 w4 = ((const float4 *)w)[c];
        float4 g4 = make_float4(1, 1, 1, 1);
        if (gate) g4 = ((const float4 *)gate)[c];
        const float e[4] = {v[i].x, v[i].y, v[i].z, v[i].w}, ww[4] = {w4.x, w4.y, w4.z, w4.w};
        const float gg[4] = {g4.x, g4.y, g4.z, g4.w};
        float *xp = &xo.x;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float g = gate ? (gate_tanh ? tanhf(gg[j]) : gg[j]) : 1.0f;
            xp[j] += g * (e[j] * inv * ww[j]);
        }
        ((float4 *)xr)[c] = xo;
    }
}

/* One wave per row: 16 lanes per head, lane owns dims d0..d0+7 (four rotation
 * pairs); a 16-byte load covers 4 heads per wave, the head's sum of squares is
 * a 16-lane shuffle reduction. The row's table values are loaded once for all
 * its heads. KONLY: K alone (Q is normalised in the attention prologue). */
template <bool KONLY>
__device__ __forceinline__ void qk_norm_rope_rows(const iris_qkprep_args_t &a, int blk) {
    const int row = blk * (NT / IRIS_WAVE) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= a.rows) return;
    const int prow = a.period ? row % a.period : row;
    const bool use_b = prow >= a.split;
    const int hl = lane & 15, hq = lane >> 4, d0 = hl * 8;
    float c[8], sn[8];
    if (a.cos_t) {
        const float4 c0 = *(const float4 *)(a.cos_t + (size_t)prow * 128 + d0);
        const float4 c1 = *(const float4 *)(a.cos_t + (size_t)prow * 128 + d0 + 4);
        const float4 s0 = *(const float4 *)(a.sin_t + (size_t)prow * 128 + d0);
        const float4 s1 = *(const float4 *)(a.sin_t + (size_t)prow * 128 + d0 + 4);
        c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w; c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
        sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w; sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) { c[j] = 1.0f; sn[j] = 0.0f; }
    }
#pragma unroll
    for (int which = KONLY ? 1 : 0; which < 2; which++) {
        if (which && a.kcos_t) {   /* K-side tables (reference-key band control) */
            const float4 c0 = *(const float4 *)(a.kcos_t + (size_t)prow * 128 + d0);
            const float4 c1 = *(const float4 *)(a.kcos_t + (size_t)prow * 128 + d0 + 4);
            const float4 s0 = *(const float4 *)(a.ksin_t + (size_t)prow * 128 + d0);
            const float4 s1 = *(const float4 *)(a.ksin_t + (size_t)prow * 128 + d0 + 4);
            c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w; c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
            sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w; sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
        }
        const float *wsel = which ? (use_b ? a.wkB : a.wkA) : (use_b ? a.wqB : a.wqA);
        const float4 w0 = *(const float4 *)(wsel + d0), w1 = *(const float4 *)(wsel + d0 + 4);
        const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        const int nh = which && a.kv_heads ? a.kv_heads : a.heads;
        const uint16_t *src = a.qkv + (size_t)row * a.ld_qkv + (which ? a.col_k : 0) + d0;
        uint16_t *dst = (which ? a.k_out : a.q_out) + (size_t)row * nh * 128 + d0;
        for (int hb = 0; hb < nh; hb += 4) {
            const int head = hb + hq;
            const bool on = head < nh;                        /* uniform per 16-lane group */
            u16x8 raw = {0, 0, 0, 0, 0, 0, 0, 0};
            if (on) raw = __builtin_nontemporal_load((const u16x8 *)(src + head * 128));
            float x[8];
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) { x[j] = bf2f(raw[j]); ss += x[j] * x[j]; }
            ss = row16_sum(ss);
            const float inv = 1.0f / sqrtf(ss / 128.0f + a.eps);
            u16x8 out;
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const float x0 = x[j] * inv * w[j], x1 = x[j + 1] * inv * w[j + 1];
                out[j] = f2bf(x0 * c[j] - x1 * sn[j]);
                out[j + 1] = f2bf(x1 * c[j] + x0 * sn[j]);
            }
            if (on) *(u16x8 *)(dst + head * 128) = out;
        }
    }
}

/* V [rows][128] (head slice of qkv) -> V^T [head][128][ld_vt], 64 rows per
 * block. LDS holds the tile as [d][row] in rows of 72 elements (16-byte
 * aligned); 8-row chunks are XOR-swizzled by (d / 8) mod 8 to spread the
 * two-row writes over the banks. Rows past the end are written as zeros. */
__device__ __forceinline__ void v_transpose_tile(const iris_qkprep_args_t &a, int tile, int head, uint16_t *t) {
    const int r0 = tile * 64, tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < 2; it++) {                       /* 32 row pairs x 16 chunks of 8 dims */
        const int item = tid + NT * it, p = item >> 4, ch = item & 15;
        const int ra = r0 + 2 * p;
        const uint16_t *src = a.qkv + (size_t)ra * a.ld_qkv + a.col_v + head * 128 + ch * 8;
        u16x8 va = {0, 0, 0, 0, 0, 0, 0, 0}, vb = {0, 0, 0, 0, 0, 0, 0, 0};
        if (ra < a.rows) va = __builtin_nontemporal_load((const u16x8 *)src);
        if (ra + 1 < a.rows) vb = __builtin_nontemporal_load((const u16x8 *)(src + a.ld_qkv));
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int d = ch * 8 + j;
            const int col = (2 * p) ^ (((d >> 3) & 7) << 3);
            *(uint32_t *)(&t[d * 72 + col]) = (uint32_t)va[j] | ((uint32_t)vb[j] << 16);
        }
    }
    __syncthreads();
    uint16_t *dst = a.vt_out + (size_t)head * 128 * a.ld_vt + r0;
#pragma unroll
    for (int it = 0; it < 4; it++) {                       /* 128 d x 8 chunks of 8 rows */
        const int item = tid + NT * it, d = item >> 3, c8 = item & 7;
        const uint4 v = *(const uint4 *)(&t[d * 72 + ((c8 ^ ((d >> 3) & 7)) << 3)]);
        *(uint4 *)(dst + (size_t)d * a.ld_vt + c8 * 8) = v;
    }
}

/* The K (and Q) normalisation and the V transpose in one launch: blocks
 * 0 .. vblocks - 1 transpose V tiles (vx tiles of 64 rows per head), the rest
 * normalise 4 rows each. The two passes are short and HBM-bound; one launch
 * runs them side by side instead of paying two ramps and two tails. */
template <bool KONLY>
__global__ __launch_bounds__(NT) void qkv_prep_kernel(const iris_qkprep_args_t a, int vblocks, int vx) {
    __shared__ __attribute__((aligned(16))) uint16_t t[128 * 72];
    const int b = blockIdx.x;
    if (b < vblocks) v_transpose_tile(a, b % vx, b / vx, t);
    else qk_norm_rope_rows<KONLY>(a, b - vblocks);
}

/* y[n] = W[n, :] . act(x) + bias[n]. One wave per row, or for K <= 256 half
 * a wave per row (lanes 32..63 take the next row); each lane takes 8
 * consecutive elements of every 512- (256-) wide chunk. XLDS (K <= 4096):
 * the block first writes act(x) to LDS once, so the SiLU of the input is not
 * recomputed for every row. */
constexpr int GEMV_XLDS = 4096;
template <bool XLDS>
__global__ __launch_bounds__(NT) void gemv_kernel(float *y, const uint16_t *W, const float *x, const float *bias,
                                                  int N, int K, int act_in) {
    __shared__ __attribute__((aligned(16))) float xl[XLDS ? GEMV_XLDS : 4];
    if constexpr (XLDS) {
        for (int k = threadIdx.x; k < K; k += NT) {
            float v = x[k];
            if (act_in == 1) v = v / (1.0f + __expf(-v));
            xl[k] = v;
        }
        __syncthreads();
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool half = K <= 256;
    const int gw = blockIdx.x * (NT / IRIS_WAVE) + wave;
    const int n = half ? 2 * gw + (lane >> 5) : gw;
    const int l = half ? lane & 31 : lane, step = half ? 256 : 512;
    float acc = 0.0f;
    if (n < N) {
        const uint16_t *w = W + (size_t)n * K;
        for (int k = l * 8; k < K; k += step) {
            const u16x8 wv = __builtin_nontemporal_load((const u16x8 *)(w + k));   /* weights: read once */
            float4 xa, xb;
            if constexpr (XLDS) {
                xa = *(const float4 *)(xl + k);
                xb = *(const float4 *)(xl + k + 4);
            } else {
                xa = *(const float4 *)(x + k);
                xb = *(const float4 *)(x + k + 4);
            }
            float xs[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float xv = xs[e];
                if (!XLDS && act_in == 1) xv = xv / (1.0f + __expf(-xv));
                acc += bf2f(wv[e]) * xv;
            }
        }
    }
    if (half) {
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    } else {
        acc = wave_sum(acc);
    }
    if (n < N && l == 0) y[n] = acc + (bias ? bias[n] : 0.0f);
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

/* x[r][c0 + j] = tanh(x[r][c0 + j]) for j < len: Z-Image's gate columns of
 * the step's modulation vectors, once per step instead of once per element
 * of every gated residual add. */
__global__ void tanh_cols_kernel(float *x, int rows, int ld, int c0, int len) {
    const size_t n = (size_t)rows * len;
    for (size_t i = blockIdx.x * (size_t)NT + threadIdx.x; i < n; i += (size_t)gridDim.x * NT) {
        float *p = x + (i / len) * ld + c0 + i % len;
        *p = tanhf(*p);
    }
}

/* Token embedding lookup (iris_qwen3.c:1080-1091): one block row per token,
 * 8 bf16 per thread per step; ids outside the table give a zero row. */
__global__ void embed_rows_kernel(float *out, const uint16_t *table, const int *ids, int rows, int cols, int vocab) {
    const int r = blockIdx.x;
    if (r >= rows) return;
    const int id = ids[r];
    float *o = out + (size_t)r * cols;
    const bool ok = id >= 0 && id < vocab;
    const uint16_t *t = table + (size_t)(ok ? id : 0) * cols;
    for (int c = threadIdx.x * 8; c < cols; c += NT * 8) {
        if (c + 8 <= cols) {
            u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
            if (ok) v = *(const u16x8 *)(t + c);
            ((float4 *)(o + c))[0] = make_float4(bf2f(v[0]), bf2f(v[1]), bf2f(v[2]), bf2f(v[3]));
            ((float4 *)(o + c))[1] = make_float4(bf2f(v[4]), bf2f(v[5]), bf2f(v[6]), bf2f(v[7]));
        } else {
            for (int j = c; j < cols; j++) o[j] = ok ? bf2f(t[j]) : 0.0f;
        }
    }
}

/* f32 block copy, one block row per row */
__global__ void copy_rows_kernel(float *dst, int ld_dst, const float *src, int ld_src, int rows, int cols) {
    const int r = blockIdx.x;
    if (r >= rows) return;
    for (int c = threadIdx.x; c < cols; c += NT) dst[(size_t)r * ld_dst + c] = src[(size_t)r * ld_src + c];
}

int grid1d(size_t n) {
    size_t b = (n + NT - 1) / NT;
    return (int)(b < 8192 ? (b ? b : 1) : 8192);
}



}  // namespace

extern "C" {

int iris_hip_rownorm(const iris_norm_args_t *a) {
    if (a->rows <= 0) return 0;
    /* float4 columns per thread of a 256-thread block */
    const int need = (a->cols / 4 + NT - 1) / NT;
    static const int vs[] = {1, 2, 3, 4, 6, 8, 12, 16};
    int v = 0;
    for (int c : vs)
        if (!v && c >= need) v = c;
    if (a->cols % 4 || a->cols <= 0 || !v) return iris_set_error("rownorm: cols=%d", a->cols);
    if (a->ldx % 4 || a->ldo % 4) return iris_set_error("rownorm: ld must be multiple of 4");
    if (a->mode < IRIS_NORM_LN_MOD || a->mode > IRIS_NORM_RMS) return iris_set_error("rownorm: mode %d", a->mode);
    /* a set that no row selects may be left NULL: it stands in for the other */
    iris_norm_args_t b = *a;
    const bool only_a = !b.period && b.split >= b.rows, only_b = !b.period && b.split <= 0;
    if (only_a) { b.shiftB = b.shiftA; b.scaleB = b.scaleA; b.wB = b.wA; }
    if (only_b) { b.shiftA = b.shiftB; b.scaleA = b.scaleB; b.wA = b.wB; }
    if (b.mode == IRIS_NORM_LN_MOD && (!b.scaleA || !b.shiftA || !b.scaleB || !b.shiftB))
        return iris_set_error("rownorm: LN_MOD needs scale and shift for the row sets in use");
    if (b.mode == IRIS_NORM_RMS && (!b.wA || !b.wB)) return iris_set_error("rownorm: RMS needs weights");
    if (b.mode == IRIS_NORM_LN_SCALE && (!b.scaleA || !b.scaleB)) return iris_set_error("rownorm: LN_SCALE needs scales");
    const dim3 grid(a->rows);
#define ROWNORM_CASE(VV)                                                                                          \
    case VV:                                                                                                      \
        if (a->mode == IRIS_NORM_LN_MOD)                                                                          \
            IRIS_LAUNCH((rownorm_kernel<VV, IRIS_NORM_LN_MOD>), grid, dim3(NT), 0, iris_stream(), b);      \
        else if (a->mode == IRIS_NORM_LN_SCALE)                                                                   \
            IRIS_LAUNCH((rownorm_kernel<VV, IRIS_NORM_LN_SCALE>), grid, dim3(NT), 0, iris_stream(), b);    \
        else                                                                                                      \
            IRIS_LAUNCH((rownorm_kernel<VV, IRIS_NORM_RMS>), grid, dim3(NT), 0, iris_stream(), b);         \
        break;
    switch (v) {
        ROWNORM_CASE(1) ROWNORM_CASE(2) ROWNORM_CASE(3) ROWNORM_CASE(4)
        ROWNORM_CASE(6) ROWNORM_CASE(8) ROWNORM_CASE(12) ROWNORM_CASE(16)
    }
#undef ROWNORM_CASE
    return iris_launch_check("rownorm_kernel");
}

int iris_hip_rms_gated_add(float *x, const float *y, const float *w, const float *gate, int rows, int cols,
                           float eps, int gate_tanh) {
    if (rows <= 0) return 0;
    const int need = (cols / 4 + NT - 1) / NT;
    if (cols % 4 || cols <= 0 || need > 16) return iris_set_error("rms_gated_add: cols=%d", cols);
    const dim3 grid(rows);
    switch (need) {
    case 1: IRIS_LAUNCH(rms_gated_add_kernel<1>, grid, dim3(NT), 0, iris_stream(), x, y, w, gate, rows, cols, eps, gate_tanh); break;
    case 2: IRIS_LAUNCH(rms_gated_add_kernel<2>, grid, dim3(NT), 0, iris_stream(), x, y, w, gate, rows, cols, eps, gate_tanh); break;
    case 3: IRIS_LAUNCH(rms_gated_add_kernel<3>, grid, dim3(NT), 0, iris_stream(), x, y, w, gate, rows, cols, eps, gate_tanh); break;
    case 4: IRIS_LAUNCH(rms_gated_add_kernel<4>, grid, dim3(NT), 0, iris_stream(), x, y, w, gate, rows, cols, eps, gate_tanh); break;
    default: IRIS_LAUNCH(rms_gated_add_kernel<16>, grid, dim3(NT), 0, iris_stream(), x, y, w, gate, rows, cols, eps, gate_tanh); break;
    }
    return iris_launch_check("rms_gated_add_kernel");
}

int iris_hip_qk_prepare(const iris_qkprep_args_t *a) {
    if (a->rows <= 0) return 0;
    if (a->ld_qkv % 8 || a->col_k % 8 || a->col_v % 8) return iris_set_error("qk_prepare: layout not 16-byte aligned");
    if (a->ld_vt < a->rows || a->ld_vt % 64) return iris_set_error("qk_prepare: ld_vt=%d", a->ld_vt);
    if (a->heads <= 0 || a->kv_heads < 0 || a->kv_heads > a->heads)
        return iris_set_error("qk_prepare: heads=%d kv_heads=%d", a->heads, a->kv_heads);
    if (((uintptr_t)a->qkv | (uintptr_t)a->q_out | (uintptr_t)a->k_out | (uintptr_t)a->vt_out) & 15)
        return iris_set_error("qk_prepare: buffers must be 16-byte aligned");
    const int kvh = a->kv_heads ? a->kv_heads : a->heads, vx = a->ld_vt / 64;
    const long long blocks = (long long)vx * kvh + (a->rows + NT / IRIS_WAVE - 1) / (NT / IRIS_WAVE);
    if (blocks >= (1LL << 31)) return iris_set_error("qk_prepare: too many rows");
    IRIS_LAUNCH(qkv_prep_kernel<false>, dim3((unsigned)blocks), dim3(NT), 0, iris_stream(), *a, vx * kvh, vx);
    return iris_launch_check("qkv_prep_kernel");
}

int iris_hip_kv_prepare(const iris_qkprep_args_t *a) {
    if (a->rows <= 0) return 0;
    if (a->ld_qkv % 8 || a->col_k % 8 || a->col_v % 8) return iris_set_error("kv_prepare: layout not 16-byte aligned");
    if (a->ld_vt < a->rows || a->ld_vt % 64) return iris_set_error("kv_prepare: ld_vt=%d", a->ld_vt);
    if (a->heads <= 0 || a->kv_heads < 0 || a->kv_heads > a->heads)
        return iris_set_error("kv_prepare: heads=%d kv_heads=%d", a->heads, a->kv_heads);
    if (!a->wkA || !a->wkB) return iris_set_error("kv_prepare: K norm weights missing");
    if (((uintptr_t)a->qkv | (uintptr_t)a->k_out | (uintptr_t)a->vt_out | (uintptr_t)a->wkA | (uintptr_t)a->wkB |
         (uintptr_t)a->cos_t | (uintptr_t)a->sin_t | (uintptr_t)a->kcos_t | (uintptr_t)a->ksin_t) & 15)
        return iris_set_error("kv_prepare: buffers must be 16-byte aligned");
    const int kvh = a->kv_heads ? a->kv_heads : a->heads, vx = a->ld_vt / 64;
    const long long blocks = (long long)vx * kvh + (a->rows + NT / IRIS_WAVE - 1) / (NT / IRIS_WAVE);
    if (blocks >= (1LL << 31)) return iris_set_error("kv_prepare: too many rows");
    IRIS_LAUNCH(qkv_prep_kernel<true>, dim3((unsigned)blocks), dim3(NT), 0, iris_stream(), *a, vx * kvh, vx);
    return iris_launch_check("qkv_prep_kernel<K>");
}

int iris_hip_gemv(float *y, const uint16_t *W, const float *x, const float *bias, int N, int K, int act_in) {
    if (N <= 0) return 0;
    if (K % 8) return iris_set_error("gemv: K=%d must be a multiple of 8", K);
    const int rows_per_block = (K <= 256 ? 2 : 1) * (NT / IRIS_WAVE);
    const dim3 grid((N + rows_per_block - 1) / rows_per_block);
    if (K <= GEMV_XLDS)
        IRIS_LAUNCH(gemv_kernel<true>, grid, dim3(NT), 0, iris_stream(), y, W, x, bias, N, K, act_in);
    else
        IRIS_LAUNCH(gemv_kernel<false>, grid, dim3(NT), 0, iris_stream(), y, W, x, bias, N, K, act_in);
    return iris_launch_check("gemv_kernel");
}

int iris_hip_nchw_to_tokens(uint16_t *out, const float *lat, int C, int hw) {
    if (hw <= 0) return 0;
    IRIS_LAUNCH(nchw_to_tokens_kernel, dim3((hw + 63) / 64, (C + 63) / 64), dim3(NT), 0, iris_stream(), out,
                       lat, C, hw);
    return iris_launch_check("nchw_to_tokens_kernel");
}

int iris_hip_f32_to_bf16(uint16_t *o, const float *x, size_t n) {
    if (!n) return 0;
    IRIS_LAUNCH(f32_to_bf16_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), o, x, n);
    return iris_launch_check("f32_to_bf16_kernel");
}

int iris_hip_bf16_to_f32(float *o, const uint16_t *x, size_t n) {
    if (!n) return 0;
    IRIS_LAUNCH(bf16_to_f32_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), o, x, n);
    return iris_launch_check("bf16_to_f32_kernel");
}

int iris_hip_euler(float *z, const float *v, const float *v2, float g, float dt, float sign, size_t n) {
    if (!n) return 0;
    IRIS_LAUNCH(euler_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), z, v, v2, g, dt, sign, n);
    return iris_launch_check("euler_kernel");
}

int iris_hip_patchify(uint16_t *o, const float *lat, int C, int H, int W, int ps) {
    size_t n = (size_t)(H / ps) * (W / ps) * ps * ps * C;
    if (!n) return 0;
    IRIS_LAUNCH(patchify_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), o, lat, C, H, W, ps);
    return iris_launch_check("patchify_kernel");
}

int iris_hip_unpatchify(float *lat, const float *pt, int C, int H, int W, int ps) {
    size_t n = (size_t)(H / ps) * (W / ps) * ps * ps * C;
    if (!n) return 0;
    IRIS_LAUNCH(unpatchify_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), lat, pt, C, H, W, ps);
    return iris_launch_check("unpatchify_kernel");
}

int iris_hip_fill_rows(float *x, const float *row, int r0, int r1, int cols) {
    if (r1 <= r0) return 0;
    size_t n = (size_t)(r1 - r0) * cols;
    IRIS_LAUNCH(fill_rows_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), x, row, r0, r1, cols);
    return iris_launch_check("fill_rows_kernel");
}

int iris_hip_tanh_cols(float *x, int rows, int ld, int c0, int len) {
    if (rows <= 0 || len <= 0) return 0;
    if (c0 < 0 || c0 + len > ld) return iris_set_error("tanh_cols: columns %d..%d outside ld %d", c0, c0 + len, ld);
    const size_t n = (size_t)rows * len;
    IRIS_LAUNCH(tanh_cols_kernel, dim3(grid1d(n)), dim3(NT), 0, iris_stream(), x, rows, ld, c0, len);
    return iris_launch_check("tanh_cols_kernel");
}

int iris_hip_embed_rows(float *out, const uint16_t *table, const int *ids, int rows, int cols, int vocab) {
    if (rows <= 0) return 0;
    if (cols <= 0 || vocab <= 0) return iris_set_error("embed_rows: cols=%d vocab=%d", cols, vocab);
    if (cols % 8 || ((uintptr_t)out | (uintptr_t)table) & 15)
        return iris_set_error("embed_rows: cols %% 8 and 16-byte aligned buffers required");
    IRIS_LAUNCH(embed_rows_kernel, dim3(rows), dim3(NT), 0, iris_stream(), out, table, ids, rows, cols, vocab);
    return iris_launch_check("embed_rows_kernel");
}

int iris_hip_copy_rows(float *dst, int ld_dst, const float *src, int ld_src, int rows, int cols) {
    if (rows <= 0 || cols <= 0) return 0;
    if (ld_dst < cols || ld_src < cols) return iris_set_error("copy_rows: ld_dst=%d ld_src=%d < cols=%d", ld_dst, ld_src, cols);
    IRIS_LAUNCH(copy_rows_kernel, dim3(rows), dim3(NT), 0, iris_stream(), dst, ld_dst, src, ld_src, rows, cols);
    return iris_launch_check("copy_rows_kernel");
}

}  /* extern "C" */

