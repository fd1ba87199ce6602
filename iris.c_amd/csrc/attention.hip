/*
 * attention.hip - flash attention for head_dim 128 on gfx950 MFMA.
 *
 * Replaces the reference's joint / self attention (iris_transformer_flux.c:
 * 1789-2022: per-head sgemm, iris_softmax_cpu, sgemm over a materialised
 * [heads, S, S] score buffer; the generic build's online-softmax variant
 * iris_kernels.c:737-1048; Z-Image's masked scalar loops
 * iris_transformer_zimage.c:689-761). Scores never leave registers.
 *
 * Block = 4 waves, 256 queries of one head (64 per wave, two 32-query
 * sub-tiles). Keys stream through LDS in tiles of 64 (double buffered):
 *   S^T[key][q] = K Q^T          (K tile = MFMA A operand from LDS,
 *                                 Q = B operand held in registers)
 *   online softmax in the log2 domain, per query column, f32
 *   O^T[d][q] += V^T P^T         (V^T tile = A operand from LDS, P = B operand
 *                                 taken straight from the S^T accumulators)
 * Computing S transposed puts each query's probabilities in the B-operand
 * layout of the PV product, so P never goes through LDS. V arrives already
 * transposed ([head][d][key], written by iris_hip_qk_prepare).
 */
#include "iris_internal.h"

namespace {

constexpr int QB = 256, KB = 64, HD = 128, NT = 256;

__device__ __forceinline__ int kswz(int row, int ch) {       /* K tile: 16 chunks of 16B per row */
    return row * HD + ((ch ^ (row & 7)) << 3);
}
__device__ __forceinline__ int vswz(int d, int unit) {       /* V^T tile: 16 units of 8B per row */
    return d * KB + ((unit ^ (d & 15)) << 2);
}

__global__ __launch_bounds__(NT) void flash_attn_kernel(const iris_attn_args_t a, float scale_log2) {
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][KB * HD];
    __shared__ __attribute__((aligned(16))) uint16_t Vs[2][HD * KB];

    const int qblk = blockIdx.x, head = blockIdx.y, bz = blockIdx.z;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, lg = lane >> 5;
    const uint16_t *Q = a.q + (size_t)bz * a.q_bstride + head * HD;
    const uint16_t *K = a.k + (size_t)bz * a.k_bstride + head * HD;
    const uint16_t *VT = a.vt + (size_t)bz * a.vt_bstride + (size_t)head * HD * a.ld_vt;
    uint16_t *O = a.o + (size_t)bz * a.o_bstride + head * HD;
    const int sq = a.sq, sk = a.sk;

    /* Q fragments: B operand, lane holds query lr of sub-tile qs, d = ds*16 + lg*8 .. +7 */
    bf16x8 qf[2][8];
#pragma unroll
    for (int qs = 0; qs < 2; qs++) {
        const int q = qblk * QB + wave * 64 + qs * 32 + lr;
#pragma unroll
        for (int ds = 0; ds < 8; ds++) {
            u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
            if (q < sq) v = *(const u16x8 *)(Q + (size_t)q * a.ld_q + ds * 16 + lg * 8);
            qf[qs][ds] = __builtin_bit_cast(bf16x8, v);
        }
    }

    f32x16 o[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[i][j][r] = 0.0f;
    float m_run[2] = {-1e30f, -1e30f}, l_run[2] = {0.0f, 0.0f};

    /* staging: 4 K chunks (16B) and 4 V^T chunks per thread per tile */
    uint4 rk[4], rv[4];
    auto gload = [&](int kt) {
        const int k0 = kt * KB;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + NT * i;
            const int row = c >> 4, ch = c & 15;
            rk[i] = (k0 + row < sk) ? *(const uint4 *)(K + (size_t)(k0 + row) * a.ld_k + ch * 8)
                                    : make_uint4(0, 0, 0, 0);
            const int d = c >> 3, vc = c & 7;
            rv[i] = *(const uint4 *)(VT + (size_t)d * a.ld_vt + k0 + vc * 8);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + NT * i;
            const int row = c >> 4, ch = c & 15;
            *(uint4 *)(&Ks[buf][kswz(row, ch)]) = rk[i];
            const int d = c >> 3, vc = c & 7;
            *(uint2 *)(&Vs[buf][vswz(d, 2 * vc)]) = make_uint2(rv[i].x, rv[i].y);
            *(uint2 *)(&Vs[buf][vswz(d, 2 * vc + 1)]) = make_uint2(rv[i].z, rv[i].w);
        }
    };

    const int nkt = (sk + KB - 1) / KB;
    gload(0);
    sstore(0);
    __syncthreads();

    for (int kt = 0; kt < nkt; ++kt) {
        const int cur = kt & 1;
        const int k0 = kt * KB;
        if (kt + 1 < nkt) gload(kt + 1);

        /* S^T for 2 key sub-tiles x 2 query sub-tiles */
        f32x16 s[2][2];
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int qs = 0; qs < 2; qs++)
#pragma unroll
                for (int r = 0; r < 16; r++) s[ks][qs][r] = 0.0f;
#pragma unroll
        for (int ds = 0; ds < 8; ds++) {
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const bf16x8 kf = __builtin_bit_cast(
                    bf16x8, *(const u16x8 *)(&Ks[cur][kswz(ks * 32 + lr, ds * 2 + lg)]));
#pragma unroll
                for (int qs = 0; qs < 2; qs++)
                    s[ks][qs] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[qs][ds], s[ks][qs], 0, 0, 0);
            }
        }

        /* mask keys past the end and outside the valid segments */
        const bool full = (k0 >= a.kv_lo0 && k0 + KB <= a.kv_hi0) || (k0 >= a.kv_lo1 && k0 + KB <= a.kv_hi1);
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int qs = 0; qs < 2; qs++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    float v = s[ks][qs][r] * scale_log2;
                    if (!full) {
                        const int key = k0 + ks * 32 + (r >> 2) * 8 + lg * 4 + (r & 3);
                        const bool ok = key < sk && ((key >= a.kv_lo0 && key < a.kv_hi0) ||
                                                     (key >= a.kv_lo1 && key < a.kv_hi1));
                        if (!ok) v = -INFINITY;
                    }
                    s[ks][qs][r] = v;
                }

        /* online softmax per query column */
        bf16x8 pf[2][4];
#pragma unroll
        for (int qs = 0; qs < 2; qs++) {
            float mx = -INFINITY;
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[ks][qs][r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(m_run[qs], mx);
            const float alpha = __builtin_amdgcn_exp2f(m_run[qs] - m_new);
            m_run[qs] = m_new;
            float rs = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const float p = __builtin_amdgcn_exp2f(s[ks][qs][r] - m_new);
                    s[ks][qs][r] = p;
                    rs += p;
                }
            rs += __shfl_xor(rs, 32, 64);
            l_run[qs] = l_run[qs] * alpha + rs;
#pragma unroll
            for (int dsub = 0; dsub < 4; dsub++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[dsub][qs][r] *= alpha;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                bf16x8 v;
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = (__bf16)s[j >> 1][qs][(j & 1) * 8 + e];
                pf[qs][j] = v;
            }
        }

        /* O^T += V^T P^T */
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int dsub = 0; dsub < 4; dsub++) {
                const int d = dsub * 32 + lr;
                const uint2 lo = *(const uint2 *)(&Vs[cur][vswz(d, 4 * j + lg)]);
                const uint2 hi = *(const uint2 *)(&Vs[cur][vswz(d, 4 * j + 2 + lg)]);
                const uint4 vv = make_uint4(lo.x, lo.y, hi.x, hi.y);
                const bf16x8 vf = __builtin_bit_cast(bf16x8, vv);
#pragma unroll
                for (int qs = 0; qs < 2; qs++)
                    o[dsub][qs] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[qs][j], o[dsub][qs], 0, 0, 0);
            }
        }

        if (kt + 1 < nkt) sstore(cur ^ 1);
        __syncthreads();
    }

    /* normalise and store O[q][d]: lane holds query lr, d = dsub*32 + (r>>2)*8 + lg*4 + (r&3) */
#pragma unroll
    for (int qs = 0; qs < 2; qs++) {
        const int q = qblk * QB + wave * 64 + qs * 32 + lr;
        if (q >= sq) continue;
        const float inv = l_run[qs] > 0.0f ? 1.0f / l_run[qs] : 0.0f;
#pragma unroll
        for (int dsub = 0; dsub < 4; dsub++)
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                const int d = dsub * 32 + rb * 8 + lg * 4;
                u16x4 v;
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = f2bf(o[dsub][qs][rb * 4 + e] * inv);
                *(u16x4 *)(O + (size_t)q * a.ld_o + d) = v;
            }
    }
}

}  // namespace

extern "C" int iris_hip_attention(const iris_attn_args_t *a) {
    if (a->sq <= 0 || a->sk <= 0 || a->heads <= 0 || a->batch <= 0) return 0;
    if (a->ld_q % 8 || a->ld_k % 8 || a->ld_o % 4 || a->ld_vt % 8)
        return iris_set_error("attention: leading dimensions must be multiples of 8");
    if (a->ld_vt < ((a->sk + KB - 1) / KB) * KB)
        return iris_set_error("attention: ld_vt %d < padded key count", a->ld_vt);
    if (((uintptr_t)a->q | (uintptr_t)a->k | (uintptr_t)a->vt) & 15)
        return iris_set_error("attention: operands must be 16-byte aligned");
    dim3 grid((a->sq + QB - 1) / QB, a->heads, a->batch);
    const float scale_log2 = a->scale * 1.4426950408889634f;
    hipLaunchKernelGGL(flash_attn_kernel, grid, dim3(NT), 0, iris_stream(), *a, scale_log2);
    return iris_launch_check("flash_attn_kernel");
}
