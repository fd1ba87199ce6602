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
 * sub-tiles); one wave per SIMD. The block's Q tile sits in LDS; keys
 * stream through LDS in tiles of 64:
 *   S^T[key][q] = K Q^T          (K tile = MFMA A operand, Q = B operand,
 *                                 both read from LDS)
 *   online softmax per query column in the log2 domain, f32: the scale and
 *   log2(e) are folded into the exp2 argument, p = exp2(fma(s, c, -m))
 *   O^T[d][q] += V^T P^T         (V^T tile = A operand from LDS, P = B operand
 *                                 taken straight from the S^T accumulators)
 * Computing S transposed puts each query's probabilities in the B-operand
 * layout of the PV product, so P never goes through LDS. V arrives already
 * transposed ([head][d][key], written by iris_hip_qk_prepare).
 *
 * Pipelining: while tile t's probabilities are formed (VALU) and multiplied
 * into O (MFMA), the scores of tile t+1 are already being computed (MFMA), so
 * the exp/sum work overlaps matrix work inside one wave. K tiles are staged two
 * tiles ahead and V tiles one ahead (two LDS buffers each).
 *
 * The running max is updated lazily: O and the row sums are rescaled only when
 * some query's tile max exceeds its running max by more than 8 (log2 units),
 * so probabilities stay <= 2^8 and most tiles skip the 128-register rescale.
 * Key masks (sequence end, padding ranges) cost one uniform branch per tile
 * and are applied only to tiles that are not fully valid.
 *
 * Blocks are ordered head-major and mapped XCD-major (block b runs on XCD
 * b % 8 and takes a contiguous range of the work list), so the query blocks
 * of one head share its K and V in one XCD's L2.
 */
#include "iris_internal.h"

namespace {

constexpr int QB = 256, KB = 64, HD = 128, NT = 256;
constexpr float RESCALE_LOG2 = 8.0f;
/* LDS rows are padded instead of swizzled, so every fragment address is one
 * base register plus an immediate offset: K and Q rows hold 128 + 8 elements
 * (272 B: 8 consecutive rows start 4 banks apart, conflict-free 16-byte
 * reads), V^T rows 64 + 4 (136 B: 16 consecutive rows start 2 banks apart,
 * conflict-free 8-byte reads). K tiles 2 x 17 KB, V^T tiles 2 x 17 KB, Q 68 KB. */
constexpr int KSTR = HD + 8, VSTR = KB + 4;
constexpr int KS_ELEMS = KB * KSTR, VS_ELEMS = HD * VSTR, QS_ELEMS = QB * KSTR;
constexpr size_t SMEM_BYTES = (size_t)(2 * KS_ELEMS + 2 * VS_ELEMS + QS_ELEMS) * 2;

typedef f32x16 stile[2][2];    /* [key sub-tile][query sub-tile] */

__global__ __launch_bounds__(NT) void flash_attn_kernel(const iris_attn_args_t a, float scale_log2, int nqb,
                                                        int per_xcd, int total) {
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    uint16_t *const Qs = smem + 2 * KS_ELEMS + 2 * VS_ELEMS;
#define KBUF(b) (smem + (b) * KS_ELEMS)
#define VBUF(b) (smem + 2 * KS_ELEMS + (b) * VS_ELEMS)

    const int L = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (L >= total) return;
    const int qblk = L % nqb, hb = L / nqb;
    const int head = hb % a.heads, bz = hb / a.heads;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, lg = lane >> 5;
    const uint16_t *Q = a.q + (size_t)bz * a.q_bstride + head * HD;
    const uint16_t *K = a.k + (size_t)bz * a.k_bstride + head * HD;
    const uint16_t *VT = a.vt + (size_t)bz * a.vt_bstride + (size_t)head * HD * a.ld_vt;
    uint16_t *O = a.o + (size_t)bz * a.o_bstride + head * HD;
    const int sq = a.sq, sk = a.sk;
    const int nkt = (sk + KB - 1) / KB;

    /* Q tile into LDS (rows past the end are zero) */
#pragma unroll 4
    for (int i = 0; i < QB * 16 / NT; i++) {
        const int c = tid + NT * i;
        const int row = c >> 4, ch = c & 15, q = qblk * QB + row;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (q < sq) v = *(const uint4 *)(Q + (size_t)q * a.ld_q + ch * 8);
        *(uint4 *)(&Qs[row * KSTR + ch * 8]) = v;
    }

    f32x16 o[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[i][j][r] = 0.0f;
    /* running max per query column (identical in the two lanes of a column) and
     * this lane's partial row sum over its half of each tile's keys */
    float m_run[2] = {-1e30f, -1e30f}, l_run[2] = {0.0f, 0.0f};

    /* staging registers: 4 K chunks (16B) and 4 V^T chunks per thread per tile,
     * loaded through buffer resources: K's range ends at its last valid row so
     * rows past the end read as zero */
    const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)K, (short)0, (int)(((size_t)(sk - 1) * a.ld_k + HD) * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)VT, (short)0, (int)((size_t)HD * a.ld_vt * 2), 0x00020000);
    const int k_off = ((tid >> 4) * a.ld_k + (tid & 15) * 8) * 2;
    const int v_off = ((tid >> 3) * a.ld_vt + (tid & 7) * 8) * 2;
    uint4 rk[4], rv[4];
    auto gload_k = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            rk[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  k_rsrc, k_off, (kt * KB + 16 * i) * a.ld_k * 2, 0));
    };
    auto gload_v = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            rv[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  v_rsrc, v_off, (32 * i * a.ld_vt + kt * KB) * 2, 0));
    };
    auto sstore_k = [&](int buf) {
        uint16_t *dst = KBUF(buf) + (tid >> 4) * KSTR + (tid & 15) * 8;
#pragma unroll
        for (int i = 0; i < 4; i++) *(uint4 *)(dst + 16 * i * KSTR) = rk[i];
    };
    auto sstore_v = [&](int buf) {
        uint16_t *dst = VBUF(buf) + (tid >> 3) * VSTR + (tid & 7) * 8;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            *(uint2 *)(dst + 32 * i * VSTR) = make_uint2(rv[i].x, rv[i].y);
            *(uint2 *)(dst + 32 * i * VSTR + 4) = make_uint2(rv[i].z, rv[i].w);
        }
    };

    /* S^T of one tile from Ks[buf] */
    auto scores = [&](int buf, stile &s) {
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int qs = 0; qs < 2; qs++)
#pragma unroll
                for (int r = 0; r < 16; r++) s[ks][qs][r] = 0.0f;
#pragma unroll
        for (int ds = 0; ds < 8; ds++) {
            bf16x8 qf[2];
#pragma unroll
            for (int qs = 0; qs < 2; qs++)
                qf[qs] = *(const bf16x8 *)(&Qs[(wave * 64 + qs * 32 + lr) * KSTR + (ds * 2 + lg) * 8]);
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const bf16x8 kf = *(const bf16x8 *)(&KBUF(buf)[(ks * 32 + lr) * KSTR + (ds * 2 + lg) * 8]);
#pragma unroll
                for (int qs = 0; qs < 2; qs++)
                    s[ks][qs] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[qs], s[ks][qs], 0, 0, 0);
            }
        }
    };

    /* keys past the end or outside [lo0, hi0) U [lo1, hi1) get -inf (uniform branch per tile);
     * then the lazy running-max update for the tile */
    auto finish_scores = [&](int kt, stile &s) {
        const int k0 = kt * KB;
        const bool full = k0 + KB <= sk && ((k0 >= a.kv_lo0 && k0 + KB <= a.kv_hi0) ||
                                            (k0 >= a.kv_lo1 && k0 + KB <= a.kv_hi1));
        if (!full) {
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = k0 + ks * 32 + (r >> 2) * 8 + lg * 4 + (r & 3);
                    const bool ok = (key < sk) & (((key >= a.kv_lo0) & (key < a.kv_hi0)) |
                                                  ((key >= a.kv_lo1) & (key < a.kv_hi1)));
#pragma unroll
                    for (int qs = 0; qs < 2; qs++) s[ks][qs][r] = ok ? s[ks][qs][r] : -INFINITY;
                }
        }
        float mx[2];
#pragma unroll
        for (int qs = 0; qs < 2; qs++) {
            float m = -INFINITY;
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int r = 0; r < 16; r++) m = fmaxf(m, s[ks][qs][r]);
            mx[qs] = fmaxf(m, __shfl_xor(m, 32, 64)) * scale_log2;
        }
        const bool need = mx[0] > m_run[0] + RESCALE_LOG2 || mx[1] > m_run[1] + RESCALE_LOG2;
        if (__any(need)) {
#pragma unroll
            for (int qs = 0; qs < 2; qs++) {
                const float m_new = fmaxf(m_run[qs], mx[qs]);
                const float alpha = __builtin_amdgcn_exp2f(m_run[qs] - m_new);
                m_run[qs] = m_new;
                l_run[qs] *= alpha;
#pragma unroll
                for (int dsub = 0; dsub < 4; dsub++)
#pragma unroll
                    for (int r = 0; r < 16; r++) o[dsub][qs][r] *= alpha;
            }
        }
    };

    /* P = exp2(S - m) as bf16 B-operand fragments, row sums, then O^T += V^T P^T from Vs[buf] */
    auto accumulate = [&](int buf, stile &s) {
        bf16x8 pf[2][4];
#pragma unroll
        for (int qs = 0; qs < 2; qs++) {
            float rs = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                bf16x8 v;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(s[j >> 1][qs][(j & 1) * 8 + e], scale_log2, -m_run[qs]));
                    rs += p;
                    v[e] = (__bf16)p;
                }
                pf[qs][j] = v;
            }
            l_run[qs] += rs;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int dsub = 0; dsub < 4; dsub++) {
                const int d = dsub * 32 + lr;
                const uint2 lo = *(const uint2 *)(&VBUF(buf)[d * VSTR + (4 * j + lg) * 4]);
                const uint2 hi = *(const uint2 *)(&VBUF(buf)[d * VSTR + (4 * j + 2 + lg) * 4]);
                const bf16x8 vf = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
                for (int qs = 0; qs < 2; qs++)
                    o[dsub][qs] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[qs][j], o[dsub][qs], 0, 0, 0);
            }
        }
    };

    /* one key tile: scores of tile kt are in sc; computes tile kt+1's scores into sn.
     * Loads past the last tile are clamped to it (in bounds, results unused). */
    auto step = [&](int kt, stile &sc, stile &sn) {
        const int last = nkt - 1;
        gload_k(min(kt + 2, last));
        gload_v(min(kt + 1, last));
        scores((kt + 1) & 1, sn);
        accumulate(kt & 1, sc);
        sstore_k(kt & 1);
        sstore_v((kt + 1) & 1);
        __syncthreads();
        if (kt + 1 < nkt) finish_scores(kt + 1, sn);
    };

    /* prologue: K0, V0, K1 staged; scores of tile 0 */
    gload_k(0);
    gload_v(0);
    sstore_k(0);
    sstore_v(0);
    gload_k(min(1, nkt - 1));
    sstore_k(1);
    __syncthreads();
    stile sA, sB;
    scores(0, sA);
    finish_scores(0, sA);

    for (int kt = 0; kt < nkt; kt += 2) {
        step(kt, sA, sB);
        if (kt + 1 < nkt) step(kt + 1, sB, sA);
    }

    /* normalise and store O[q][d]: lane holds query lr, d = dsub*32 + (r>>2)*8 + lg*4 + (r&3) */
#pragma unroll
    for (int qs = 0; qs < 2; qs++) {
        const int q = qblk * QB + wave * 64 + qs * 32 + lr;
        const float l = l_run[qs] + __shfl_xor(l_run[qs], 32, 64);
        if (q >= sq) continue;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
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

#undef KBUF
#undef VBUF

}  // namespace

extern "C" int iris_hip_attention(const iris_attn_args_t *a) {
    if (a->sq <= 0 || a->sk <= 0 || a->heads <= 0 || a->batch <= 0) return 0;
    if (a->ld_q % 8 || a->ld_k % 8 || a->ld_o % 4 || a->ld_vt % 8)
        return iris_set_error("attention: leading dimensions must be multiples of 8");
    if (a->ld_vt < ((a->sk + KB - 1) / KB) * KB)
        return iris_set_error("attention: ld_vt %d < padded key count", a->ld_vt);
    if (((uintptr_t)a->q | (uintptr_t)a->k | (uintptr_t)a->vt) & 15)
        return iris_set_error("attention: operands must be 16-byte aligned");
    const int nqb = (a->sq + QB - 1) / QB;
    const long long total = (long long)nqb * a->heads * a->batch;
    if (total > (1LL << 28)) return iris_set_error("attention: grid too large");
    const int per_xcd = (int)((total + 7) / 8);
    const float scale_log2 = a->scale * 1.4426950408889634f;
    static bool attr_set = false;
    if (!attr_set) {
        if (iris_check(hipFuncSetAttribute((const void *)flash_attn_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)SMEM_BYTES),
                       "attention smem attribute"))
            return -1;
        attr_set = true;
    }
    hipLaunchKernelGGL(flash_attn_kernel, dim3(8 * per_xcd), dim3(NT), SMEM_BYTES, iris_stream(), *a, scale_log2,
                       nqb, per_xcd, (int)total);
    return iris_launch_check("flash_attn_kernel");
}
