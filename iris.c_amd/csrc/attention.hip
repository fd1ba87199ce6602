/*
 * attention.hip - flash attention for head_dim 128 on gfx950 MFMA.
 *
 * Replaces the reference's joint / self attention (iris_transformer_flux.c:
 * 1789-2022: per-head sgemm, iris_softmax_cpu, sgemm over a materialised
 * [heads, S, S] score buffer; the generic build's online-softmax variant
 * iris_kernels.c:737-1048; Z-Image's masked scalar loops
 * iris_transformer_zimage.c:689-761). Scores never leave registers.
 *
 * Block = 8 waves, 256 queries of one head (32 per wave), two waves per SIMD:
 * while one wave forms probabilities (VALU) the other's matrix products run.
 * A wave's Q fragments, scores, probabilities and output accumulators all fit
 * in its 256 registers. Keys stream through LDS in tiles of 64 (two stages):
 *   S^T[key][q] = K Q^T          (K tile = MFMA A operand from LDS,
 *                                 Q = B operand held in registers)
 *   online softmax per query column in the log2 domain, f32: the scale and
 *   log2(e) are folded into the exp2 argument, p = exp2(fma(s, c, -m))
 *   O^T[d][q] += V^T P^T         (V^T tile = A operand from LDS, P = B operand
 *                                 taken straight from the S^T accumulators)
 * Computing S transposed puts each query's probabilities in the B-operand
 * layout of the PV product, so P never goes through LDS. V arrives already
 * transposed ([head][d][key], written by iris_hip_qk_prepare).
 *
 * Grouped-query attention reads K / V head h / kv_group for query head h.
 * With causal set a block stops at the key tile of its last query and tiles
 * past a wave's first query are masked per element (key <= query).
 *
 * The running max is updated lazily: O and the row sums are rescaled only when
 * some query's tile max exceeds its running max by more than 8 (log2 units),
 * so probabilities stay <= 2^8 and most tiles skip the rescale. Key masks
 * (sequence end, padding ranges) cost one uniform branch per tile and are
 * applied only to tiles that are not fully valid.
 *
 * LDS rows are padded instead of swizzled, so every fragment address is one
 * base register plus an immediate offset: K rows hold 128 + 8 elements (272 B:
 * 16 consecutive rows start 4 banks apart, conflict-free 16-byte reads), V^T
 * rows 64 + 4 (136 B: 32 consecutive rows start 2 banks apart, conflict-free
 * 8-byte reads). Global loads go through buffer descriptors; K's range ends at
 * its last valid row so rows past the end read as zero.
 *
 * Blocks are ordered head-major and mapped XCD-major (block b runs on XCD
 * b % 8 and takes a contiguous range of the work list), so the query blocks
 * of one head share its K and V in one XCD's L2.
 */
#include "iris_internal.h"

namespace {

constexpr int QB = 256, KB = 64, HD = 128, NT = 512, NW = NT / 64, QW = QB / NW;
constexpr float RESCALE_LOG2 = 8.0f;
constexpr int KSTR = HD + 8, VSTR = KB + 4;
constexpr int KS_ELEMS = KB * KSTR, VS_ELEMS = HD * VSTR;
constexpr size_t SMEM_BYTES = (size_t)(2 * KS_ELEMS + 2 * VS_ELEMS) * 2;
static_assert(QW == 32, "one 32-query MFMA column block per wave");

__global__ __launch_bounds__(NT) void flash_attn_kernel(const iris_attn_args_t a, float scale_log2, int nqb,
                                                        int per_xcd, int total) {
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
#define KBUF(b) (smem + (b) * KS_ELEMS)
#define VBUF(b) (smem + 2 * KS_ELEMS + (b) * VS_ELEMS)

    const int L = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (L >= total) return;
    const int qblk = L % nqb, hb = L / nqb;
    const int head = hb % a.heads, bz = hb / a.heads;
    const int kv_head = a.kv_group > 1 ? head / a.kv_group : head;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, lg = lane >> 5;
    const uint16_t *Q = a.q + (size_t)bz * a.q_bstride + head * HD;
    const uint16_t *K = a.k + (size_t)bz * a.k_bstride + kv_head * HD;
    const uint16_t *VT = a.vt + (size_t)bz * a.vt_bstride + (size_t)kv_head * HD * a.ld_vt;
    uint16_t *O = a.o + (size_t)bz * a.o_bstride + head * HD;
    const int sq = a.sq, sk = a.sk;
    /* causal: the block's last query needs keys up to its own index */
    const int nkt = a.causal ? (min(sk, min(sq, (qblk + 1) * QB)) + KB - 1) / KB : (sk + KB - 1) / KB;
    const int wave_q0 = qblk * QB + wave * QW;

    /* Q fragments (B operand): lane holds query lr of the wave's 32, d = ds*16 + lg*8 .. +7 */
    const int q_row = qblk * QB + wave * QW + lr;
    bf16x8 qf[8];
#pragma unroll
    for (int ds = 0; ds < 8; ds++) {
        u16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
        if (q_row < sq) v = *(const u16x8 *)(Q + (size_t)q_row * a.ld_q + ds * 16 + lg * 8);
        qf[ds] = __builtin_bit_cast(bf16x8, v);
    }

    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[i][r] = 0.0f;
    /* running max of the lane's query column (same in both lanes of the column)
     * and this lane's partial row sum over its half of each tile's keys */
    float m_run = -1e30f, l_run = 0.0f;

    /* staging: 2 K chunks (16B) and 2 V^T chunks per thread per tile */
    const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)K, (short)0, (int)(((size_t)(sk - 1) * a.ld_k + HD) * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)VT, (short)0, (int)((size_t)HD * a.ld_vt * 2), 0x00020000);
    const int k_off = ((tid >> 4) * a.ld_k + (tid & 15) * 8) * 2;     /* rows tid/16 (+32) */
    const int v_off = ((tid >> 3) * a.ld_vt + (tid & 7) * 8) * 2;     /* d rows tid/8 (+64) */
    uint4 rk[2], rv[2];
    auto gload = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            rk[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  k_rsrc, k_off, (kt * KB + 32 * i) * a.ld_k * 2, 0));
            rv[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  v_rsrc, v_off, (64 * i * a.ld_vt + kt * KB) * 2, 0));
        }
    };
    auto sstore = [&](int buf) {
        uint16_t *kd = KBUF(buf) + (tid >> 4) * KSTR + (tid & 15) * 8;
        uint16_t *vd = VBUF(buf) + (tid >> 3) * VSTR + (tid & 7) * 8;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            *(uint4 *)(kd + 32 * i * KSTR) = rk[i];
            *(uint2 *)(vd + 64 * i * VSTR) = make_uint2(rv[i].x, rv[i].y);
            *(uint2 *)(vd + 64 * i * VSTR + 4) = make_uint2(rv[i].z, rv[i].w);
        }
    };

    gload(0);
    sstore(0);
    if (nkt > 1) gload(1);
    __syncthreads();

    for (int kt = 0; kt < nkt; ++kt) {
        const int cur = kt & 1, k0 = kt * KB;
        /* S^T for the tile: 2 key sub-tiles of 32 x the wave's 32 queries */
        f32x16 s[2];
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int r = 0; r < 16; r++) s[ks][r] = 0.0f;
#pragma unroll
        for (int ds = 0; ds < 8; ds++) {
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const bf16x8 kf = *(const bf16x8 *)(&KBUF(cur)[(ks * 32 + lr) * KSTR + (ds * 2 + lg) * 8]);
                s[ks] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ds], s[ks], 0, 0, 0);
            }
        }
        /* the stage read in step kt-1 is free: tile kt+1 goes there, tile kt+2's loads start */
        if (kt + 1 < nkt) sstore(cur ^ 1);
        if (kt + 2 < nkt) gload(kt + 2);

        const bool full = k0 + KB <= sk && ((k0 >= a.kv_lo0 && k0 + KB <= a.kv_hi0) ||
                                            (k0 >= a.kv_lo1 && k0 + KB <= a.kv_hi1)) &&
                          !(a.causal && k0 + KB - 1 > wave_q0);
        if (!full) {
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = k0 + ks * 32 + (r >> 2) * 8 + lg * 4 + (r & 3);
                    const bool ok = (key < sk) & (((key >= a.kv_lo0) & (key < a.kv_hi0)) |
                                                  ((key >= a.kv_lo1) & (key < a.kv_hi1))) &
                                    (!a.causal | (key <= q_row));
                    s[ks][r] = ok ? s[ks][r] : -INFINITY;
                }
        }
        if (a.key_bias != 0.0f && k0 + KB > a.bias_from) {
            /* logit bias on keys >= bias_from, in units of the raw scores */
            const float bs = a.key_bias / a.scale;
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = k0 + ks * 32 + (r >> 2) * 8 + lg * 4 + (r & 3);
                    s[ks][r] += key >= a.bias_from ? bs : 0.0f;
                }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[ks][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * scale_log2;
        if (__any(mx > m_run + RESCALE_LOG2)) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int dsub = 0; dsub < 4; dsub++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[dsub][r] *= alpha;
        }

        /* P = exp2(S - m) as bf16 B-operand fragments; O^T += V^T P^T */
        bf16x8 pf[4];
        float rs = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            bf16x8 v;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float p = __builtin_amdgcn_exp2f(fmaf(s[j >> 1][(j & 1) * 8 + e], scale_log2, -m_run));
                rs += p;
                v[e] = (__bf16)p;
            }
            pf[j] = v;
        }
        l_run += rs;
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int dsub = 0; dsub < 4; dsub++) {
                const int d = dsub * 32 + lr;
                const uint2 lo = *(const uint2 *)(&VBUF(cur)[d * VSTR + (4 * j + lg) * 4]);
                const uint2 hi = *(const uint2 *)(&VBUF(cur)[d * VSTR + (4 * j + 2 + lg) * 4]);
                const bf16x8 vf = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
                o[dsub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[j], o[dsub], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    /* normalise and store O[q][d]: lane holds query lr, d = dsub*32 + (r>>2)*8 + lg*4 + (r&3) */
    const float l = l_run + __shfl_xor(l_run, 32, 64);
    if (q_row < sq) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int dsub = 0; dsub < 4; dsub++)
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                const int d = dsub * 32 + rb * 8 + lg * 4;
                u16x4 v;
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = f2bf(o[dsub][rb * 4 + e] * inv);
                *(u16x4 *)(O + (size_t)q_row * a.ld_o + d) = v;
            }
    }
#undef KBUF
#undef VBUF
}

}  // namespace

extern "C" int iris_hip_attention(const iris_attn_args_t *a) {
    if (a->sq <= 0 || a->sk <= 0 || a->heads <= 0 || a->batch <= 0) return 0;
    if (a->ld_q % 8 || a->ld_k % 8 || a->ld_o % 4 || a->ld_vt % 8)
        return iris_set_error("attention: leading dimensions must be multiples of 8");
    if (a->ld_vt < ((a->sk + KB - 1) / KB) * KB)
        return iris_set_error("attention: ld_vt %d < padded key count", a->ld_vt);
    if (a->kv_group < 0 || (a->kv_group > 1 && a->heads % a->kv_group))
        return iris_set_error("attention: %d heads not a multiple of kv_group %d", a->heads, a->kv_group);
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
