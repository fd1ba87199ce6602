/*
 * attention.hip - flash attention for head_dim 128 on gfx950 MFMA.
 *
 * Replaces the reference's joint / self attention (iris_transformer_flux.c:
 * 1789-2022: per-head sgemm, iris_softmax_cpu, sgemm over a materialised
 * [heads, S, S] score buffer; the generic build's online-softmax variant
 * iris_kernels.c:737-1048; Z-Image's masked scalar loops
 * iris_transformer_zimage.c:689-761) and, in its prologue, the Q half of
 * apply_qk_norm + apply_rope_2d (iris_transformer_flux.c:1464-1518,
 * :1026-1048). Scores never leave registers.
 *
 * Block = 8 waves, 256 queries of one head (32 per wave). Per 64-key tile a
 * wave runs
 *   S^T[key][q] = K Q^T          (K tile = MFMA A operand from LDS,
 *                                 Q = B operand held in registers)
 *   online softmax per query column in the log2 domain, f32: the scale and
 *   log2(e) are folded into the exp2 argument, p = exp2(fma(s, c, -m))
 *   O^T[d][q] += V^T P^T         (V^T tile = A operand from LDS, P = B operand
 *                                 taken straight from the S^T accumulators)
 * Computing S transposed puts each query's probabilities in the B-operand
 * layout of the PV product, so P never goes through LDS. V arrives already
 * transposed ([head][d][key], written by iris_hip_kv_prepare).
 *
 * Wave groups in ping-pong: waves w and w + 4 share SIMD w, group 0 = waves
 * 0..3, group 1 = waves 4..7. Phases are separated by block barriers; in
 * every phase one group runs matrix products (M phase: PV of the previous
 * tile, then QK of this tile: 32 MFMAs) while the other forms probabilities
 * (V phase: masks, max, rescale, exp2, row sums: VALU), so each SIMD's
 * matrix core and VALU work at the same time:
 *   phase 2t:     group 0 M(t)      group 1 V(t-1)
 *   phase 2t + 1: group 0 V(t)      group 1 M(t)
 * Keys and values stream through two K and two V^T stages. In its M(t)
 * phase each group stores its half of K(t+1) and V(t) from registers (loaded
 * one phase pair earlier) and issues the loads of K(t+2) and V(t+1):
 *   - K(t+1) goes to the K stage of K(t-1), read in phases 2t-2 and 2t-1,
 *     and is read from phase 2t+2;
 *   - V(t) goes to the V stage of V(t-2), read (PV of tile t-2) in phases
 *     2t-2 and 2t-1, and is read from phase 2t+2.
 * A barrier waits only for the wave's LDS operations, not for its global
 * loads in flight.
 *
 * With a Q prologue (qn_wA set) each wave normalises its 32 raw query rows
 * row by row (16 lanes per row: coalesced reads of the projection and of the
 * per-pair RoPE tables), RMS-normalises each head row in f32, rotates the
 * pairs (2i, 2i+1) and rounds to bf16 once: the arithmetic of the K pass,
 * without writing and re-reading Q. The rows go through LDS into the MFMA
 * operand layout.
 *
 * The running max is updated lazily: O and the row sums are rescaled only when
 * some query's tile max exceeds its running max by more than 8 (log2 units),
 * so probabilities stay <= 2^8 and most tiles skip the rescale. Key masks
 * (sequence end, padding ranges) cost one uniform branch per tile and are
 * applied only to tiles that are not fully valid. Causal masking and the key
 * logit bias are separate instantiations, so the joint attention of the
 * denoiser carries none of their code.
 *
 * LDS rows are padded instead of swizzled, so every fragment address is one
 * base register plus an immediate offset: K rows hold 128 + 8 elements (272 B:
 * 16 consecutive rows start 4 banks apart, conflict-free 16-byte reads). V^T
 * rows take one of two layouts. One block per unit: rows of 64 + 8 (144 B: 16
 * consecutive rows start at 16 distinct 4-bank groups), each 16 keys stored
 * in the order the P fragments take them (keys 0-3, 8-11, 4-7, 12-15), so a
 * lane's 8 keys of one PV product are one 16-byte read. Balanced schedule:
 * rows of 64 + 4 (136 B) in key order, read as two 8-byte halves, which
 * measured faster there (540 units of 4096 keys, same box: 345.7 us against
 * 407.5 us with the 16-byte layout, while one block per unit gains with it:
 * 432 units of 4608 keys 258.1 -> 253.3 us). Global loads go through buffer
 * descriptors; K's range ends at its last valid row so rows past the end read
 * as zero.
 *
 * Blocks are ordered head-major and mapped XCD-major (block b runs on XCD
 * b % 8 and takes a contiguous range of the work list), so the query blocks
 * of one head share its K and V in one XCD's L2.
 */
#include "iris_internal.h"

#include <string.h>

namespace {

constexpr int QB = 256, KB = 64, HD = 128, NT = 512, NW = NT / 64, QW = QB / NW;
constexpr float RESCALE_LOG2 = 8.0f;
constexpr int KSTR = HD + 8, KS_ELEMS = KB * KSTR;
static_assert(QW == 32, "one 32-query MFMA column block per wave");

enum { F_FUSEQ = 1, F_CAUSAL = 2, F_BIAS = 4, F_SPLIT = 8 };

/* LDS of one block: two K stages, two V^T stages and, with the Q prologue,
 * each wave's 32 normalised, rotated rows after them */
template <int FEAT> struct AttnLds {
    static constexpr bool V16 = !(FEAT & F_SPLIT); /* V^T read as 16-byte chunks */
    static constexpr int VSTR = V16 ? KB + 8 : KB + 4, VS_ELEMS = HD * VSTR;
    static constexpr int QS_OFF = 2 * KS_ELEMS + 2 * VS_ELEMS;
    static constexpr size_t BYTES = (size_t)QS_OFF * 2 + ((FEAT & F_FUSEQ) ? (size_t)NW * 32 * KSTR * 2 : 0);
};

/* Balanced schedule (F_SPLIT): the nkt key tiles of all units (query block,
 * head, batch) form one range of units * nkt steps, dealt out to the blocks
 * (one per CU) in contiguous pieces: block slot s takes per + (s < rem)
 * steps. Slots are numbered XCD-major (slot s runs on XCD s / bpx), so one
 * XCD's blocks work on neighbouring units, mostly of one head, and share its
 * K and V in L2. A unit done by several blocks is finished by the last of
 * them to arrive (cnt[unit] counts arrivals and is left at zero), which
 * merges the partial softmax states in slot order: o and (m, l) of each
 * block's first segment in slot 2s, of its last in slot 2s + 1. */
struct AttnSplit {
    int nkt, per, rem, bpx;
    int *cnt;
    float *ws;   /* o partials, then (m, l) pairs */
    int slots;
};
constexpr int SPLIT_MAX_UNITS = 1 << 16;
constexpr size_t SPLIT_CNT_BYTES = SPLIT_MAX_UNITS * sizeof(int);
constexpr size_t SPLIT_SLOT_BYTES = (size_t)NT * 64 * 4 + (size_t)NT * 8;   /* o, then (m, l) per lane */

__device__ __forceinline__ int split_start(const AttnSplit &sp, int s) { return s * sp.per + min(s, sp.rem); }
__device__ __forceinline__ int split_slot_of(const AttnSplit &sp, int i) {
    const int big = sp.rem * (sp.per + 1);
    return i < big ? i / (sp.per + 1) : sp.rem + (i - big) / sp.per;
}

/* one segment of a unit: key tiles [t0, t0 + tn) of unit L; part != 0: a
 * piece of a unit split over several blocks (slot owner s, first segment of
 * that block or not) */
struct AttnSeg {
    int part, s, first;
};

/* s_waitcnt immediate: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8 */
constexpr int waitcnt_imm(int vm, int lgkm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8); }

template <int FEAT>
__device__ __forceinline__ void attn_segment(const iris_attn_args_t &a, float scale_log2, int nqb, const int L,
                                             const int t0, int tn, const AttnSplit &sp, const AttnSeg sg) {
    constexpr bool FUSEQ = FEAT & F_FUSEQ, CAUSAL = FEAT & F_CAUSAL, BIAS = FEAT & F_BIAS;
    constexpr bool V16 = AttnLds<FEAT>::V16;
    constexpr int VSTR = AttnLds<FEAT>::VSTR, VS_ELEMS = AttnLds<FEAT>::VS_ELEMS, QS_OFF = AttnLds<FEAT>::QS_OFF;
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
#define KBUF(b) (smem + (b) * KS_ELEMS)
#define VBUF(b) (smem + 2 * KS_ELEMS + (b) * VS_ELEMS)

    const int qblk = L % nqb, hb = L / nqb;
    const int head = hb % a.heads, bz = hb / a.heads;
    const int kv_head = a.kv_group > 1 ? head / a.kv_group : head;
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, lg = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2, gt = tid & 255;
    const uint16_t *Q = a.q + (size_t)bz * a.q_bstride + head * HD;
    const uint16_t *K = a.k + (size_t)bz * a.k_bstride + kv_head * HD;
    const uint16_t *VT = a.vt + (size_t)bz * a.vt_bstride + (size_t)kv_head * HD * a.ld_vt;
    uint16_t *O = a.o + (size_t)bz * a.o_bstride + head * HD;
    const int sq = a.sq, sk = a.sk;
    /* the segment's key tiles, t0 .. t0 + nkt - 1 (tn < 0: all; causal: the
     * block's last query needs keys up to its own index) */
    const int nkt = tn >= 0 ? tn
                            : CAUSAL ? (min(sk, min(sq, (qblk + 1) * QB)) + KB - 1) / KB : (sk + KB - 1) / KB;
    const int wave_q0 = qblk * QB + wave * QW;
    const int q_row = wave_q0 + lr;

    /* Every tile offset goes into the VGPR offset, which the buffer range check
     * covers (the SGPR offset is not checked): K rows past sk - 1 read as zero. */
    const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)K, (short)0, (int)(((size_t)(sk - 1) * a.ld_k + HD) * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)VT, (short)0, (int)((size_t)HD * a.ld_vt * 2), 0x00020000);

    /* this group's half of a tile: K rows 32 grp + gt/16 (+ 16), chunk gt % 16;
     * V^T d rows 64 grp + gt/8 (+ 32), chunk gt % 8 */
    const int kh_off = ((32 * grp + (gt >> 4)) * a.ld_k + (gt & 15) * 8) * 2;
    const int vh_off = ((64 * grp + (gt >> 3)) * a.ld_vt + (gt & 7) * 8) * 2;
    uint16_t *const kh_dst = smem + (32 * grp + (gt >> 4)) * KSTR + (gt & 15) * 8;
    /* V^T chunk c = gt % 8 holds keys 8c .. 8c + 7 of the tile; in the 16-byte
     * layout that is key block c / 2, half c % 2: its first 4 keys go to
     * 4 (c % 2), its last 4 to 8 + 4 (c % 2) of the block */
    uint16_t *const vh_dst = smem + 2 * KS_ELEMS + (64 * grp + (gt >> 3)) * VSTR +
                             (V16 ? 16 * ((gt & 7) >> 1) + 4 * (gt & 1) : 8 * (gt & 7));
    uint4 rk[2], rv[2];
    auto load_k = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 2; i++)
            rk[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  k_rsrc, kh_off + ((t0 + kt) * KB + 16 * i) * a.ld_k * 2, 0, 0));
    };
    auto load_v = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 2; i++)
            rv[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  v_rsrc, vh_off + (32 * i * a.ld_vt + (t0 + kt) * KB) * 2, 0, 0));
    };
    auto store_k = [&](int stage) {
#pragma unroll
        for (int i = 0; i < 2; i++) *(uint4 *)(kh_dst + stage * KS_ELEMS + 16 * i * KSTR) = rk[i];
    };
    auto store_v = [&](int stage) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            uint16_t *d = vh_dst + stage * VS_ELEMS + 32 * i * VSTR;
            *(uint2 *)d = make_uint2(rv[i].x, rv[i].y);
            *(uint2 *)(d + (V16 ? 8 : 4)) = make_uint2(rv[i].z, rv[i].w);
        }
    };
    /* the whole K(0) tile: rows tid/16 and + 32, chunk tid % 16 */
    uint4 k0r[2];
    {
        const int k_off = ((tid >> 4) * a.ld_k + (tid & 15) * 8) * 2 + t0 * KB * a.ld_k * 2;
        k0r[0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(k_rsrc, k_off, 0, 0));
        k0r[1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(k_rsrc, k_off + 32 * a.ld_k * 2,
                                                                                  0, 0));
    }
    /* Q loads next, so that their latency and K(0)'s overlap: the fragments
     * (B operand: lane holds query lr of the wave's 32, d = ds*16 + lg*8 ..
     * +7), or for the prologue the wave's 32 raw rows row by row, 16 lanes
     * per row and 8 dims per lane, and their pair tables (coalesced) */
    bf16x8 qf[8];
    u16x8 raw[8];
    float4 c4[8], s4[8], wa0, wa1, wb0, wb1;
    const int rl = lane >> 4, hl = lane & 15, d0 = hl * 8;
    if (!FUSEQ) {
#pragma unroll
        for (int ds = 0; ds < 8; ds++) {
            u16x8 r = {0, 0, 0, 0, 0, 0, 0, 0};
            if (q_row < sq) r = *(const u16x8 *)(Q + (size_t)q_row * a.ld_q + ds * 16 + lg * 8);
            qf[ds] = __builtin_bit_cast(bf16x8, r);
        }
    } else {
        wa0 = *(const float4 *)(a.qn_wA + d0);
        wa1 = *(const float4 *)(a.qn_wA + d0 + 4);
        wb0 = *(const float4 *)(a.qn_wB + d0);
        wb1 = *(const float4 *)(a.qn_wB + d0 + 4);
#pragma unroll
        for (int pass = 0; pass < 8; pass++) {
            const int row = wave_q0 + pass * 4 + rl;
            raw[pass] = (u16x8){0, 0, 0, 0, 0, 0, 0, 0};
            if (row < sq) raw[pass] = *(const u16x8 *)(Q + (size_t)row * a.ld_q + d0);
            c4[pass] = make_float4(1, 1, 1, 1);
            s4[pass] = make_float4(0, 0, 0, 0);
            if (!a.rope_pos && a.rope_cos) {
                const size_t tr = (size_t)(row < sq ? row : 0) * (HD / 2) + hl * 4;
                c4[pass] = *(const float4 *)(a.rope_cos + tr);
                s4[pass] = *(const float4 *)(a.rope_sin + tr);
            }
        }
        if (a.rope_pos) {
            /* factored tables: the lane's 4 pairs hl*4 .. +3 lie on axis hl / 4
             * at entries (hl % 4) * 4 .. +3 of the shared frequency table */
            int pos[8];
#pragma unroll
            for (int pass = 0; pass < 8; pass++) {
                const int row = wave_q0 + pass * 4 + rl;
                pos[pass] = a.rope_pos[(size_t)(row < sq ? row : 0) * 4 + (hl >> 2)];
                pos[pass] = min(max(pos[pass], 0), a.rope_axis_len - 1);
            }
            const float *tc = a.rope_axis + (hl & 3) * 4, *ts = tc + (size_t)a.rope_axis_len * 16;
#pragma unroll
            for (int pass = 0; pass < 8; pass++) {
                c4[pass] = *(const float4 *)(tc + pos[pass] * 16);
                s4[pass] = *(const float4 *)(ts + pos[pass] * 16);
            }
        }
    }
    /* K(1) and V(0) in flight during the Q arithmetic (unconditional, the
     * index clamped: no branch for the wait counters to merge) */
    load_k(min(1, nkt - 1));
    load_v(0);
    {
        uint16_t *kd = KBUF(0) + (tid >> 4) * KSTR + (tid & 15) * 8;
        *(uint4 *)kd = k0r[0];
        *(uint4 *)(kd + 32 * KSTR) = k0r[1];
    }

    /* Q prologue: the raw rows loaded above, with the arithmetic of the K
     * pass (16-lane row sums by DPP), staged in LDS as [32][KSTR] and read
     * back in the B-operand layout */
    auto q_prologue = [&]() {
        uint16_t *qs = smem + QS_OFF + wave * 32 * KSTR;
#pragma unroll
        for (int pass = 0; pass < 8; pass++) {
            const int rw = pass * 4 + rl, row = wave_q0 + rw;
            float x[8], ss = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) { x[j] = bf2f(raw[pass][j]); ss += x[j] * x[j]; }
            ss = row16_sum(ss);
            const float inv = 1.0f / sqrtf(ss / 128.0f + a.qn_eps);
            const bool sa = row < a.qn_split;
            const float ww[8] = {sa ? wa0.x : wb0.x, sa ? wa0.y : wb0.y, sa ? wa0.z : wb0.z, sa ? wa0.w : wb0.w,
                                 sa ? wa1.x : wb1.x, sa ? wa1.y : wb1.y, sa ? wa1.z : wb1.z, sa ? wa1.w : wb1.w};
            const float c[4] = {c4[pass].x, c4[pass].y, c4[pass].z, c4[pass].w};
            const float sn[4] = {s4[pass].x, s4[pass].y, s4[pass].z, s4[pass].w};
            u16x8 out;
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const float x0 = x[j] * inv * ww[j], x1 = x[j + 1] * inv * ww[j + 1];
                out[j] = f2bf(x0 * c[j >> 1] - x1 * sn[j >> 1]);
                out[j + 1] = f2bf(x1 * c[j >> 1] + x0 * sn[j >> 1]);
            }
            *(u16x8 *)(qs + rw * KSTR + d0) = out;
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));   /* the wave's own LDS writes, read by its other lanes */
#pragma unroll
        for (int ds = 0; ds < 8; ds++) qf[ds] = *(const bf16x8 *)(qs + lr * KSTR + (ds * 2 + lg) * 8);
    };
    if (FUSEQ) q_prologue();

    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[i][r] = 0.0f;
    /* running max of the lane's query column (same in both lanes of the column)
     * and this lane's partial row sum over its half of each tile's keys */
    float m_run = -1e30f, l_run = 0.0f;
    f32x16 s[2];
    bf16x8 pf[4];

    auto bar = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    /* PV of the tile in V stage vst: O^T += V^T P^T */
    auto pv = [&](int vst) {
        const uint16_t *vb = VBUF(vst);
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int dsub = 0; dsub < 4; dsub++) {
                const int d = dsub * 32 + lr;
                /* keys 16j + 4lg .. +3 and 16j + 8 + 4lg .. +3: the k order of pf[j] */
                bf16x8 vf;
                if constexpr (V16) {
                    vf = *(const bf16x8 *)(&vb[d * VSTR + 16 * j + 8 * lg]);
                } else {
                    const uint2 lo = *(const uint2 *)(&vb[d * VSTR + 16 * j + 4 * lg]);
                    const uint2 hi = *(const uint2 *)(&vb[d * VSTR + 16 * j + 8 + 4 * lg]);
                    vf = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
                }
                o[dsub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[j], o[dsub], 0, 0, 0);
            }
        }
    };
    /* S^T of the tile in K stage kst */
    auto qk = [&](int kst) {
        const uint16_t *kb = KBUF(kst);
#pragma unroll
        for (int ks = 0; ks < 2; ks++)
#pragma unroll
            for (int r = 0; r < 16; r++) s[ks][r] = 0.0f;
#pragma unroll
        for (int ds = 0; ds < 8; ds++) {
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const bf16x8 kf = *(const bf16x8 *)(&kb[(ks * 32 + lr) * KSTR + (ds * 2 + lg) * 8]);
                s[ks] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ds], s[ks], 0, 0, 0);
            }
        }
    };
    /* one wave issues the MFMAs of an M phase alone on its SIMD, so fragment
     * reads run 4 ahead of the products that use them: DS reads, then
     * alternating MFMA / DS read */
    auto interleave = [&](int n_mfma) {
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        for (int i = 0; i < n_mfma - 4; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    };

    /* V phase of tile t: masks, max, lazy rescale, P = exp2(S - m) as bf16
     * B-operand fragments, row sums */
    auto v_phase = [&](int t) {
        const int k0 = (t0 + t) * KB;
        const bool full = k0 + KB <= sk && ((k0 >= a.kv_lo0 && k0 + KB <= a.kv_hi0) ||
                                            (k0 >= a.kv_lo1 && k0 + KB <= a.kv_hi1)) &&
                          !(CAUSAL && k0 + KB - 1 > wave_q0);
        if (!full) {
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = k0 + ks * 32 + (r >> 2) * 8 + lg * 4 + (r & 3);
                    bool ok = (key < sk) & (((key >= a.kv_lo0) & (key < a.kv_hi0)) |
                                            ((key >= a.kv_lo1) & (key < a.kv_hi1)));
                    if (CAUSAL) ok = ok & (key <= q_row);
                    s[ks][r] = ok ? s[ks][r] : -INFINITY;
                }
        }
        if (BIAS && k0 + KB > a.bias_from) {
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
        {   /* max with the other half-wave's keys of the same query columns */
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
            mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * scale_log2;
        }
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
    };

    /* In its M(t) phase a group stages K(t+1) and V(t) from registers, loads
     * K(t+2) and V(t+1) (indices clamped to the last tile near the end: a
     * clamped K lands in a stage nothing reads again), then runs PV(t-1) and
     * QK(t). Group 0: M(0) V(0) M(1) ... V(nkt-1) M(nkt); group 1 one phase
     * later. Both execute 2 nkt + 3 barriers. */
    bar();   /* K(0) staged */
    if (grp) bar();
    if (nkt > 1) store_k(1);
    store_v(0);
    load_k(min(2, nkt - 1));
    if (nkt > 1) load_v(1);
    qk(0);
    bar();
    v_phase(0);
    bar();
    for (int t = 1; t < nkt; t++) {
        store_k((t + 1) & 1);
        store_v(t & 1);
        load_k(min(t + 2, nkt - 1));
        load_v(min(t + 1, nkt - 1));
        pv((t - 1) & 1);
        qk(t & 1);
        interleave(32);
        bar();
        v_phase(t);
        bar();
    }
    pv((nkt - 1) & 1);
    bar();
    if (!grp) bar();

    if ((FEAT & F_SPLIT) && sg.part) {
        /* a piece of the unit: store o, m, l at system coherence (written
         * through the XCDs' L2 caches, no cache-wide flush), count the
         * arrival; the last block to arrive merges the pieces in slot order */
        __shared__ int arrived;
        const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
            (void *)sp.ws, (short)0, (int)(sp.slots * SPLIT_SLOT_BYTES), 0x00020000);
        constexpr int COHERENT = 1 | 16;   /* sc0 | sc1 */
        const int o_end = sp.slots * NT * 64 * 4;
        auto o_off = [&](int slot, int i) { return ((slot * 16 + i) * NT + tid) * 16; };
        auto ml_off = [&](int slot) { return o_end + (slot * NT + tid) * 8; };
        const int slot = 2 * sg.s + (sg.first ? 0 : 1);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const f32x4 v = {o[i >> 2][(i & 3) * 4], o[i >> 2][(i & 3) * 4 + 1], o[i >> 2][(i & 3) * 4 + 2],
                             o[i >> 2][(i & 3) * 4 + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), wr, o_off(slot, i), 0, COHERENT);
        }
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, make_float2(m_run, l_run)), wr, ml_off(slot), 0,
                                              COHERENT);
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));   /* written through before the arrival is counted */
        __syncthreads();
        if (tid == 0) arrived = __hip_atomic_fetch_add(sp.cnt + L, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __syncthreads();
        const int j0 = split_slot_of(sp, L * sp.nkt), j1 = split_slot_of(sp, (L + 1) * sp.nkt - 1);
        if (arrived != j1 - j0) return;
        /* merged state: m = max m_j, o = sum o_j 2^(m_j - m), l likewise */
        float m_all = -INFINITY;
        for (int j = j0; j <= j1; j++) {
            const int sj = 2 * j + (split_start(sp, j) / sp.nkt == L ? 0 : 1);
            const float2 ml = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(wr, ml_off(sj), 0, COHERENT));
            m_all = fmaxf(m_all, ml.x);
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[i][r] = 0.0f;
        l_run = 0.0f;
        for (int j = j0; j <= j1; j++) {
            const int sj = 2 * j + (split_start(sp, j) / sp.nkt == L ? 0 : 1);
            const float2 ml = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(wr, ml_off(sj), 0, COHERENT));
            const float f = __builtin_amdgcn_exp2f(ml.x - m_all);
            l_run += ml.y * f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, o_off(sj, i), 0,
                                                                                                 COHERENT));
#pragma unroll
                for (int e = 0; e < 4; e++) o[i >> 2][(i & 3) * 4 + e] += v[e] * f;
            }
        }
        if (tid == 0) __hip_atomic_store(sp.cnt + L, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }

    /* normalise and store O[q][d]: lane holds query lr, d = dsub*32 + (r>>2)*8 + lg*4 + (r&3) */
    const float l = l_run + __shfl_xor(l_run, 32, 64);
    /* 16-byte stores need every batch slot's rows 16-byte aligned as well */
    if ((a.ld_o & 7) == 0 && ((uintptr_t)a.o & 15) == 0 && (a.batch == 1 || (a.o_bstride & 7) == 0)) {
        /* through LDS (every stage is free after the last barrier): the block's
         * 256 rows of 128 + 8 elements, then 16-byte chunks of whole rows, so a
         * store instruction writes 4 full rows instead of 16-byte pieces of 32 */
        constexpr int OSTR = HD + 8;
        static_assert(QB * OSTR <= QS_OFF, "the O tile fits the K and V stages");
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        uint16_t *const orow = smem + (wave * QW + lr) * OSTR;
#pragma unroll
        for (int dsub = 0; dsub < 4; dsub++)
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                u16x4 v;
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = f2bf(o[dsub][rb * 4 + e] * inv);
                *(u16x4 *)(orow + dsub * 32 + rb * 8 + lg * 4) = v;
            }
        __syncthreads();
        uint16_t *const Ob = O + (size_t)(qblk * QB) * a.ld_o;
        const int nrow = min(QB, sq - qblk * QB);
#pragma unroll
        for (int i = 0; i < QB * (HD / 8) / NT; i++) {
            const int c = tid + NT * i, row = c >> 4, ch = c & 15;
            if (row < nrow) *(uint4 *)(Ob + (size_t)row * a.ld_o + ch * 8) = *(const uint4 *)(smem + row * OSTR + ch * 8);
        }
    } else if (q_row < sq) {
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

template <int FEAT>
__global__ __launch_bounds__(NT) void flash_attn_kernel(const iris_attn_args_t a, float scale_log2, int nqb,
                                                        int per_xcd, int total, const AttnSplit sp) {
    if constexpr (!(FEAT & F_SPLIT)) {
        const int L = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
        if (L >= total) return;
        attn_segment<FEAT>(a, scale_log2, nqb, L, 0, -1, sp, AttnSeg{0, 0, 0});
    } else {
        const int s = (blockIdx.x & 7) * sp.bpx + (blockIdx.x >> 3), end = split_start(sp, s + 1);
        for (int it = split_start(sp, s), first = 1; it < end; first = 0) {
            const int unit = it / sp.nkt, t0 = it - unit * sp.nkt, tn = min(sp.nkt - t0, end - it);
            if (!first) __syncthreads();   /* the previous segment's LDS reads are done */
            attn_segment<FEAT>(a, scale_log2, nqb, unit, t0, tn, sp, AttnSeg{tn != sp.nkt, s, first});
            it += tn;
        }
    }
}

template <int FEAT>
int launch(const iris_attn_args_t *a, float scale_log2, int nqb, int per_xcd, int total, const AttnSplit &sp) {
    constexpr size_t smem = AttnLds<FEAT>::BYTES;
    static bool attr_set = false;
    if (!attr_set) {
        if (iris_check(hipFuncSetAttribute((const void *)flash_attn_kernel<FEAT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem),
                       "attention smem attribute"))
            return -1;
        attr_set = true;
    }
    static const char *const name[16] = {
        "flash_attn_kernel<0>",  "flash_attn_kernel<1>",  "flash_attn_kernel<2>",  "flash_attn_kernel<3>",
        "flash_attn_kernel<4>",  "flash_attn_kernel<5>",  "flash_attn_kernel<6>",  "flash_attn_kernel<7>",
        "flash_attn_kernel<8>",  "flash_attn_kernel<9>",  "flash_attn_kernel<10>", "flash_attn_kernel<11>",
        "flash_attn_kernel<12>", "flash_attn_kernel<13>", "flash_attn_kernel<14>", "flash_attn_kernel<15>"};
    const unsigned grid = (FEAT & F_SPLIT) ? 8u * sp.bpx : 8u * per_xcd;
    const int prof = iris_prof_begin(name[FEAT & 15], grid);
    hipLaunchKernelGGL(flash_attn_kernel<FEAT>, dim3(grid), dim3(NT), smem, iris_stream(), *a, scale_log2, nqb, per_xcd,
                       total, sp);
    iris_prof_end(prof);
    return iris_launch_check("flash_attn_kernel");
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
    const bool fuseq = a->qn_wA != nullptr;
    if (fuseq && (!a->qn_wB || ((uintptr_t)a->qn_wA | (uintptr_t)a->qn_wB | (uintptr_t)a->rope_cos |
                                (uintptr_t)a->rope_sin) & 15 || (a->rope_cos && !a->rope_sin)))
        return iris_set_error("attention: Q prologue needs both norm weight sets and 16-byte aligned tables");
    if (a->rope_pos && (!fuseq || !a->rope_axis || ((uintptr_t)a->rope_axis & 15) || a->rope_axis_len <= 0 ||
                        a->rope_axis_len > (1 << 15)))
        return iris_set_error("attention: factored RoPE needs the Q prologue, a 16-byte aligned table and "
                              "1 .. 32768 positions");
    const int nqb = (a->sq + QB - 1) / QB;
    const long long total = (long long)nqb * a->heads * a->batch;
    if (total > (1LL << 28)) return iris_set_error("attention: grid too large");
    const int per_xcd = (int)((total + 7) / 8);
    const float scale_log2 = a->scale * 1.4426950408889634f;
    int feat = (fuseq ? F_FUSEQ : 0) | (a->causal ? F_CAUSAL : 0) | (a->key_bias != 0.0f ? F_BIAS : 0);
    /* balanced schedule when one block per unit needs two or more rounds of
     * blocks (one per CU) that are on average less than 80 % full, and a
     * workspace is given. Merging the pieces' partial states goes through
     * memory at system coherence (128 KiB of o per piece) and every piece
     * repeats the Q prologue, so a single part-empty round stays one block per
     * unit (same box, 128-dim heads: 144 units of 1536 keys 47.3 us, 63.3 us
     * balanced, the idle CUs letting the busy ones clock higher), while 540
     * units of 4096 keys take 390.3 -> 356.6 us and 270 units 136.5 ->
     * 129.7 us balanced. */
    AttnSplit sp;
    memset(&sp, 0, sizeof(sp));
    const int cus = iris_cu_count(), nkt = (a->sk + KB - 1) / KB;
    if (!a->causal && a->ws && cus > 0 && cus % 8 == 0 && total <= SPLIT_MAX_UNITS &&
        a->ws_bytes >= iris_hip_attention_workspace_bytes()) {
        const long long rounds = (total + cus - 1) / cus;
        const long long steps = total * (long long)nkt;
        if (rounds >= 2 && (double)total < 0.8 * (double)(rounds * cus) && steps / cus >= 8 && steps < (1LL << 31)) {
            if (((uintptr_t)a->ws & 255)) return iris_set_error("attention: workspace must be 256-byte aligned");
            sp.nkt = nkt;
            sp.per = (int)(steps / cus);
            sp.rem = (int)(steps % cus);
            sp.bpx = cus / 8;
            sp.cnt = (int *)a->ws;
            sp.ws = (float *)((char *)a->ws + SPLIT_CNT_BYTES);
            sp.slots = 2 * cus;
            feat |= F_SPLIT;
        }
    }
    switch (feat) {
    case 0: return launch<0>(a, scale_log2, nqb, per_xcd, (int)total, sp);
    case F_FUSEQ: return launch<F_FUSEQ>(a, scale_log2, nqb, per_xcd, (int)total, sp);
    case F_CAUSAL: return launch<F_CAUSAL>(a, scale_log2, nqb, per_xcd, (int)total, sp);
    case F_FUSEQ | F_CAUSAL: return launch<F_FUSEQ | F_CAUSAL>(a, scale_log2, nqb, per_xcd, (int)total, sp);
    case F_BIAS: return launch<F_BIAS>(a, scale_log2, nqb, per_xcd, (int)total, sp);
    case F_FUSEQ | F_BIAS: return launch<F_FUSEQ | F_BIAS>(a, scale_log2, nqb, per_xcd, (int)total, sp);
    case F_SPLIT: return launch<F_SPLIT>(a, scale_log2, nqb, per_xcd, (int)total, sp);
    case F_FUSEQ | F_SPLIT: return launch<F_FUSEQ | F_SPLIT>(a, scale_log2, nqb, per_xcd, (int)total, sp);
    case F_BIAS | F_SPLIT: return launch<F_BIAS | F_SPLIT>(a, scale_log2, nqb, per_xcd, (int)total, sp);
    case F_FUSEQ | F_BIAS | F_SPLIT:
        return launch<F_FUSEQ | F_BIAS | F_SPLIT>(a, scale_log2, nqb, per_xcd, (int)total, sp);
    default: return iris_set_error("attention: causal masking with a key bias is not supported");
    }
}

extern "C" size_t iris_hip_attention_workspace_bytes(void) {
    if (!iris_hip_available()) return 0;
    return SPLIT_CNT_BYTES + 2 * (size_t)iris_cu_count() * SPLIT_SLOT_BYTES;
}
