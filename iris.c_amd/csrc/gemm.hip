/*
 * gemm.hip - bf16 x bf16 -> f32 MFMA GEMM for gfx950 with fused epilogues.
 *
 * Replaces the reference's linears (LINEAR_BF16_OR_F32 -> iris_linear ->
 * cblas_sgemm, iris_transformer_flux.c:121-131, iris_kernels.c:220-290) and the
 * elementwise passes that follow them (gated_add :136-143, iris_silu_mul
 * iris_kernels.c:626-638, the split/concat copies :3833-3840, :3897-3902).
 *
 * out = A[M,K] . W[N,K]^T. Block tile 256x256x64 with 512 threads = 8 waves in
 * a 4x2 arrangement (2 waves per SIMD, so one wave's MFMAs run while the other
 * waits on LDS or on a load's issue); each wave owns 64x128 as 2x4
 * v_mfma_f32_32x32x16_bf16 tiles and reads the next 16-wide K slice's operand
 * fragments from LDS while the current slice's MFMAs run.
 *
 * A and W stream through two 64 KiB LDS stages filled by LDS-DMA
 * (buffer_load ... lds): global data goes straight into LDS, with no staging
 * registers and no ds_write, whose data FIFO limited the register-staged
 * version. Each row of a stage is a full 128-byte line of the operand, so
 * every request to HBM fetches whole lines. The stages are separate
 * __shared__ objects, which lets the compiler wait only for the DMA of the
 * stage it reads. LDS serves a 16-byte-per-lane read 16 lanes at a time over
 * 64 banks: a group reads rows r..r+15 at one logical 16-byte chunk, and XOR
 * with (row / 2) mod 8 puts those rows on 16 distinct (row parity, chunk)
 * bank groups.
 *
 * Loads use buffer resources whose range ends at the operand's last valid row,
 * so rows past M (or N) read as zero without predicates. Blocks are mapped
 * XCD-major: block b runs on XCD b % 8 and takes a contiguous range of tiles,
 * ordered in groups of 8 M-tiles, so concurrently running blocks of one XCD
 * share A and W panels in that XCD's L2.
 */
#include "iris_internal.h"

#include <string.h>

namespace {

constexpr int BM = 256, BN = 256, BK = 64, NT = 512;
constexpr int WAVES_M = 4, WAVES_N = 2, TW_M = BM / WAVES_M, TW_N = BN / WAVES_N;
constexpr int FM = TW_M / 32, FN = TW_N / 32;
constexpr int TILE_ELEMS = BM * BK;                 /* A tile = W tile = 16384 bf16 */
constexpr int NWAVES = NT / 64;
constexpr int DMA_ROWS = 8;                         /* rows of one 64-lane x 16-byte LDS-DMA load */
constexpr int DMA_PER_OPND = BM / DMA_ROWS / NWAVES; /* per wave per operand per K-step = 4 */
constexpr int GROUP_M = 8;
constexpr int MAXP = 4;

struct GemmParams {
    iris_gemm_problem_t p[MAXP];
    int tiles_m[MAXP], tiles_n[MAXP], tile_start[MAXP + 1];
    int nprob, total, per_xcd;
};

__device__ __forceinline__ int swz(int row, int chunk) {   /* element offset in a tile */
    return row * BK + ((chunk ^ ((row >> 1) & 7)) << 3);
}

/* s_waitcnt immediate: vmcnt in bits 3:0 and 15:14, expcnt 6:4 (no wait),
 * lgkmcnt 11:8 */
constexpr int waitcnt_imm(int vm, int lgkm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8); }

typedef __attribute__((address_space(3))) void lds_void;

__global__ __launch_bounds__(NT) void gemm_bf16_kernel(const GemmParams P) {
    /* two stages, each an A tile then a W tile; separate objects so the
     * compiler tracks the LDS-DMA writes of one stage apart from reads of
     * the other */
    __shared__ __attribute__((aligned(16))) uint16_t lds0[2 * TILE_ELEMS];
    __shared__ __attribute__((aligned(16))) uint16_t lds1[2 * TILE_ELEMS];
    const int b = blockIdx.x;
    const int L = (b & 7) * P.per_xcd + (b >> 3);
    if (L >= P.total) return;
    int pi = 0;
#pragma unroll
    for (int i = 1; i < MAXP; i++)
        if (i < P.nprob && L >= P.tile_start[i]) pi = i;
    const iris_gemm_problem_t pr = P.p[pi];
    const int t = L - P.tile_start[pi];
    const int tmc = P.tiles_m[pi], tnc = P.tiles_n[pi];
    const int group = t / (GROUP_M * tnc);
    const int first_m = group * GROUP_M;
    const int gsz = min(tmc - first_m, GROUP_M);
    const int tm = first_m + (t % (GROUP_M * tnc)) % gsz;
    const int tn = (t % (GROUP_M * tnc)) / gsz;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int lr = lane & 31, lg = lane >> 5;

    /* LDS-DMA: load j of an operand covers tile rows 8j..8j+7 and writes
     * 1 KiB at byte j*1024 of the operand's tile, lane l at + 16l, i.e. row
     * 8j + l/8, stored chunk l%8. The lane fetches the global chunk that the
     * swizzle puts there: chunk (l%8) ^ ((row >> 1) & 7), which depends on j
     * only through j's parity. Rows past M (N) read as zero through the
     * buffer range. */
    const uint16_t *a_base = pr.A + (size_t)m0 * pr.lda;
    const uint16_t *w_base = pr.W + (size_t)n0 * pr.ldw;
    const int a_rows = min(BM, pr.M - m0), w_rows = min(BN, pr.N - n0);
    const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a_base, (short)0, a_rows * pr.lda * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)w_base, (short)0, w_rows * pr.ldw * 2, 0x00020000);
    const int drow = lane >> 3, dch = lane & 7;
    int a_voff[2], w_voff[2];
#pragma unroll
    for (int par = 0; par < 2; par++) {
        const int c = dch ^ ((4 * par + (drow >> 1)) & 7);
        const int row = wave * DMA_PER_OPND * DMA_ROWS + drow;    /* first load of this wave */
        a_voff[par] = (row * pr.lda + c * 8) * 2;
        w_voff[par] = (row * pr.ldw + c * 8) * 2;
    }
    const int a_step = DMA_ROWS * pr.lda * 2, w_step = DMA_ROWS * pr.ldw * 2;
    auto dma = [&](uint16_t *stage, int kt) {
        const int k0 = kt * BK * 2;
#pragma unroll
        for (int i = 0; i < DMA_PER_OPND; i++) {
            const int j = wave * DMA_PER_OPND + i;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_void *)(stage + j * 512), 16,
                                                     a_voff[i & 1] + i * a_step, k0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_void *)(stage + TILE_ELEMS + j * 512), 16,
                                                     w_voff[i & 1] + i * w_step, k0, 0, 0);
        }
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int nk = pr.K / BK;
    bf16x8 a[2][FM], w[2][FN];
    auto frag = [&](const uint16_t *stage, int kk, int buf) {
        const uint16_t *As = stage;
        const uint16_t *Ws = stage + TILE_ELEMS;
        const int ch = kk * 2 + lg;
#pragma unroll
        for (int mi = 0; mi < FM; mi++) a[buf][mi] = *(const bf16x8 *)(As + swz(wm * TW_M + mi * 32 + lr, ch));
#pragma unroll
        for (int ni = 0; ni < FN; ni++) w[buf][ni] = *(const bf16x8 *)(Ws + swz(wn * TW_N + ni * 32 + lr, ch));
    };
    auto mfmas = [&](int buf) {
#pragma unroll
        for (int mi = 0; mi < FM; mi++)
#pragma unroll
            for (int ni = 0; ni < FN; ni++)
                acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[buf][mi], w[buf][ni], acc[mi][ni], 0, 0, 0);
    };
    /* FM + FN fragment reads spread over FM * FN MFMAs */
    auto sched_reads = [&]() {
#pragma unroll
        for (int i = 0; i < FM + FN; i++) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - (FM + FN), 0);
    };

    /* K-step t reads stage t&1. Slice 0 of the step is read during slice 3
     * of the previous step; slices 1..3 one slice ahead of their MFMAs. The
     * DMA of tile t+1 into the other stage was issued in slice 3 of step t-1;
     * before slice 3 each wave waits for its own DMA and its LDS reads, and the
     * barrier makes the whole tile visible and the current stage free, so
     * slice 3 issues the DMA of tile t+2 into the current stage and reads
     * slice 0 of tile t+1. Past the last tile the DMA repeats tile nk-1 into a
     * stage nothing reads. */
    auto kstep = [&](uint16_t *cur, uint16_t *nxt, int kt) {
        frag(cur, 1, 1);
        mfmas(0);
        sched_reads();
        frag(cur, 2, 0);
        mfmas(1);
        sched_reads();
        frag(cur, 3, 1);
        mfmas(0);
        sched_reads();
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
        __builtin_amdgcn_s_barrier();
        dma(cur, min(kt + 2, nk - 1));
        frag(nxt, 0, 0);
        mfmas(1);
#pragma unroll
        for (int i = 0; i < FM + FN; i++) {
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x020, 2 * DMA_PER_OPND - (FM + FN), 0);
        __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - (FM + FN), 0);
    };

    dma(lds0, 0);
    dma(lds1, min(1, nk - 1));
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * DMA_PER_OPND, 15));   /* tile 0 landed */
    __builtin_amdgcn_s_barrier();
    frag(lds0, 0, 0);
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
        kstep(lds0, lds1, kt);
        kstep(lds1, lds0, kt + 1);
    }
    if (kt < nk) kstep(lds0, lds1, kt);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));   /* no DMA outstanding at exit */

    /* ---- epilogue: lane holds column lr of each 32x32 tile, rows
     *      (r>>2)*8 + lg*4 + (r&3) ---- */
    const int M = pr.M, N = pr.N, ldo = pr.ldo;
    const float *vec = pr.vec;
    const int row0 = m0 + wm * TW_M;
    /* interior tiles skip the per-element bounds checks */
    if (m0 + BM <= M && n0 + BN <= N) {
        switch (pr.epi) {
        case IRIS_EPI_F32:
        case IRIS_EPI_BF16:
        case IRIS_EPI_GATED_ADD: {
#pragma unroll
            for (int ni = 0; ni < FN; ni++) {
                const int col = n0 + wn * TW_N + ni * 32 + lr;
                const float v = vec ? vec[col] : (pr.epi == IRIS_EPI_GATED_ADD ? 1.0f : 0.0f);
#pragma unroll
                for (int mi = 0; mi < FM; mi++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const size_t o = (size_t)(row0 + mi * 32 + (r >> 2) * 8 + lg * 4 + (r & 3)) * ldo + col;
                        const float x = acc[mi][ni][r];
                        if (pr.epi == IRIS_EPI_F32) ((float *)pr.out)[o] = x + v;
                        else if (pr.epi == IRIS_EPI_BF16) ((uint16_t *)pr.out)[o] = f2bf_hw(x + v);
                        else ((float *)pr.out)[o] += v * x;
                    }
            }
            return;
        }
        case IRIS_EPI_SWIGLU: {
#pragma unroll
            for (int g = 0; g < FN / 2; g++) {
                const int col = ((n0 + wn * TW_N + g * 64) >> 1) + lr;
#pragma unroll
                for (int mi = 0; mi < FM; mi++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int row = row0 + mi * 32 + (r >> 2) * 8 + lg * 4 + (r & 3);
                        const float gt = acc[mi][2 * g][r], up = acc[mi][2 * g + 1][r];
                        ((uint16_t *)pr.out)[(size_t)row * ldo + col] = f2bf_hw(silu_fast(gt) * up);
                    }
            }
            return;
        }
        default:
            break;
        }
    }
    switch (pr.epi) {
    case IRIS_EPI_F32:
    case IRIS_EPI_BF16:
    case IRIS_EPI_GATED_ADD: {
#pragma unroll
        for (int ni = 0; ni < FN; ni++) {
            const int col = n0 + wn * TW_N + ni * 32 + lr;
            if (col >= N) continue;
            const float v = vec ? vec[col] : (pr.epi == IRIS_EPI_GATED_ADD ? 1.0f : 0.0f);
#pragma unroll
            for (int mi = 0; mi < FM; mi++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = row0 + mi * 32 + (r >> 2) * 8 + lg * 4 + (r & 3);
                    if (row >= M) continue;
                    const size_t o = (size_t)row * ldo + col;
                    const float x = acc[mi][ni][r];
                    if (pr.epi == IRIS_EPI_F32) ((float *)pr.out)[o] = x + v;
                    else if (pr.epi == IRIS_EPI_BF16) ((uint16_t *)pr.out)[o] = f2bf_hw(x + v);
                    else ((float *)pr.out)[o] += v * x;
                }
        }
        break;
    }
    case IRIS_EPI_SWIGLU: {
        /* each 64 columns of the wave are one interleaved group: tile 2g = 32
         * gate rows, tile 2g+1 = the matching 32 up rows; output column =
         * group * 32 + lr */
#pragma unroll
        for (int g = 0; g < FN / 2; g++) {
            const int col = ((n0 + wn * TW_N + g * 64) >> 1) + lr;
            if (col >= (N >> 1)) continue;
#pragma unroll
            for (int mi = 0; mi < FM; mi++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = row0 + mi * 32 + (r >> 2) * 8 + lg * 4 + (r & 3);
                    if (row >= M) continue;
                    const float gt = acc[mi][2 * g][r], up = acc[mi][2 * g + 1][r];
                    ((uint16_t *)pr.out)[(size_t)row * ldo + col] = f2bf_hw(silu_fast(gt) * up);
                }
        }
        break;
    }
    case IRIS_EPI_F32_T: {
#pragma unroll
        for (int ni = 0; ni < FN; ni++) {
            const int col = n0 + wn * TW_N + ni * 32 + lr;
            if (col >= N) continue;
            const float v = vec ? vec[col] : 0.0f;
#pragma unroll
            for (int mi = 0; mi < FM; mi++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = row0 + mi * 32 + (r >> 2) * 8 + lg * 4 + (r & 3);
                    if (row < M) ((float *)pr.out)[(size_t)col * ldo + row] = acc[mi][ni][r] + v;
                }
        }
        break;
    }
    default:
        break;
    }
}

}  // namespace

extern "C" int iris_hip_gemm(const iris_gemm_problem_t *probs, int n) {
    if (n < 1 || n > MAXP) return iris_set_error("gemm: %d problems (1..%d)", n, MAXP);
    GemmParams P;
    memset(&P, 0, sizeof(P));
    P.nprob = n;
    int total = 0;
    for (int i = 0; i < n; i++) {
        const iris_gemm_problem_t &p = probs[i];
        P.p[i] = p;
        P.tile_start[i] = total;
        if (p.M <= 0 || p.N <= 0) { P.tiles_m[i] = P.tiles_n[i] = 0; continue; }
        if (p.K <= 0 || p.K % BK) return iris_set_error("gemm: K=%d must be a positive multiple of %d", p.K, BK);
        if (p.lda % 8 || p.ldw % 8 || p.lda < p.K || p.ldw < p.K)
            return iris_set_error("gemm: lda=%d ldw=%d must be multiples of 8 and >= K=%d", p.lda, p.ldw, p.K);
        if (((uintptr_t)p.A | (uintptr_t)p.W) & 15) return iris_set_error("gemm: A/W must be 16-byte aligned");
        if (!p.A || !p.W || !p.out) return iris_set_error("gemm: null operand");
        if (p.epi == IRIS_EPI_SWIGLU && (p.N % 64)) return iris_set_error("gemm: SwiGLU needs N %% 64 == 0");
        if (p.epi < 0 || p.epi > IRIS_EPI_F32_T) return iris_set_error("gemm: epilogue %d", p.epi);
        const int ldo_need = p.epi == IRIS_EPI_SWIGLU ? p.N / 2 : p.epi == IRIS_EPI_F32_T ? p.M : p.N;
        if (p.ldo < ldo_need) return iris_set_error("gemm: ldo=%d < %d", p.ldo, ldo_need);
        /* 32-bit buffer offsets: one tile's rows must span < 2 GiB */
        if ((long long)BM * p.lda * 2 >= (1LL << 31) || (long long)BN * p.ldw * 2 >= (1LL << 31))
            return iris_set_error("gemm: leading dimension too large");
        P.tiles_m[i] = (p.M + BM - 1) / BM;
        P.tiles_n[i] = (p.N + BN - 1) / BN;
        total += P.tiles_m[i] * P.tiles_n[i];
    }
    for (int i = n; i <= MAXP; i++) P.tile_start[i] = total;
    if (total == 0) return 0;
    P.total = total;
    P.per_xcd = (total + 7) / 8;
    hipLaunchKernelGGL(gemm_bf16_kernel, dim3(8 * P.per_xcd), dim3(NT), 0, iris_stream(), P);
    return iris_launch_check("gemm_bf16_kernel");
}
