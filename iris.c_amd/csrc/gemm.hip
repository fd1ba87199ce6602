/*
 * gemm.hip - bf16 x bf16 -> f32 MFMA GEMM for gfx950 with fused epilogues.
 *
 * Replaces the reference's linears (LINEAR_BF16_OR_F32 -> iris_linear ->
 * cblas_sgemm, iris_transformer_flux.c:121-131, iris_kernels.c:220-290) and the
 * elementwise passes that follow them (gated_add :136-143, iris_silu_mul
 * iris_kernels.c:626-638, the split/concat copies :3833-3840, :3897-3902).
 * The same kernel body also runs the VAE's implicit-GEMM 3x3 convolutions
 * (iris_vae.c:203-251) and the row softmax of its bottleneck attention in the
 * epilogues of two passes over the score product (iris_vae.c:320-335).
 *
 * out = A[M,K] . W[N,K]^T. Block tile 256x256x64 with 512 threads = 8 waves in
 * a 4x2 arrangement; each wave owns 64x128 as 4x8 v_mfma_f32_16x16x32_bf16
 * tiles (narrower block tiles: 256x224 for plain GEMMs whose last round of
 * 256-wide tiles would be part-empty, 256x128 for convolutions of at most
 * 128 output channels). The 16x16x32 form does the same work per LDS byte as 32x32x16 and,
 * with the chip at its power limit on random data, sustains about 10 % more
 * MFMA throughput.
 *
 * Waves w and w+4 share a SIMD. The two groups (waves 0..3, waves 4..7) run
 * ping-pong: separated by block barriers, one group reads a whole 64-wide K
 * step of operand fragments from LDS and issues loads while the other runs
 * that step's 64 MFMAs, so every SIMD always has a wave issuing MFMAs and no
 * MFMA waits behind a load that is waiting for the address unit.
 *
 * A and W stream through two 64 KiB LDS stages filled by LDS-DMA
 * (buffer_load ... lds): global data goes straight into LDS, with no staging
 * registers and no ds_write. Each row of a stage is a full 128-byte line of
 * the operand, so every request to HBM fetches whole lines. The stages are
 * separate __shared__ objects, which lets the compiler wait only for the DMA
 * of the stage it reads. LDS serves a 16-byte-per-lane read 16 lanes at a
 * time over 64 banks: a group reads rows r..r+15 at one logical 16-byte chunk,
 * and XOR with (row / 2) mod 8 puts those rows on 16 distinct (row parity,
 * chunk) bank groups.
 *
 * Loads use buffer resources whose range ends at the operand's last valid row,
 * so rows past M (or N) read as zero without predicates. Blocks are mapped
 * XCD-major: block b runs on XCD b % 8 and takes a contiguous range of tiles,
 * ordered in groups of 8 M-tiles, so concurrently running blocks of one XCD
 * share A and W panels in that XCD's L2.
 */
#include "iris_internal.h"

#include <algorithm>
#include <mutex>
#include <string.h>

namespace {

constexpr int BM = 256, BN = 256, BK = 64, NT = 512;
constexpr int WAVES_M = 4, WAVES_N = 2, TW_M = BM / WAVES_M;
constexpr int FM = TW_M / 16;
constexpr int TILE_ELEMS = BM * BK;                 /* A tile = W tile = 16384 bf16 */
constexpr int DMA_ROWS = 8;                         /* rows of one 64-lane x 16-byte LDS-DMA load */
constexpr int GROUP_M = 8;
constexpr int MAXP = 4;

struct GemmParams {
    iris_gemm_problem_t p[MAXP];
    int tiles_m[MAXP], tiles_n[MAXP], tile_start[MAXP + 1];
    int nprob, total, per_xcd;
    /* split-K: problem i with chunks[i] > 1 has tiles_m[i] * tiles_n[i] *
     * chunks[i] blocks; block t of it works on K chunk t / (tiles_m * tiles_n)
     * (kchunk[i] elements) and writes its f32 partial product to
     * ws[i] + chunk * ws_stride[i] (M x N, row stride N) */
    int chunks[MAXP], kchunk[MAXP];
    float *ws[MAXP];
    long long ws_stride[MAXP];
    /* two-phase launch: blocks [0, phase_blocks) take tiles [0, phase_tiles)
     * (phase_blocks = 8 ceil(phase_tiles / 8), XCD-major over that range),
     * the blocks after them tiles [phase_tiles, total) (XCD-major, per_xcd
     * each), so the tiles of the first phase are dispatched before any of the
     * second's. 0: one phase. */
    int phase_tiles, phase_blocks;
    /* implicit 3x3 convolution (one problem, CONV kernels only): A is the bf16
     * NHWC input of (conv_h >> up) x (conv_w >> up) pixels, 2^cin_bshift bytes
     * per pixel; output row m is pixel (m / conv_w, m % conv_w) and K index
     * tap * cin + c reads channel c of the pixel at offset
     * (tap / 3 - 1, tap % 3 - 1) */
    int conv_h, conv_w, conv_up, conv_cpt_shift, conv_cin_bshift;
    unsigned conv_in_bytes;
    /* GroupNorm statistics of a convolution's output (CONV kernels, no
     * split-K): per row tile and group, sum and sum of squares in f64 */
    double *gn_part;
    int gn_groups;
    /* row softmax of scaled products (MODES 4, 5; one problem): s = sm_scale
     * * acc in log2 units, columns past N excluded. MODE 4: per row and tile,
     * (max s, sum 2^(s - max)) into sm_stat[row * tiles_n + tile column];
     * MODE 5: bf16 2^(s - sm_row[row].x) * sm_row[row].y into out, and zeros
     * in columns N .. sm_pad - 1 */
    float sm_scale;
    float2 *sm_stat;
    const float2 *sm_row;
    int sm_pad;
};

__device__ __forceinline__ int swz(int row, int chunk) {   /* element offset in a tile */
    return row * BK + ((chunk ^ ((row >> 1) & 7)) << 3);
}

/* s_waitcnt immediate: vmcnt in bits 3:0 and 15:14, expcnt 6:4 (no wait),
 * lgkmcnt 11:8 */
constexpr int waitcnt_imm(int vm, int lgkm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8); }

typedef __attribute__((address_space(3))) void lds_void;

/* element offset of (row, col) in a staged output half of OC columns: rows
 * padded by 16 bytes, or for 256 columns (a full 64 KiB stage) with the
 * 16-byte chunk index XORed with row % 16 */
template <int OC> __device__ __forceinline__ int opos(int row, int col) {
    if constexpr (OC == 256) return row * 256 + ((((col >> 3) ^ (row & 15)) << 3) | (col & 7));
    else return row * (OC + 8) + col;
}

/* bf16 epilogue of a whole tile through LDS (the caller has checked that the
 * tile is in range and the output rows 16-byte aligned). Group g (rows
 * GR g .. GR g + GR - 1, GR = 128 for 256-row tiles) stages its rows in
 * stage g. SWIGLU: accumulator
 * columns are 32-row gate / up groups, OC = half the tile width. */
template <int OC, bool SWIGLU, int FM_, int FNT_>
__device__ __forceinline__ void stage_out(const f32x4 (&acc)[FM_][FNT_], uint16_t *lds0, uint16_t *lds1,
                                          const iris_gemm_problem_t &pr, const float *vec, int m0, int oc0, int wm,
                                          int wn, int twn) {
    static_assert(128 * (OC == 256 ? 256 : OC + 8) * 2 <= 2 * TILE_ELEMS * 2, "a staged half fits one stage");
    constexpr int CPR = OC / 8; /* 16-byte chunks per row */
    constexpr int GR = 32 * FM_; /* rows of a wave group: 2 waves of 16 FM_ rows */
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
    const int grp = (tid >> 6) >> 2;
    uint16_t *const st = grp ? lds1 : lds0;
    const int hrow = (wm & 1) * (16 * FM_) + lr;
    __syncthreads(); /* every wave is done with the K loop's stages */
    if constexpr (SWIGLU) {
#pragma unroll
        for (int g = 0; g < FNT_ / 4; g++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int col = ((wn * twn + g * 64) >> 1) + h * 16 + lg * 4;
#pragma unroll
                for (int mi = 0; mi < FM_; mi++) {
                    const f32x4 gt = acc[mi][4 * g + h], up = acc[mi][4 * g + 2 + h];
                    uint16_t y[4];
#pragma unroll
                    for (int r = 0; r < 4; r++) y[r] = f2bf_hw(silu_fast(gt[r]) * up[r]);
                    *(uint2 *)(st + opos<OC>(hrow + mi * 16, col)) =
                        make_uint2((uint32_t)y[0] | ((uint32_t)y[1] << 16), (uint32_t)y[2] | ((uint32_t)y[3] << 16));
                }
            }
    } else {
#pragma unroll
        for (int ni = 0; ni < FNT_; ni++) {
            const int col = wn * twn + ni * 16 + lg * 4;
            float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (vec) {
                const float4 t = *(const float4 *)(vec + oc0 + col);
                v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
            }
#pragma unroll
            for (int mi = 0; mi < FM_; mi++) {
                const f32x4 x = acc[mi][ni];
                *(uint2 *)(st + opos<OC>(hrow + mi * 16, col)) =
                    make_uint2((uint32_t)f2bf_hw(x[0] + v[0]) | ((uint32_t)f2bf_hw(x[1] + v[1]) << 16),
                               (uint32_t)f2bf_hw(x[2] + v[2]) | ((uint32_t)f2bf_hw(x[3] + v[3]) << 16));
            }
        }
    }
    __syncthreads();
    uint16_t *const out = (uint16_t *)pr.out + (size_t)(m0 + GR * grp) * pr.ldo + oc0;
    const int gt = tid & 255;
#pragma unroll
    for (int i = 0; i < GR * CPR / 256; i++) {
        const int c = gt + 256 * i, row = c / CPR, ch = c - row * CPR;
        *(uint4 *)(out + (size_t)row * pr.ldo + ch * 8) = *(const uint4 *)(st + opos<OC>(row, ch * 8));
    }
}

/* The epilogues of MODES 4 and 5 (the products of one query block against
 * the keys of one 256-wide tile): per-row statistics of the tile (STATS), or
 * the probabilities. Lane l holds row lr of each 16x16 tile at columns
 * lg*4 .. lg*4+3; a row's 256 columns are spread over the 4 lanes lr + 16j of
 * a wave and the 2 waves across N. */
template <bool STATS, int FNT_>
__device__ __forceinline__ void softmax_epilogue(f32x4 (&acc)[FM][FNT_], const GemmParams &P,
                                                 const iris_gemm_problem_t &pr, int m0, int n0, int tn, int wm, int wn,
                                                 uint16_t *lds0, uint16_t *lds1) {
    constexpr int TWN_ = FNT_ * 16, BNT_ = TWN_ * WAVES_N;
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
    const int M = pr.M, N = pr.N;
    const int rowb = m0 + wm * TW_M + lr, colb = n0 + wn * TWN_ + lg * 4;
    /* scaled scores in place; columns past N hold -inf (2^-inf = 0) */
#pragma unroll
    for (int mi = 0; mi < FM; mi++)
#pragma unroll
        for (int ni = 0; ni < FNT_; ni++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                acc[mi][ni][r] = colb + ni * 16 + r < N ? acc[mi][ni][r] * P.sm_scale : -INFINITY;
    if constexpr (STATS) {
        /* the tile's row max, then its row sum of 2^(s - max): lane, the
         * row's 4 lanes (xor 16, 32), the 2 waves across N (in LDS) */
        __shared__ float red[2][WAVES_N][BM];
#pragma unroll
        for (int mi = 0; mi < FM; mi++) {
            float m = -INFINITY;
#pragma unroll
            for (int ni = 0; ni < FNT_; ni++)
                m = fmaxf(m, fmaxf(fmaxf(acc[mi][ni][0], acc[mi][ni][1]), fmaxf(acc[mi][ni][2], acc[mi][ni][3])));
            m = fmaxf(m, __shfl_xor(m, 16, 64));
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            if (lg == 0) red[0][wn][wm * TW_M + mi * 16 + lr] = m;
        }
        __syncthreads();
#pragma unroll
        for (int mi = 0; mi < FM; mi++) {
            const int rr = wm * TW_M + mi * 16 + lr;
            const float mt = fmaxf(red[0][0][rr], red[0][1][rr]);
            float l = 0.0f;
#pragma unroll
            for (int ni = 0; ni < FNT_; ni++)
#pragma unroll
                for (int r = 0; r < 4; r++) l += __builtin_amdgcn_exp2f(acc[mi][ni][r] - mt);
            l += __shfl_xor(l, 16, 64);
            l += __shfl_xor(l, 32, 64);
            if (lg == 0) red[1][wn][rr] = l;
        }
        __syncthreads();
        if (tid < BM && m0 + tid < M)
            P.sm_stat[(size_t)(m0 + tid) * P.tiles_n[0] + tn] =
                make_float2(fmaxf(red[0][0][tid], red[0][1][tid]), red[1][0][tid] + red[1][1][tid]);
        return;
    } else {
#pragma unroll
        for (int mi = 0; mi < FM; mi++) {
            const int row = rowb + mi * 16;
            const float2 rs = row < M ? P.sm_row[row] : make_float2(0.0f, 0.0f);
#pragma unroll
            for (int ni = 0; ni < FNT_; ni++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[mi][ni][r] = __builtin_amdgcn_exp2f(acc[mi][ni][r] - rs.x) * rs.y;
        }
        const int ldo = pr.ldo;
        if (m0 + BM <= M && n0 + BNT_ <= N && (ldo & 7) == 0 && ((uintptr_t)pr.out & 15) == 0) {
            stage_out<BNT_, false, FM, FNT_>(acc, lds0, lds1, pr, nullptr, m0, n0, wm, wn, TWN_);
            return;
        }
        /* edge tiles element by element, zeros in the padding columns */
#pragma unroll
        for (int mi = 0; mi < FM; mi++) {
            const int row = rowb + mi * 16;
            if (row >= M) continue;
#pragma unroll
            for (int ni = 0; ni < FNT_; ni++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int col = colb + ni * 16 + r;
                    if (col < P.sm_pad)
                        ((uint16_t *)pr.out)[(size_t)row * ldo + col] = col < N ? f2bf_hw(acc[mi][ni][r]) : (uint16_t)0;
                }
        }
    }
}

/* MODE 0: GEMM; 1: 3x3 convolution, stride 1, input optionally read through
 * a nearest 2x upsample; 2: 3x3 convolution, stride 2, right/bottom padding;
 * 3: GEMM with a second K segment (A2, W2) after the first; 4, 5: GEMMs
 * whose epilogue is a row softmax pass (softmax_epilogue: row statistics,
 * probabilities). The modes are
 * separate kernels: the load-issue phase has no cycles to spare for the
 * address arithmetic of the modes it does not run. */
template <int MODE, int BNT = BN, int BMT = BM>
__global__ __launch_bounds__(NT) void gemm_bf16_kernel(const GemmParams P) {
    constexpr bool CONV = MODE == 1 || MODE == 2, SEG2 = MODE == 3, SMX = MODE == 4 || MODE == 5;
    /* BNT: block tile width, 256, or (MODE 0, no SwiGLU) 224 = 2 waves x 7
     * MFMA tiles, for launches whose 256-wide tiles leave the last wave of
     * blocks part-empty, or (convolutions) 128 = 2 waves x 4 MFMA tiles for
     * outputs of at most 128 channels, which a 256-wide tile would compute
     * half empty */
    static_assert(BNT == BN || (BNT == 224 && MODE == 0) || (BNT == 128 && (MODE == 1 || MODE == 2)),
                  "narrow tiles are for plain GEMMs and convolutions");
    /* BMT: block tile height, 256, or 128 (plain GEMMs on few rows: twice
     * the tiles of a 256-row tile; wave tile 32 x 128) */
    static_assert(BMT == BM || (BMT == 128 && MODE == 0 && BNT == BN), "128-row tiles are for plain GEMMs");
    constexpr int TWN = BNT / WAVES_N, FNT = TWN / 16, W_DMA = BNT / DMA_ROWS / 4;
    constexpr int TWM = BMT / WAVES_M, FMT = TWM / 16, A_DMA = BMT / DMA_ROWS / 4;
    /* two stages, each an A tile then a W tile; separate objects so the
     * compiler tracks the LDS-DMA writes of one stage apart from reads of
     * the other */
    __shared__ __attribute__((aligned(16))) uint16_t lds0[2 * TILE_ELEMS];
    __shared__ __attribute__((aligned(16))) uint16_t lds1[2 * TILE_ELEMS];
    const int b = blockIdx.x;
    int L;
    if (b < P.phase_blocks) {
        L = (b & 7) * (P.phase_blocks >> 3) + (b >> 3);
        if (L >= P.phase_tiles) return;
    } else {
        const int b2 = b - P.phase_blocks;
        L = P.phase_tiles + (b2 & 7) * P.per_xcd + (b2 >> 3);
        if (L >= P.total) return;
    }
    int pi = 0;
#pragma unroll
    for (int i = 1; i < MAXP; i++)
        if (i < P.nprob && L >= P.tile_start[i]) pi = i;
    iris_gemm_problem_t pr = P.p[pi];
    int t = L - P.tile_start[pi];
    int kt0 = 0;   /* first K step of this block's chunk (split-K convolution) */
    if (P.chunks[pi] > 1) {
        const int per = P.tiles_m[pi] * P.tiles_n[pi];
        const int chunk = t / per;
        const int k0 = chunk * P.kchunk[pi];
        t -= chunk * per;
        if (CONV) kt0 = k0 / BK;
        else pr.A += k0;
        pr.W += k0;
        pr.K = min(P.kchunk[pi], pr.K - k0);
        pr.out = P.ws[pi] + chunk * P.ws_stride[pi];
        pr.ldo = pr.N;
        pr.vec = nullptr;
        pr.epi = IRIS_EPI_F32;
    }
    const int tmc = P.tiles_m[pi], tnc = P.tiles_n[pi];
    const int group = t / (GROUP_M * tnc);
    const int first_m = group * GROUP_M;
    const int gsz = min(tmc - first_m, GROUP_M);
    const int tm = first_m + (t % (GROUP_M * tnc)) % gsz;
    const int tn = (t % (GROUP_M * tnc)) / gsz;
    const int m0 = tm * BMT, n0 = tn * BNT;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    /* waves w and w + 4 share SIMD w: group 0 (waves 0..3) and group 1
     * (waves 4..7) alternate between an LDS phase and an MFMA phase */
    const int grp = wave >> 2, gw = wave & 3;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int lr = lane & 15, lg = lane >> 4;

    /* LDS-DMA: load j of an operand covers tile rows 8j..8j+7 and writes
     * 1 KiB at byte j*1024 of the operand's tile, lane l at + 16l, i.e. row
     * 8j + l/8, stored chunk l%8; the lane fetches global chunk
     * (l%8) ^ ((row >> 1) & 7), which depends on j only through its parity.
     * Group 0 loads the A tiles and group 1 the W tiles; wave gw of a group
     * issues A loads j = 8gw..8gw+7 and W loads j = W_DMA gw .. + W_DMA-1
     * (W_DMA = 7 for 224-wide tiles, where the parity of j is that of
     * gw + i). */
    const uint16_t *a_base = pr.A + (size_t)m0 * pr.lda;
    const uint16_t *w_base = pr.W + (size_t)n0 * pr.ldw;
    const int a_rows = min(BMT, pr.M - m0), w_rows = min(BNT, pr.N - n0);
    const __amdgpu_buffer_rsrc_t a_rsrc =
        CONV ? __builtin_amdgcn_make_buffer_rsrc((void *)pr.A, (short)0, (int)P.conv_in_bytes, 0x00020000)
             : __builtin_amdgcn_make_buffer_rsrc((void *)a_base, (short)0, a_rows * pr.lda * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)w_base, (short)0, w_rows * pr.ldw * 2, 0x00020000);
    const int drow = lane >> 3, dch = lane & 7;
    int a_voff[2], w_voff[2], a_chunk[2];
#pragma unroll
    for (int par = 0; par < 2; par++) {
        const int c = dch ^ ((4 * par + (drow >> 1)) & 7);
        const int row = gw * A_DMA * DMA_ROWS + drow;
        a_voff[par] = (row * pr.lda + c * 8) * 2;
        /* W: load i of wave gw is tile load j = W_DMA gw + i */
        const int cw = dch ^ ((4 * ((par + (W_DMA & 1) * gw) & 1) + (drow >> 1)) & 7);
        w_voff[par] = ((gw * W_DMA * DMA_ROWS + drow) * pr.ldw + cw * 8) * 2;
        a_chunk[par] = c * 16;
    }
    const int a_step = DMA_ROWS * pr.lda * 2, w_step = DMA_ROWS * pr.ldw * 2;
    /* second segment (MODE 3): the same lane layout over A2 / W2; a lane's
     * offset there is its first-segment offset + row * (ld2 - ld) * 2, formed
     * at each load from scalars chosen by the K step, so the two segments
     * share one load sequence and no registers are held for the second */
    const int nk1 = pr.K / BK;
    const int dma_row = gw * A_DMA * DMA_ROWS + drow;
    __amdgpu_buffer_rsrc_t a2_rsrc = a_rsrc, w2_rsrc = w_rsrc;
    if (SEG2) {
        a2_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)(pr.A2 + (size_t)m0 * pr.lda2), (short)0,
                                                    a_rows * pr.lda2 * 2, 0x00020000);
        w2_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)(pr.W2 + (size_t)n0 * pr.ldw2), (short)0,
                                                    w_rows * pr.ldw2 * 2, 0x00020000);
    }
    /* convolution: the output pixel of each row this lane loads, y << 16 | x;
     * rows past M get y = 0x4000, outside every image */
    uint32_t pix[A_DMA];
    if (CONV) {
#pragma unroll
        for (int i = 0; i < A_DMA; i++) {
            const int m = m0 + gw * A_DMA * DMA_ROWS + i * DMA_ROWS + drow;
            pix[i] = m < pr.M ? ((uint32_t)(m / P.conv_w) << 16) | (uint32_t)(m % P.conv_w) : 0x40000000u;
        }
    }
    auto dma_a = [&](uint16_t *stage, int kt) {
        if (CONV) {
            /* K step kt covers channels 64 * (kt mod cin/64) .. +63 of tap kt / (cin/64);
             * taps outside the image (zero padding) get an offset past the end of the
             * buffer, which reads as zero */
            const int kg = kt + kt0;
            const int tap = kg >> P.conv_cpt_shift;
            const int soff = (kg & ((1 << P.conv_cpt_shift) - 1)) * (BK * 2);
            const int ty = tap / 3;
            const int dy = ty - 1, dx = tap - 3 * ty - 1;
            /* MODE 1: input pixel ((y + dy) >> up, (x + dx) >> up); MODE 2 (stride 2,
             * zero padding on the right and bottom only): input pixel
             * (2y + dy + 1, 2x + dx + 1) of a (2 conv_h) x (2 conv_w) image */
            const int up = MODE == 1 ? P.conv_up : 0;
            const int hin = MODE == 2 ? 2 * P.conv_h : P.conv_h, win = MODE == 2 ? 2 * P.conv_w : P.conv_w;
            constexpr int mul = MODE == 2 ? 2 : 1, off = MODE == 2 ? 1 : 0;
#pragma unroll
            for (int i = 0; i < A_DMA; i++) {
                const int yy = (int)(pix[i] >> 16) * mul + dy + off, xx = (int)(pix[i] & 0xffffu) * mul + dx + off;
                const bool ok = (unsigned)yy < (unsigned)hin && (unsigned)xx < (unsigned)win;
                const int src = ((((yy >> up) * (win >> up)) + (xx >> up)) << P.conv_cin_bshift) + a_chunk[i & 1];
                __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_void *)(stage + (gw * A_DMA + i) * 512), 16,
                                                         ok ? src : (int)0x80000000u, soff, 0, 0);
            }
        } else if (SEG2) {
            const bool s2 = kt >= nk1;
            const __amdgpu_buffer_rsrc_t r = s2 ? a2_rsrc : a_rsrc;
            const int extra = s2 ? dma_row * ((pr.lda2 - pr.lda) * 2) : 0;
            const int step = s2 ? DMA_ROWS * pr.lda2 * 2 : a_step, ks = (s2 ? kt - nk1 : kt) * BK * 2;
#pragma unroll
            for (int i = 0; i < A_DMA; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)(stage + (gw * A_DMA + i) * 512), 16,
                                                         a_voff[i & 1] + extra + i * step, ks, 0, 0);
        } else {
#pragma unroll
            for (int i = 0; i < A_DMA; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (lds_void *)(stage + (gw * A_DMA + i) * 512),
                                                         16, a_voff[i & 1] + i * a_step, kt * BK * 2, 0, 0);
        }
    };
    auto dma_w = [&](uint16_t *stage, int kt) {
        if (SEG2) {
            const bool s2 = kt >= nk1;
            const __amdgpu_buffer_rsrc_t r = s2 ? w2_rsrc : w_rsrc;
            const int extra = s2 ? dma_row * ((pr.ldw2 - pr.ldw) * 2) : 0;
            const int step = s2 ? DMA_ROWS * pr.ldw2 * 2 : w_step, ks = (s2 ? kt - nk1 : kt) * BK * 2;
#pragma unroll
            for (int i = 0; i < W_DMA; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(r,
                                                         (lds_void *)(stage + TILE_ELEMS + (gw * W_DMA + i) * 512),
                                                         16, w_voff[i & 1] + extra + i * step, ks, 0, 0);
        } else {
#pragma unroll
            for (int i = 0; i < W_DMA; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc,
                                                         (lds_void *)(stage + TILE_ELEMS + (gw * W_DMA + i) * 512),
                                                         16, w_voff[i & 1] + i * w_step, kt * BK * 2, 0, 0);
        }
    };

    f32x4 acc[FMT][FNT];
#pragma unroll
    for (int i = 0; i < FMT; i++)
#pragma unroll
        for (int j = 0; j < FNT; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][j][r] = 0.0f;

    const int nk = (pr.K + (SEG2 ? pr.K2 : 0)) / BK;
    /* fragments of one K-step: two 32-wide slices */
    bf16x8 a[2][FMT], w[2][FNT];
    auto frags = [&](const uint16_t *stage) {
        const uint16_t *As = stage;
        const uint16_t *Ws = stage + TILE_ELEMS;
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            const int ch = kk * 4 + lg;
#pragma unroll
            for (int mi = 0; mi < FMT; mi++) a[kk][mi] = *(const bf16x8 *)(As + swz(wm * TWM + mi * 16 + lr, ch));
#pragma unroll
            for (int ni = 0; ni < FNT; ni++) w[kk][ni] = *(const bf16x8 *)(Ws + swz(wn * TWN + ni * 16 + lr, ch));
        }
    };
    auto mfmas = [&](int kk) {
#pragma unroll
            for (int mi = 0; mi < FMT; mi++)
#pragma unroll
                for (int ni = 0; ni < FNT; ni++)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w[kk][ni], a[kk][mi], acc[mi][ni], 0, 0, 0);
    };
/* explicit waits and barriers stay where they are written */
#define WAIT(vm, lgkm)                                              \
    do {                                                            \
        __builtin_amdgcn_sched_barrier(0);                          \
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(vm, lgkm));          \
        __builtin_amdgcn_sched_barrier(0);                          \
    } while (0)
    auto barrier = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    /* Barrier-separated phases; group 0 runs L(t), C(t) in phases 2t, 2t+1,
     * group 1 runs L(t), C(t) in phases 2t+1, 2t+2. L(t) reads tile t (stage
     * t&1) into registers, C(t) runs its MFMAs, so on every SIMD one wave
     * issues MFMAs while the other reads LDS. Loads are issued only in L
     * phases (a load waiting for the address unit holds up the instructions
     * behind it) and each group issues half of every tile:
     *  - group 0 issues A of tile t+1 in L(t): stage (t+1)&1 last held tile
     *    t-1, read by both groups before phase 2t; it waits for the loads at
     *    the end of C(t), before phase 2t+2 where tile t+1 is first read;
     *  - group 1 issues W of tile t+2 in L(t), into the stage it has just
     *    read. Two waves of the group read each W row, so the loads wait for
     *    a barrier in the middle of phase 2t+1 that every wave of the group
     *    reaches only after its reads of tile t have returned (group 0 read
     *    tile t in phase 2t and meets this barrier between the two halves of
     *    C(t)). Group 1 waits for the loads in L(t+1), before phase 2t+4.
     * Every wait is for all of a wave's loads: completions of LDS-DMA loads
     * are not ordered, so a partial count does not mean the oldest loads are
     * done. Past the last tile the loads repeat tile nk-1 into a stage
     * nothing reads again. */
    auto step0 = [&](uint16_t *cur, uint16_t *nxt, int kt) {
        frags(cur);
        dma_a(nxt, min(kt + 1, nk - 1));
        /* spread the loads over the fragment reads */
#pragma unroll
        for (int i = 0; i < A_DMA; i++) {
            __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
        WAIT(63, 0);
        barrier();
        mfmas(0);
        barrier();   /* group 1's reads of tile kt are done */
        mfmas(1);
        WAIT(0, 0);
        barrier();
    };
    auto step1 = [&](uint16_t *cur, int kt) {
        frags(cur);
        WAIT(0, 0);
        barrier();   /* every wave of the group has read tile kt */
        dma_w(cur, min(kt + 2, nk - 1));
        barrier();
        mfmas(0);
        mfmas(1);
        if (kt + 1 < nk) barrier();
    };

    if (grp) {
        dma_w(lds0, 0);
        WAIT(0, 0);
        barrier();
        dma_w(lds1, min(1, nk - 1));
        barrier();
        int kt = 0;
        for (; kt + 1 < nk; kt += 2) {
            step1(lds0, kt);
            step1(lds1, kt + 1);
        }
        if (kt < nk) step1(lds0, kt);
    } else {
        dma_a(lds0, 0);
        WAIT(0, 0);
        barrier();
        int kt = 0;
        for (; kt + 1 < nk; kt += 2) {
            step0(lds0, lds1, kt);
            step0(lds1, lds0, kt + 1);
        }
        if (kt < nk) step0(lds0, lds1, kt);
    }
    WAIT(0, 0);   /* no DMA outstanding at exit */
#undef WAIT
    if constexpr (SMX) {
        softmax_epilogue<MODE == 4, FNT>(acc, P, pr, m0, n0, tn, wm, wn, lds0, lds1);
        return;
    }

    /* ---- epilogue: W is the MFMAs' first operand, so lane l holds row lr of
     *      each 16x16 tile at the 4 consecutive columns lg*4 .. lg*4+3 ---- */
    const int M = pr.M, N = pr.N, ldo = pr.ldo;
    const float *vec = pr.vec;
    const int rowb = m0 + wm * TWM + lr;
    const int colb = n0 + wn * TWN + lg * 4;
    /* whole tile in range and 4-wide accesses aligned: one 8- or 16-byte
     * access per lane and 16x16 tile */
    const bool aligned = (ldo & 3) == 0 && ((uintptr_t)pr.out & 15) == 0 && ((uintptr_t)vec & 15) == 0;
    const bool full = m0 + BMT <= M && n0 + BNT <= N && aligned;
    /* GroupNorm statistics of a convolution's output: each lane sums the
     * values it writes per 4-channel chunk (one group: groups are multiples
     * of 4 channels), then the tile's sums per group are formed in a fixed
     * order below (the direct stores: the tile's values stay in registers) */
    const bool gn = CONV && P.gn_part != nullptr;
    float gs1[FNT], gs2[FNT];
#pragma unroll
    for (int ni = 0; ni < FNT; ni++) gs1[ni] = gs2[ni] = 0.0f;
    auto gn_add = [&](int ni, float y) {
        gs1[ni] += y;
        gs2[ni] += y * y;
    };
    /* Whole tiles of bf16 output (plain or SwiGLU) go out through LDS: each
     * group writes its 128 rows into one of the stages, now free, and then
     * stores them as 16-byte chunks of whole rows, so one store instruction
     * covers full 128-byte lines instead of 32-byte pieces of 16 rows (the
     * direct stores left the waves stalled on issue). */
    bool staged = false;
    if (full && (ldo & 7) == 0 && (pr.epi == IRIS_EPI_BF16 || (BNT == BN && pr.epi == IRIS_EPI_SWIGLU))) {
        if (gn) {   /* a convolution's bf16 tile: the sums of the values before rounding */
#pragma unroll
            for (int ni = 0; ni < FNT; ni++) {
                const float4 t = vec ? *(const float4 *)(vec + colb + ni * 16) : make_float4(0, 0, 0, 0);
#pragma unroll
                for (int mi = 0; mi < FMT; mi++) {
                    gn_add(ni, acc[mi][ni][0] + t.x);
                    gn_add(ni, acc[mi][ni][1] + t.y);
                    gn_add(ni, acc[mi][ni][2] + t.z);
                    gn_add(ni, acc[mi][ni][3] + t.w);
                }
            }
        }
        if (pr.epi == IRIS_EPI_SWIGLU) stage_out<BNT / 2, true, FMT, FNT>(acc, lds0, lds1, pr, vec, m0, n0 >> 1, wm, wn, TWN);
        else stage_out<BNT, false, FMT, FNT>(acc, lds0, lds1, pr, vec, m0, n0, wm, wn, TWN);
        if (!gn) return;
        staged = true;
    }
    if (!staged) switch (pr.epi) {
    case IRIS_EPI_F32:
    case IRIS_EPI_BF16:
    case IRIS_EPI_GATED_ADD:
    case IRIS_EPI_ADD: {
        const float vdef = pr.epi == IRIS_EPI_GATED_ADD ? 1.0f : 0.0f;
#pragma unroll
        for (int ni = 0; ni < FNT; ni++) {
            const int col = colb + ni * 16;
            /* a lane's 4 columns are all in range or (N % 4 == 0 aside) all out */
            const bool cols4 = full || (aligned && col + 3 < N);
            float v[4];
            if (cols4 && vec) {
                const float4 t = *(const float4 *)(vec + col);
                v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = vec && col + r < N ? vec[col + r] : vdef;
            }
#pragma unroll
            for (int mi = 0; mi < FMT; mi++) {
                const int row = rowb + mi * 16;
                const f32x4 x = acc[mi][ni];
                const size_t o = (size_t)row * ldo + col;
                if (full || (cols4 && row < M)) {
                    float4 y;
                    if (pr.epi == IRIS_EPI_F32) {
                        y = make_float4(x[0] + v[0], x[1] + v[1], x[2] + v[2], x[3] + v[3]);
                        *(float4 *)((float *)pr.out + o) = y;
                    } else if (pr.epi == IRIS_EPI_BF16) {
                        y = make_float4(x[0] + v[0], x[1] + v[1], x[2] + v[2], x[3] + v[3]);
                        uint2 p;
                        p.x = (uint32_t)f2bf_hw(y.x) | ((uint32_t)f2bf_hw(y.y) << 16);
                        p.y = (uint32_t)f2bf_hw(y.z) | ((uint32_t)f2bf_hw(y.w) << 16);
                        *(uint2 *)((uint16_t *)pr.out + o) = p;
                    } else if (pr.epi == IRIS_EPI_GATED_ADD) {
                        float4 *dst = (float4 *)((float *)pr.out + o);
                        y = *dst;
                        y.x += v[0] * x[0]; y.y += v[1] * x[1]; y.z += v[2] * x[2]; y.w += v[3] * x[3];
                        *dst = y;
                    } else {
                        float4 *dst = (float4 *)((float *)pr.out + o);
                        y = *dst;
                        y.x += x[0] + v[0]; y.y += x[1] + v[1]; y.z += x[2] + v[2]; y.w += x[3] + v[3];
                        *dst = y;
                    }
                    if (gn) {
                        gn_add(ni, y.x);
                        gn_add(ni, y.y);
                        gn_add(ni, y.z);
                        gn_add(ni, y.w);
                    }
                } else if (row < M) {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        if (col + r >= N) continue;
                        float *const f = (float *)pr.out + o + r;
                        float y = x[r] + v[r];
                        if (pr.epi == IRIS_EPI_F32) *f = y;
                        else if (pr.epi == IRIS_EPI_BF16) ((uint16_t *)pr.out)[o + r] = f2bf_hw(y);
                        else if (pr.epi == IRIS_EPI_GATED_ADD) *f = y = *f + v[r] * x[r];
                        else *f = y = *f + (x[r] + v[r]);
                        if (gn) gn_add(ni, y);
                    }
                }
            }
        }
        break;
    }
    case IRIS_EPI_SWIGLU:
        if constexpr (BNT == BN) {
            /* each 64 columns of the wave are one interleaved group: tiles 4g,
             * 4g+1 = 32 gate rows, tiles 4g+2, 4g+3 = the matching 32 up rows;
             * output columns = group * 32 + h * 16 + lg * 4 + (0..3) */
#pragma unroll
            for (int g = 0; g < FNT / 4; g++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int col = ((n0 + wn * TWN + g * 64) >> 1) + h * 16 + lg * 4;
#pragma unroll
                    for (int mi = 0; mi < FMT; mi++) {
                        const int row = rowb + mi * 16;
                        const f32x4 gt = acc[mi][4 * g + h], up = acc[mi][4 * g + 2 + h];
                        uint16_t y[4];
#pragma unroll
                        for (int r = 0; r < 4; r++) y[r] = f2bf_hw(silu_fast(gt[r]) * up[r]);
                        uint16_t *dst = (uint16_t *)pr.out + (size_t)row * ldo + col;
                        if (full) {
                            *(uint2 *)dst = make_uint2((uint32_t)y[0] | ((uint32_t)y[1] << 16),
                                                       (uint32_t)y[2] | ((uint32_t)y[3] << 16));
                        } else if (row < M) {
#pragma unroll
                            for (int r = 0; r < 4; r++)
                                if (col + r < (N >> 1)) dst[r] = y[r];
                        }
                    }
                }
        }
        break;
    case IRIS_EPI_F32_T: {
#pragma unroll
        for (int ni = 0; ni < FNT; ni++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int col = colb + ni * 16 + r;
                if (col >= N) continue;
                const float v = vec ? vec[col] : 0.0f;
#pragma unroll
                for (int mi = 0; mi < FMT; mi++) {
                    const int row = rowb + mi * 16;
                    if (row < M) ((float *)pr.out)[(size_t)col * ldo + row] = acc[mi][ni][r] + v;
                }
            }
        break;
    }
    default:
        break;
    }
    if constexpr (CONV) {
        if (gn) {
            /* per wave, the 16 lanes of a row hold one 4-channel chunk's 16
             * rows of each of the wave's 4 row blocks: the chunk's sums over
             * the wave's 64 rows, then over the tile's 4 waves in M and the
             * group's chunks in order, in f64 */
            __shared__ float gnl[WAVES_M * WAVES_N * FNT * 4 * 2];
#pragma unroll
            for (int ni = 0; ni < FNT; ni++) {
                const float s = row16_sum(gs1[ni]), q = row16_sum(gs2[ni]);
                if (lr == 0) {
                    float *d = gnl + (((wm * WAVES_N + wn) * FNT + ni) * 4 + lg) * 2;
                    d[0] = s;
                    d[1] = q;
                }
            }
            __syncthreads();
            const int G = P.gn_groups, cpg = N / G, t = threadIdx.x;
            if (t < BNT / cpg && n0 + t * cpg < N) {
                double s = 0.0, q = 0.0;
                for (int c = t * cpg; c < (t + 1) * cpg; c += 4) {
                    const int w = c % TWN;
                    for (int wm_ = 0; wm_ < WAVES_M; wm_++) {
                        const float *d = gnl + (((wm_ * WAVES_N + c / TWN) * FNT + w / 16) * 4 + (w % 16) / 4) * 2;
                        s += (double)d[0];
                        q += (double)d[1];
                    }
                }
                double *dst = P.gn_part + ((size_t)(m0 / BMT) * G + n0 / cpg + t) * 2;
                dst[0] = s;
                dst[1] = q;
            }
        }
    }
}

/* Split-K partials of up to MAXP problems, reduced in one launch: each
 * output element is the sum of its problem's partials in chunk order
 * (deterministic), then that problem's epilogue. A thread takes VW = vw[i]
 * consecutive output elements of a row (4 where the partial rows, the output
 * and the bias allow 16-byte accesses, else 1); each element gets the same
 * additions either way. */
struct ReduceParams {
    iris_gemm_problem_t p[MAXP];
    const float *ws[MAXP];
    long long stride[MAXP];
    int chunks[MAXP], vw[MAXP];
    long long start[MAXP + 1];   /* first work item of each problem; start[n] = all */
    int n;
};

__global__ void splitk_reduce_kernel(const ReduceParams R) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= R.start[R.n]) return;
    int pi = 0;
#pragma unroll
    for (int j = 1; j < MAXP; j++)
        if (j < R.n && i >= R.start[j]) pi = j;
    const iris_gemm_problem_t p = R.p[pi];
    const float *ws = R.ws[pi];
    const long long stride = R.stride[pi];
    const int splits = R.chunks[pi];
    const int nout = p.epi == IRIS_EPI_SWIGLU ? p.N / 2 : p.N;
    if (R.vw[pi] == 4) {
        const long long e = (i - R.start[pi]) * 4;
        const int m = (int)(e / nout), c = (int)(e % nout);
        if (p.epi == IRIS_EPI_SWIGLU) {
            /* W rows interleaved in 32-row gate / up groups; c % 4 == 0 keeps
             * the four columns in one group */
            const int gc = (c >> 5) * 64 + (c & 31);
            float4 g = make_float4(0.0f, 0.0f, 0.0f, 0.0f), u = g;
            for (int k = 0; k < splits; k++) {
                const float *row = ws + k * stride + (size_t)m * p.N;
                const float4 a = ld_stream((const float4 *)(row + gc)), b = ld_stream((const float4 *)(row + gc + 32));
                g.x += a.x; g.y += a.y; g.z += a.z; g.w += a.w;
                u.x += b.x; u.y += b.y; u.z += b.z; u.w += b.w;
            }
            *(uint2 *)((uint16_t *)p.out + (size_t)m * p.ldo + c) =
                make_uint2((uint32_t)f2bf_hw(silu_fast(g.x) * u.x) | ((uint32_t)f2bf_hw(silu_fast(g.y) * u.y) << 16),
                           (uint32_t)f2bf_hw(silu_fast(g.z) * u.z) | ((uint32_t)f2bf_hw(silu_fast(g.w) * u.w) << 16));
            return;
        }
        float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int k = 0; k < splits; k++) {
            const float4 a = ld_stream((const float4 *)(ws + k * stride + (size_t)m * p.N + c));
            s.x += a.x; s.y += a.y; s.z += a.z; s.w += a.w;
        }
        const float vd = p.epi == IRIS_EPI_GATED_ADD ? 1.0f : 0.0f;
        const float4 v = p.vec ? *(const float4 *)(p.vec + c) : make_float4(vd, vd, vd, vd);
        const size_t o = (size_t)m * p.ldo + c;
        switch (p.epi) {
        case IRIS_EPI_F32:
            *(float4 *)((float *)p.out + o) = make_float4(s.x + v.x, s.y + v.y, s.z + v.z, s.w + v.w);
            break;
        case IRIS_EPI_BF16:
            *(uint2 *)((uint16_t *)p.out + o) =
                make_uint2((uint32_t)f2bf_hw(s.x + v.x) | ((uint32_t)f2bf_hw(s.y + v.y) << 16),
                           (uint32_t)f2bf_hw(s.z + v.z) | ((uint32_t)f2bf_hw(s.w + v.w) << 16));
            break;
        case IRIS_EPI_GATED_ADD: {
            float4 *dst = (float4 *)((float *)p.out + o);
            float4 y = *dst;
            y.x += v.x * s.x; y.y += v.y * s.y; y.z += v.z * s.z; y.w += v.w * s.w;
            *dst = y;
            break;
        }
        case IRIS_EPI_ADD: {
            float4 *dst = (float4 *)((float *)p.out + o);
            float4 y = *dst;
            y.x += s.x + v.x; y.y += s.y + v.y; y.z += s.z + v.z; y.w += s.w + v.w;
            *dst = y;
            break;
        }
        default: break;
        }
        return;
    }
    const long long e = i - R.start[pi];
    const int m = (int)(e / nout), c = (int)(e % nout);
    if (p.epi == IRIS_EPI_SWIGLU) {
        const int gc = (c >> 5) * 64 + (c & 31);
        float g = 0.0f, u = 0.0f;
        for (int k = 0; k < splits; k++) {
            g += ws[k * stride + (size_t)m * p.N + gc];
            u += ws[k * stride + (size_t)m * p.N + gc + 32];
        }
        ((uint16_t *)p.out)[(size_t)m * p.ldo + c] = f2bf_hw(silu_fast(g) * u);
        return;
    }
    float s = 0.0f;
    for (int k = 0; k < splits; k++) s += ws[k * stride + (size_t)m * p.N + c];
    switch (p.epi) {
    case IRIS_EPI_F32: ((float *)p.out)[(size_t)m * p.ldo + c] = s + (p.vec ? p.vec[c] : 0.0f); break;
    case IRIS_EPI_BF16: ((uint16_t *)p.out)[(size_t)m * p.ldo + c] = f2bf_hw(s + (p.vec ? p.vec[c] : 0.0f)); break;
    case IRIS_EPI_GATED_ADD: ((float *)p.out)[(size_t)m * p.ldo + c] += (p.vec ? p.vec[c] : 1.0f) * s; break;
    case IRIS_EPI_F32_T: ((float *)p.out)[(size_t)c * p.ldo + m] = s + (p.vec ? p.vec[c] : 0.0f); break;
    case IRIS_EPI_ADD: ((float *)p.out)[(size_t)m * p.ldo + c] += s + (p.vec ? p.vec[c] : 0.0f); break;
    default: break;
    }
}

/* the reduce launch over the split problems of a launch (n of them) */
int launch_reduce(const iris_gemm_problem_t *ps, float *const *ws, const long long *stride, const int *chunks, int n) {
    ReduceParams R;
    memset(&R, 0, sizeof(R));
    R.n = n;
    long long items = 0;
    for (int i = 0; i < n; i++) {
        const iris_gemm_problem_t &p = ps[i];
        R.p[i] = p;
        R.ws[i] = ws[i];
        R.stride[i] = stride[i];
        R.chunks[i] = chunks[i];
        const int nout = p.epi == IRIS_EPI_SWIGLU ? p.N / 2 : p.N;
        const int ob = p.epi == IRIS_EPI_BF16 || p.epi == IRIS_EPI_SWIGLU ? 8 : 16;
        const bool v4 = p.epi != IRIS_EPI_F32_T && nout % 4 == 0 && p.N % 4 == 0 && p.ldo % 4 == 0 &&
                        ((uintptr_t)p.out % ob) == 0 && ((uintptr_t)p.vec % 16) == 0 && ((uintptr_t)ws[i] % 16) == 0;
        R.vw[i] = v4 ? 4 : 1;
        R.start[i] = items;
        items += (long long)p.M * nout / R.vw[i];
    }
    for (int i = n; i <= MAXP; i++) R.start[i] = items;
    if (items == 0) return 0;
    IRIS_LAUNCH(splitk_reduce_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, iris_stream(), R);
    return iris_launch_check("splitk_reduce_kernel");
}

int check_problem(const iris_gemm_problem_t &p) {
    if (p.K <= 0 || p.K % BK) return iris_set_error("gemm: K=%d must be a positive multiple of %d", p.K, BK);
    if (p.lda % 8 || p.ldw % 8 || p.lda < p.K || p.ldw < p.K)
        return iris_set_error("gemm: lda=%d ldw=%d must be multiples of 8 and >= K=%d", p.lda, p.ldw, p.K);
    if (((uintptr_t)p.A | (uintptr_t)p.W) & 15) return iris_set_error("gemm: A/W must be 16-byte aligned");
    if (!p.A || !p.W || !p.out) return iris_set_error("gemm: null operand");
    if (p.epi == IRIS_EPI_SWIGLU && (p.N % 64)) return iris_set_error("gemm: SwiGLU needs N %% 64 == 0");
    if (p.epi < 0 || p.epi > IRIS_EPI_ADD) return iris_set_error("gemm: epilogue %d", p.epi);
    if (p.K2 < 0 || p.K2 % BK) return iris_set_error("gemm: K2=%d must be a multiple of %d", p.K2, BK);
    if (p.K2 > 0) {
        if (!p.A2 || !p.W2 || (((uintptr_t)p.A2 | (uintptr_t)p.W2) & 15))
            return iris_set_error("gemm: second segment operands null or not 16-byte aligned");
        if (p.lda2 % 8 || p.ldw2 % 8 || p.lda2 < p.K2 || p.ldw2 < p.K2)
            return iris_set_error("gemm: lda2=%d ldw2=%d must be multiples of 8 and >= K2=%d", p.lda2, p.ldw2, p.K2);
        if ((long long)BM * p.lda2 * 2 >= (1LL << 31) || (long long)BN * p.ldw2 * 2 >= (1LL << 31))
            return iris_set_error("gemm: second segment leading dimension too large");
    }
    const int ldo_need = p.epi == IRIS_EPI_SWIGLU ? p.N / 2 : p.epi == IRIS_EPI_F32_T ? p.M : p.N;
    if (p.ldo < ldo_need) return iris_set_error("gemm: ldo=%d < %d", p.ldo, ldo_need);
    /* 32-bit buffer offsets: one tile's rows must span < 2 GiB */
    if ((long long)BM * p.lda * 2 >= (1LL << 31) || (long long)BN * p.ldw * 2 >= (1LL << 31))
        return iris_set_error("gemm: leading dimension too large");
    return 0;
}

}  // namespace

namespace {

/* One launch of up to MAXP problems. want[i] > 1 (want may be NULL) splits
 * problem i over K into that many chunks of whole K steps: its f32 partials
 * go to the workspace (after those of the split problems before it) and one
 * reduce launch after the GEMM sums them and applies the epilogues. Tiles
 * are 256 wide, or 224 wide (plain GEMM, no SwiGLU output written by the
 * tiles) when that needs fewer rounds of tile widths: with one block per CU
 * a launch takes ceil(blocks / CUs) rounds, each as long as one tile's width.
 * The tile width does not change any output element's accumulation order.
 * phase1 > 0: the tiles of the first phase1 problems are dispatched before
 * those of the others (a launch whose last problems fill a part-empty last
 * round); bnt > 0 forces the tile width. bmt = 128: 128 x 256 tiles (no
 * second K segment). */
int launch_gemm(const iris_gemm_problem_t *probs, int n, const int *want, float *ws, size_t ws_bytes,
                int phase1 = 0, int force_bnt = 0, int bmt = BM) {
    if (!probs || n < 1 || n > MAXP) return iris_set_error("gemm: %d problems (1..%d)", n, MAXP);
    GemmParams P;
    memset(&P, 0, sizeof(P));
    P.nprob = n;
    bool seg2 = false, swiglu_tiles = false, split = false;
    size_t ws_used = 0;
    for (int i = 0; i < n; i++) {
        const iris_gemm_problem_t &p = probs[i];
        P.p[i] = p;
        P.chunks[i] = 1;
        if (p.M <= 0 || p.N <= 0) continue;
        if (check_problem(p)) return -1;
        if (bmt != BM && p.K2) return iris_set_error("gemm: 128-row tiles take no second K segment");
        P.tiles_m[i] = (p.M + bmt - 1) / bmt;
        if (want && want[i] > 1) {
            const int nk = p.K / BK;
            const int kchunk = (nk + want[i] - 1) / want[i] * BK;
            const int chunks = (p.K + kchunk - 1) / kchunk;
            /* K of one step leaves one chunk: that is the plain product */
            if (chunks > 1) {
                if (p.K2) return iris_set_error("gemm_splitk: no second K segment");
                P.chunks[i] = chunks;
                P.kchunk[i] = kchunk;
                P.ws_stride[i] = (long long)p.M * p.N;
                P.ws[i] = ws + ws_used / sizeof(float);
                ws_used += (size_t)chunks * P.ws_stride[i] * sizeof(float);
                split = true;
            }
        }
        seg2 = seg2 || p.K2 > 0;
        swiglu_tiles = swiglu_tiles || (p.epi == IRIS_EPI_SWIGLU && P.chunks[i] == 1);
    }
    if (split && (!ws || ((uintptr_t)ws & 15) || ws_used > ws_bytes))
        return iris_set_error("gemm_splitk: workspace of %zu bytes for %zu bytes of f32 partials", ws_bytes, ws_used);
    long long t256 = 0, t224 = 0;
    for (int i = 0; i < n; i++) {
        if (!P.tiles_m[i]) continue;
        t256 += (long long)P.tiles_m[i] * ((probs[i].N + 255) / 256) * P.chunks[i];
        t224 += (long long)P.tiles_m[i] * ((probs[i].N + 223) / 224) * P.chunks[i];
    }
    if (t256 == 0) return 0;
    int bnt = BN;
    const int cus = iris_cu_count();
    if (bmt != BM) {
        bnt = BN;
    } else if (force_bnt == 224 && !seg2 && !swiglu_tiles) {
        bnt = 224;
    } else if (!force_bnt && !seg2 && !swiglu_tiles && cus > 0) {
        const long long w256 = (t256 + cus - 1) / cus * BN, w224 = (t224 + cus - 1) / cus * 224;
        if (w224 * 100 < w256 * 97) bnt = 224;
    }
    int total = 0;
    for (int i = 0; i < n; i++) {
        P.tile_start[i] = total;
        if (!P.tiles_m[i]) continue;
        P.tiles_n[i] = (probs[i].N + bnt - 1) / bnt;
        total += P.tiles_m[i] * P.tiles_n[i] * P.chunks[i];
    }
    for (int i = n; i <= MAXP; i++) P.tile_start[i] = total;
    P.total = total;
    if (phase1 > 0 && phase1 < n) {
        P.phase_tiles = P.tile_start[phase1];
        P.phase_blocks = (P.phase_tiles + 7) / 8 * 8;
    }
    P.per_xcd = (total - P.phase_tiles + 7) / 8;
    const dim3 grid(P.phase_blocks + 8 * P.per_xcd);
    if (bmt != BM)
        IRIS_LAUNCH((gemm_bf16_kernel<0, 256, 128>), grid, dim3(NT), 0, iris_stream(), P);
    else if (bnt == 224)
        IRIS_LAUNCH((gemm_bf16_kernel<0, 224>), grid, dim3(NT), 0, iris_stream(), P);
    else if (seg2)
        IRIS_LAUNCH(gemm_bf16_kernel<3>, grid, dim3(NT), 0, iris_stream(), P);
    else
        IRIS_LAUNCH(gemm_bf16_kernel<0>, grid, dim3(NT), 0, iris_stream(), P);
    if (iris_launch_check("gemm_bf16_kernel")) return -1;
    if (!split) return 0;
    iris_gemm_problem_t rp[MAXP];
    float *rws[MAXP];
    long long rstride[MAXP];
    int rchunks[MAXP], nr = 0;
    for (int i = 0; i < n; i++)
        if (P.chunks[i] > 1) {
            rp[nr] = probs[i];
            rws[nr] = P.ws[i];
            rstride[nr] = P.ws_stride[i];
            rchunks[nr++] = P.chunks[i];
        }
    return launch_reduce(rp, rws, rstride, rchunks, nr);
}

}  // namespace

/* A launch whose 256-row tiles fill at most half of the CUs runs on 128-row
 * tiles (twice the tiles, one round; the same additions per element): on the
 * products measured (512-1536 rows) they took 0.71-0.79 of the time. */
extern "C" int iris_hip_gemm(const iris_gemm_problem_t *probs, int n) {
    if (!probs || n < 1 || n > MAXP) return iris_set_error("gemm: %d problems (1..%d)", n, MAXP);
    const int cus = iris_cu_count();
    long long tiles = 0;
    bool seg2 = false;
    for (int i = 0; i < n; i++) {
        if (probs[i].M <= 0 || probs[i].N <= 0) continue;
        tiles += (long long)((probs[i].M + BM - 1) / BM) * ((probs[i].N + BN - 1) / BN);
        seg2 = seg2 || probs[i].K2 > 0;
    }
    const bool half = tiles > 0 && !seg2 && cus > 0 && 2 * tiles <= cus;
    return launch_gemm(probs, n, nullptr, nullptr, 0, 0, 0, half ? 128 : BM);
}

/* Split-K partials without a caller workspace: a file-scope device array of
 * IRIS_NOALLOC_SCRATCH_BYTES, held by each GPU the library runs on until the
 * process ends. Host code never passes the array's name to a kernel (on the
 * host it is a stand-in, not a device address): its device address is looked
 * up once per device with hipGetSymbolAddress and kept per device. Every
 * call on a GPU shares that GPU's array, so calls that overlap on one GPU
 * (different streams, threads) race. Each chunk's partial overwrites its
 * whole M x N region, so nothing is cleared between calls. */
__device__ __align__(256) float scratch[IRIS_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {
constexpr int MAX_DEVICES = 64;
void *g_scratch_ptr[MAX_DEVICES];
std::mutex g_scratch_mutex;

float *scratch_ptr() {
    int dev = -1;
    if (iris_check(hipGetDevice(&dev), "noalloc: hipGetDevice")) return nullptr;
    if (dev < 0 || dev >= MAX_DEVICES) {
        iris_set_error("noalloc: device %d outside 0..%d", dev, MAX_DEVICES - 1);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        if (iris_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "noalloc: hipGetSymbolAddress")) return nullptr;
        g_scratch_ptr[dev] = ptr;
    }
    return (float *)g_scratch_ptr[dev];
}
}  // namespace

extern "C" int iris_hip_gemm_splitk_noalloc(const iris_gemm_problem_t *p, int splits) {
    if (!p) return iris_set_error("gemm_splitk_noalloc: null problem");
    if (splits <= 1) return iris_hip_gemm(p, 1);
    if (p->M <= 0 || p->N <= 0) return 0;
    if (check_problem(*p)) return -1;
    const int nk = p->K / BK;
    const int kchunk = (nk + splits - 1) / splits * BK;
    const size_t chunks = (size_t)((p->K + kchunk - 1) / kchunk);
    /* one chunk is the plain product, which needs no scratch */
    if (chunks <= 1) return iris_hip_gemm(p, 1);
    const size_t need = chunks * (size_t)p->M * (size_t)p->N * sizeof(float);
    if (need > IRIS_NOALLOC_SCRATCH_BYTES)
        return iris_set_error("gemm_splitk_noalloc: %zu chunks x %d x %d f32 partials need %zu bytes, the scratch "
                              "holds %zu", chunks, p->M, p->N, need, (size_t)IRIS_NOALLOC_SCRATCH_BYTES);
    float *ws = scratch_ptr();
    if (!ws) return -1;
    return iris_hip_gemm_splitk(p, splits, ws, IRIS_NOALLOC_SCRATCH_BYTES);
}

extern "C" int iris_hip_gemm_splitk(const iris_gemm_problem_t *p, int splits, float *ws, size_t ws_bytes) {
    if (!p) return iris_set_error("gemm_splitk: null problem");
    return launch_gemm(p, 1, &splits, ws, ws_bytes);
}

namespace {

/* the problem restricted to output rows [r0, M) (rows = true) or output
 * columns [c0, N) */
iris_gemm_problem_t sub_problem(const iris_gemm_problem_t &p, bool rows, int from) {
    iris_gemm_problem_t q = p;
    const size_t es = (p.epi == IRIS_EPI_BF16 || p.epi == IRIS_EPI_SWIGLU) ? 2 : 4;
    if (rows) {
        q.A = p.A + (size_t)from * p.lda;
        q.out = (char *)p.out + es * (p.epi == IRIS_EPI_F32_T ? (size_t)from : (size_t)from * p.ldo);
        q.M = p.M - from;
    } else {
        q.W = p.W + (size_t)from * p.ldw;
        if (p.vec) q.vec = p.vec + from;
        const size_t col = p.epi == IRIS_EPI_SWIGLU ? (size_t)from / 2 : (size_t)from;
        q.out = (char *)p.out + es * (p.epi == IRIS_EPI_F32_T ? col * p.ldo : col);
        q.N = p.N - from;
    }
    return q;
}

/* A product whose 256-wide tiles fill one or more whole rounds of blocks on
 * the CUs and then a part-empty last round: the whole rounds run as they
 * are, and the leftover tiles -- taken as whole tile rows (or columns) at
 * the end of the output -- are split over K across the CUs the whole rounds
 * free, in the same launch, with one reduce launch after it. Taken when a
 * cost estimate in units of one round (the split pieces' share of a round,
 * plus the reduce pass's traffic at 4.5 TB/s and its launch) beats the plain
 * launch at either tile width by 8 %. Returns the number of chunks (0: not
 * taken) and the two problems. */
int tail_plan(const iris_gemm_problem_t &p, size_t ws_bytes, iris_gemm_problem_t parts[2]) {
    const int cus = iris_cu_count();
    if (cus <= 0 || p.K2 || p.M <= 0 || p.N <= 0) return 0;
    const int tm = (p.M + BM - 1) / BM, tn = (p.N + BN - 1) / BN, nk = p.K / BK;
    const long long T = (long long)tm * tn, full = T / cus, tail = T - full * cus;
    if (full < 1 || tail == 0 || nk < 8) return 0;
    const int kr = (int)((tail + tn - 1) / tn), kc = (int)((tail + tm - 1) / tm);
    const bool rows_ok = kr < tm, cols_ok = kc < tn && !(p.epi == IRIS_EPI_SWIGLU && (p.N % 64));
    if (!rows_ok && !cols_ok) return 0;
    const bool rows = rows_ok && (!cols_ok || (long long)kr * tn <= (long long)kc * tm);
    const int from = rows ? (tm - kr) * BM : (tn - kc) * BN;
    const long long tail_tiles = rows ? (long long)kr * tn : (long long)kc * tm;
    const size_t part_bytes = rows ? (size_t)(p.M - from) * p.N * 4 : (size_t)p.M * (p.N - from) * 4;
    int pieces = (int)std::min<long long>(cus / tail_tiles, nk / 4);
    while (pieces > 1 && (size_t)pieces * part_bytes > ws_bytes) pieces--;
    if (pieces < 2) return 0;
    /* estimates in units of one round of 256-wide tiles over the whole K */
    const double round_us = 2.0 * BM * BN * (double)p.K / 5.1e12 * 1e6;
    const bool rmw = p.epi == IRIS_EPI_GATED_ADD || p.epi == IRIS_EPI_ADD;
    const double out_bytes = part_bytes / 4.0 * ((p.epi == IRIS_EPI_BF16 || p.epi == IRIS_EPI_SWIGLU) ? 2 : 4) *
                             (rmw ? 2 : 1);
    const double reduce_us = ((double)pieces * part_bytes + out_bytes) / 4.5e12 * 1e6 + 6.0;
    const double split_cost = (double)full + 1.0 / pieces + reduce_us / round_us;
    double plain = (double)full + 1.0;
    if (p.epi != IRIS_EPI_SWIGLU) {
        const long long t224 = (long long)tm * ((p.N + 223) / 224);
        plain = std::min(plain, (double)((t224 + cus - 1) / cus) * 224.0 / 256.0);
    }
    if (split_cost > 0.92 * plain) return 0;
    parts[0] = p;
    if (rows) parts[0].M = from;
    else parts[0].N = from;
    parts[1] = sub_problem(p, rows, from);
    return pieces;
}

}  // namespace

extern "C" int iris_hip_gemm_fill_n(const iris_gemm_problem_t *probs, int n, float *ws, size_t ws_bytes) {
    if (!probs || n < 1 || n > MAXP) return iris_set_error("gemm_fill: %d problems (1..%d)", n, MAXP);
    const int cus = iris_cu_count();
    long long tiles = 0, tiles128 = 0;
    size_t per = 0, out_bytes = 0;
    int min_nk = 1 << 30, max_nk = 0;
    bool seg2 = false;
    for (int i = 0; i < n; i++) {
        const iris_gemm_problem_t &p = probs[i];
        if (p.M <= 0 || p.N <= 0) continue;
        tiles += (long long)((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
        tiles128 += (long long)((p.M + 127) / 128) * ((p.N + BN - 1) / BN);
        per += (size_t)p.M * (size_t)p.N * sizeof(float);
        const bool rmw = p.epi == IRIS_EPI_GATED_ADD || p.epi == IRIS_EPI_ADD;
        const size_t es = p.epi == IRIS_EPI_BF16 ? 2 : p.epi == IRIS_EPI_SWIGLU ? 1 : rmw ? 8 : 4;
        out_bytes += (size_t)p.M * (size_t)p.N * es;
        min_nk = std::min(min_nk, p.K / BK);
        max_nk = std::max(max_nk, p.K / BK);
        seg2 = seg2 || p.K2 > 0;
    }
    /* Tiles filling at most half of the CUs and a long K: split K into up to
     * CUs / tiles chunks of at least 4 K steps, as many as the workspace
     * holds, on 256 x 256 tiles, or on 128 x 256 tiles where those still fit
     * one round (twice the tiles, so fewer chunks: less reduce traffic and
     * shorter f32 partial epilogues) and an estimate of the launch and its
     * reduce is lower. The estimate (us): K steps per block times the step
     * time of the tile shape with the chip partly idle, plus a tile's
     * prologue and partial store, plus the reduce pass's traffic at 4.5 TB/s
     * and its launch; measured over the encoder, caption, embedder and
     * 512x512 products, it picks the faster shape in each. */
    if (tiles > 0 && !seg2 && cus > 0 && ws && 2 * tiles <= cus && min_nk >= 8) {
        auto fit = [&](long long s) {
            s = std::max(1LL, std::min<long long>(s, min_nk / 4));
            while (s > 1 && (size_t)s * per > ws_bytes) s--;
            return (int)s;
        };
        auto est = [&](bool half, int s) {
            const double step = half ? 0.9 : 1.3, fixed = half ? 8.0 : 14.0;
            const double red = s > 1 ? ((double)s * per + out_bytes) / 4.5e6 + 6.0 : 0.0;
            return (double)max_nk / s * step + fixed + red;
        };
        const int s256 = fit(cus / tiles);
        const int s128 = tiles128 <= cus ? fit(cus / tiles128) : 0;
        int want[MAXP];
        if (s128 > 0 && est(true, s128) < est(false, s256)) {
            for (int i = 0; i < n; i++) want[i] = s128;
            return launch_gemm(probs, n, s128 > 1 ? want : nullptr, ws, ws_bytes, 0, 0, 128);
        }
        if (s256 > 1) {
            for (int i = 0; i < n; i++) want[i] = s256;
            return launch_gemm(probs, n, want, ws, ws_bytes);
        }
    }
    if (n == 1 && ws && !((uintptr_t)ws & 15)) {
        iris_gemm_problem_t parts[2];
        const int pieces = tail_plan(probs[0], ws_bytes, parts);
        if (pieces > 1) {
            if (check_problem(probs[0])) return -1;
            const int want[2] = {1, pieces};
            return launch_gemm(parts, 2, want, ws, ws_bytes, 1, BN);
        }
    }
    return launch_gemm(probs, n, nullptr, nullptr, 0);
}

extern "C" int iris_hip_gemm_fill(const iris_gemm_problem_t *p, float *ws, size_t ws_bytes) {
    if (!p) return iris_set_error("gemm_fill: null problem");
    return iris_hip_gemm_fill_n(p, 1, ws, ws_bytes);
}

namespace {

/* per row, one wave: the tiles' (max, sum) pairs merged into (max, 1 / sum);
 * lane j takes tiles j, j + 64, ..., then the wave's butterfly (a fixed
 * order) */
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float2 *stat, int tiles, int rows,
                                                           float2 *row_out) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float2 *s = stat + (size_t)r * tiles;
    float m = -INFINITY;
    for (int t = lane; t < tiles; t += 64) m = fmaxf(m, s[t].x);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    float l = 0.0f;
    for (int t = lane; t < tiles; t += 64) l += s[t].y * __builtin_amdgcn_exp2f(s[t].x - m);
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
    if (lane == 0) row_out[r] = make_float2(m, 1.0f / l);
}

}  // namespace

extern "C" int iris_hip_softmax_scores(const uint16_t *q, int ld_q, const uint16_t *k, int ld_k, int M, int N, int d,
                                       float scale, uint16_t *p, int ld_p, int pad_n, float *stat, float *row) {
    if (!q || !k || !p || !stat || !row || M <= 0 || N <= 0)
        return iris_set_error("softmax_scores: null buffer or empty shape (%d x %d)", M, N);
    const int tiles_n = (N + BN - 1) / BN;
    if (pad_n < N || pad_n > tiles_n * BN || ld_p < pad_n)
        return iris_set_error("softmax_scores: pad %d for %d columns (ld %d)", pad_n, N, ld_p);
    if (((uintptr_t)stat | (uintptr_t)row) & 7) return iris_set_error("softmax_scores: statistics not 8-byte aligned");
    if ((long long)M * tiles_n >= (1LL << 31)) return iris_set_error("softmax_scores: too many rows");
    GemmParams P;
    memset(&P, 0, sizeof(P));
    iris_gemm_problem_t &pr = P.p[0];
    pr.A = q; pr.lda = ld_q; pr.W = k; pr.ldw = ld_k; pr.out = p; pr.ldo = ld_p;
    pr.M = M; pr.N = N; pr.K = d; pr.epi = IRIS_EPI_BF16;
    if (check_problem(pr)) return -1;
    P.nprob = 1;
    P.chunks[0] = 1;
    P.tiles_m[0] = (M + BM - 1) / BM;
    P.tiles_n[0] = tiles_n;
    P.total = P.tiles_m[0] * tiles_n;
    for (int i = 1; i <= MAXP; i++) P.tile_start[i] = P.total;
    P.per_xcd = (P.total + 7) / 8;
    P.sm_scale = scale * 1.44269504088896341f;   /* log2(e): scores in log2 units */
    P.sm_stat = (float2 *)stat;
    P.sm_pad = pad_n;
    const dim3 grid(8 * P.per_xcd);
    IRIS_LAUNCH(gemm_bf16_kernel<4>, grid, dim3(NT), 0, iris_stream(), P);
    if (iris_launch_check("gemm_bf16_kernel<4> (row statistics)")) return -1;
    IRIS_LAUNCH(softmax_rows_kernel, dim3((M + 3) / 4), dim3(256), 0, iris_stream(), (const float2 *)stat, tiles_n, M,
                (float2 *)row);
    if (iris_launch_check("softmax_rows_kernel")) return -1;
    P.sm_row = (const float2 *)row;
    IRIS_LAUNCH(gemm_bf16_kernel<5>, grid, dim3(NT), 0, iris_stream(), P);
    return iris_launch_check("gemm_bf16_kernel<5> (probabilities)");
}

extern "C" int iris_hip_conv3x3(const iris_conv3x3_t *c) {
    if (!c || !c->in || !c->wt || !c->out) return iris_set_error("conv3x3: null operand");
    if (c->cin < 64 || c->cin > 8192 || (c->cin & (c->cin - 1)))
        return iris_set_error("conv3x3: cin=%d must be a power of two in 64..8192", c->cin);
    if (c->up < 0 || c->up > 2) return iris_set_error("conv3x3: up=%d (0, 1 or 2)", c->up);
    if (c->H <= 0 || c->W <= 0 || c->H > 8000 || c->W > 8000 || (c->up == 1 && ((c->H | c->W) & 1)))
        return iris_set_error("conv3x3: output %dx%d", c->H, c->W);
    if (c->epi != IRIS_EPI_F32 && c->epi != IRIS_EPI_BF16 && c->epi != IRIS_EPI_ADD)
        return iris_set_error("conv3x3: epilogue %d (F32, BF16 or ADD)", c->epi);
    const size_t in_pix = c->up == 1 ? (size_t)(c->H / 2) * (c->W / 2)
                          : c->up == 2 ? (size_t)(2 * c->H) * (2 * c->W) : (size_t)c->H * c->W;
    const size_t in_bytes = in_pix * (size_t)c->cin * 2;
    if (in_bytes >= (1ull << 31)) return iris_set_error("conv3x3: input of %zu bytes (< 2 GiB)", in_bytes);
    if ((long long)c->H * c->W >= (1LL << 31)) return iris_set_error("conv3x3: too many pixels");
    iris_gemm_problem_t p;
    memset(&p, 0, sizeof(p));
    p.A = c->in;
    p.W = c->wt;
    p.out = c->out;
    p.vec = c->bias;
    p.M = c->H * c->W;
    p.N = c->cout;
    p.K = 9 * c->cin;
    p.lda = p.ldw = p.K;
    p.ldo = c->ldo;
    p.epi = c->epi;
    if (p.N <= 0) return 0;
    if (check_problem(p)) return -1;
    GemmParams P;
    memset(&P, 0, sizeof(P));
    P.nprob = 1;
    P.p[0] = p;
    /* 128-wide tiles for at most 128 output channels (the decoder's
     * full-resolution convolutions): same per-element accumulation order */
    const int bnt = p.N <= 128 ? 128 : BN;
    P.tiles_m[0] = (p.M + BM - 1) / BM;
    P.tiles_n[0] = (p.N + bnt - 1) / bnt;
    P.conv_h = c->H;
    P.conv_w = c->W;
    P.conv_up = c->up;
    P.conv_cpt_shift = __builtin_ctz((unsigned)c->cin) - 6;
    P.conv_cin_bshift = __builtin_ctz((unsigned)c->cin) + 1;
    P.conv_in_bytes = (unsigned)in_bytes;
    if (c->gn_part) {
        const int G = c->gn_groups, cpg = G > 0 && p.N % G == 0 ? p.N / G : 0;
        if (cpg == 0 || cpg % 4 || bnt % cpg || c->splits > 1 || ((uintptr_t)c->gn_part & 7))
            return iris_set_error("conv3x3: GroupNorm statistics need groups of a multiple of 4 channels dividing the "
                                  "%d-wide tile, no split-K and an 8-byte aligned buffer (cout %d, groups %d, splits %d)",
                                  bnt, p.N, G, c->splits);
        P.gn_part = c->gn_part;
        P.gn_groups = G;
    }
    int chunks = 1;
    long long stride = 0;
    P.chunks[0] = 1;
    if (c->splits > 1) {
        const int nk = p.K / BK;
        P.kchunk[0] = (nk + c->splits - 1) / c->splits * BK;
        chunks = (p.K + P.kchunk[0] - 1) / P.kchunk[0];
        stride = (long long)p.M * p.N;
        if (!c->ws || ((uintptr_t)c->ws & 15) || (size_t)chunks * stride * sizeof(float) > c->ws_bytes)
            return iris_set_error("conv3x3: split-K workspace of %zu bytes for %d x %d x %d f32", c->ws_bytes, chunks,
                                  p.M, p.N);
    }
    P.total = P.tiles_m[0] * P.tiles_n[0] * chunks;
    for (int i = 1; i <= MAXP; i++) P.tile_start[i] = P.total;
    P.per_xcd = (P.total + 7) / 8;
    if (chunks > 1) {
        P.chunks[0] = chunks;
        P.ws[0] = c->ws;
        P.ws_stride[0] = stride;
    }
    if (c->up == 2 && bnt == 128)
        IRIS_LAUNCH((gemm_bf16_kernel<2, 128>), dim3(8 * P.per_xcd), dim3(NT), 0, iris_stream(), P);
    else if (c->up == 2)
        IRIS_LAUNCH(gemm_bf16_kernel<2>, dim3(8 * P.per_xcd), dim3(NT), 0, iris_stream(), P);
    else if (bnt == 128)
        IRIS_LAUNCH((gemm_bf16_kernel<1, 128>), dim3(8 * P.per_xcd), dim3(NT), 0, iris_stream(), P);
    else
        IRIS_LAUNCH(gemm_bf16_kernel<1>, dim3(8 * P.per_xcd), dim3(NT), 0, iris_stream(), P);
    if (iris_launch_check("gemm_bf16_kernel<conv>")) return -1;
    if (chunks == 1) return 0;
    float *rws = c->ws;
    return launch_reduce(&p, &rws, &stride, &chunks, 1);
}
