/*
 * iris_hip.h - C ABI of the MI355X (gfx950) HIP layer.
 *
 * Plain pointers and sizes only; every pointer named d_* is device memory
 * returned by iris_hip_malloc (or any hipMalloc'd pointer of this process).
 * All launches are asynchronous on the library's one stream; iris_hip_sync()
 * waits. Functions return 0 on success and a negative value on error, with a
 * message in iris_hip_last_error(), which mirrors the reference's "0 means
 * the caller falls back" convention (iris_metal.h:23-60) without a fallback:
 * the host code reports the error and returns NULL.
 *
 * This layer takes the place the Metal runtime has in the reference
 * (iris_metal.h: device init :23-40, weight cache keyed by host pointer
 * :710-730, batch/command buffers :315-320, GPU tensors :158-223, kernels of
 * iris_shaders.metal). Coarse per-step entry points live in
 * iris_transformer.h; the kernel-level exports below serve the host code and
 * the parity tests.
 */
#ifndef IRIS_HIP_H
#define IRIS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- device, memory, stream (cf. iris_metal_init / iris_metal_available) ---- */
int iris_hip_init(int device);
int iris_hip_available(void);
const char *iris_hip_last_error(void);
const char *iris_hip_device_name(void);
void *iris_hip_malloc(size_t bytes);                 /* NULL on failure */
void iris_hip_free(void *d_ptr);
int iris_hip_memcpy_h2d(void *d_dst, const void *src, size_t bytes);   /* on the stream */
int iris_hip_memcpy_d2h(void *dst, const void *d_src, size_t bytes);   /* synchronous */
int iris_hip_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes); /* on the stream */
int iris_hip_memset(void *d_dst, int value, size_t bytes);             /* not for captured work */
int iris_hip_sync(void);
size_t iris_hip_mem_in_use(void);

/* ---- timing: events recorded on the library stream ---- */
int iris_hip_event_record(int slot);                 /* slot 0..63 */
float iris_hip_event_elapsed_ms(int slot_start, int slot_end);

/* ---- per-kernel profile of eager launches ----
 * No counterpart in the reference's interface; it backs the reference's
 * profile counters (iris_print_blas_profile / iris_reset_blas_profile,
 * iris_transformer_flux.c:55-80). While enabled, every kernel the library
 * launches outside graph capture is bracketed by two events on the library
 * stream, and the denoiser runs its forward launch by launch instead of
 * replaying its captured graph, so the records cover a whole step.
 * enable() syncs and clears the records; read() syncs and aggregates them by
 * (kernel, grid size) into out (at most max entries; returns the count). */
typedef struct {
    const char *kernel;   /* the kernel as launched, e.g. "gemm_bf16_kernel<0>" */
    long long grid;       /* workgroups per launch */
    int calls;
    double total_ms, min_ms, max_ms;
} iris_kernel_time_t;
int iris_hip_profile_enable(int on);
int iris_hip_profile_enabled(void);
int iris_hip_profile_read(iris_kernel_time_t *out, int max);

/* ---- side stream (no counterpart in the reference) ----
 * Work that does not feed what follows it on the library stream can run
 * beside it: iris_hip_fork makes the side stream wait for everything enqueued
 * on the library stream so far; launches made between iris_hip_side(1) and
 * iris_hip_side(0) go to the side stream; iris_hip_join makes the library
 * stream wait for everything enqueued on the side stream. Inside a graph
 * capture of the library stream the side stream is captured with it (fork
 * and join become dependency edges); every fork is joined before the capture
 * ends. Synchronisation and copies stay on the library stream. */
int iris_hip_fork(void);
void iris_hip_side(int on);
int iris_hip_join(void);

/* ---- graph capture of the library stream (cf. iris_gpu_batch_begin/end) ---- */
int iris_hip_graph_begin(void);
void *iris_hip_graph_end(void);                      /* instantiated graph, NULL on error */
int iris_hip_graph_launch(void *graph);
void iris_hip_graph_destroy(void *graph);

/* ---- bf16 MFMA GEMM: out = A[M,K] . W[N,K]^T with a fused epilogue ---- */
enum {
    IRIS_EPI_F32 = 0,        /* out f32[M,ldo] = acc (+ vec[n] bias)                 */
    IRIS_EPI_BF16 = 1,       /* out bf16[M,ldo] = acc (+ vec[n] bias)                */
    IRIS_EPI_GATED_ADD = 2,  /* out f32[M,ldo] += vec[n] * acc  (vec NULL: += acc)   */
    IRIS_EPI_SWIGLU = 3,     /* W rows interleaved in 32-row gate/up groups:
                                out bf16[M,ldo] col j = silu(gate_j) * up_j         */
    IRIS_EPI_F32_T = 4,      /* out f32[n*ldo + m] = acc (+ vec[n] bias): transposed */
    IRIS_EPI_ADD = 5         /* out f32[M,ldo] += acc (+ vec[n] bias): residual add  */
};

typedef struct {
    const uint16_t *A;   /* bf16 [M][lda]                           */
    const uint16_t *W;   /* bf16 [N][ldw] (row n = output feature)  */
    void *out;
    const float *vec;    /* bias / gate per output column, or NULL  */
    int M, N, K;         /* K % 64 == 0                             */
    int lda, ldw, ldo;
    int epi;
    /* optional second K segment accumulated into the same product (K2 = 0:
     * none; K2 % 64 == 0): out = A W^T + A2 W2^T with A2 bf16 [M][lda2] and
     * W2 bf16 [N][ldw2]. A low-rank adapter runs as [x | x A^T] [W | s B]^T,
     * in f32 accumulation before the epilogue. Not for split-K. */
    const uint16_t *A2, *W2;
    int K2, lda2, ldw2;
} iris_gemm_problem_t;

/* Up to 4 independent problems in one launch (e.g. the txt and img streams). */
int iris_hip_gemm(const iris_gemm_problem_t *problems, int n_problems);

/* No counterpart in the reference: one problem with K cut into `splits`
 * chunks, for outputs with too few 256x256 tiles to fill the chip (a
 * 512-token text encoder's N 2560 products make 20). Each chunk's f32 partial
 * product goes to the caller's workspace (splits * M * N floats), then one
 * kernel sums the chunks in order (deterministic) and applies the epilogue. */
int iris_hip_gemm_splitk(const iris_gemm_problem_t *problem, int splits, float *d_workspace, size_t workspace_bytes);

/* No counterpart in the reference. One problem, split-K when its 256x256
 * tiles fill less than half of the device's CUs and K has at least 8 steps
 * of 64: up to CUs / tiles chunks of at least 4 steps, as many as the
 * workspace holds (splits * M * N floats); otherwise the plain launch. For
 * the products on few rows (a 512-token caption or text stream, a 128-column
 * final projection) that leave most of the chip idle. */
int iris_hip_gemm_fill(const iris_gemm_problem_t *problem, float *d_workspace, size_t workspace_bytes);

/* No counterpart in the reference. iris_hip_gemm_fill over up to 4
 * independent problems in one launch (the txt and img streams of a double
 * block): when their 256x256 tiles together fill at most half of the CUs and
 * every K has at least 8 steps, each problem is split into the same number of
 * K chunks (its partials after those of the problems before it in the
 * workspace: splits * sum of M * N floats) and one reduce launch applies the
 * epilogues; otherwise one plain launch, as iris_hip_gemm. For the output
 * and down projections of a 512x512 image (1536 rows), which make 72 tiles
 * on a 256-CU device. */
int iris_hip_gemm_fill_n(const iris_gemm_problem_t *problems, int n_problems, float *d_workspace,
                         size_t workspace_bytes);

/* No counterpart in the reference. iris_hip_gemm_splitk without a
 * workspace, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * f32 partials go to a device array the library holds, of
 * IRIS_NOALLOC_SCRATCH_BYTES per GPU, kept until the process ends. Calls no
 * allocating routine (with the per-kernel profile of iris_hip_profile_enable
 * on, a debugging mode, the profile's own event pairs are created on their
 * first use). Rejects problems whose chunks x M x N f32 partials exceed the
 * array (error, -1); a K of one step is the plain product and needs none.
 * Every call on one GPU shares its array: calls that overlap on one GPU race.
 * Results equal iris_hip_gemm_splitk's bit for bit. */
#define IRIS_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int iris_hip_gemm_splitk_noalloc(const iris_gemm_problem_t *problem, int splits);

/* 3x3 convolution, stride 1, zero padding 1, as an implicit GEMM on the MFMA
 * kernel above (replaces vae_conv2d -> iris_conv2d for the 3x3 convolutions,
 * iris_vae.c:148-166, iris_kernels.c:363): the A tiles are gathered from the
 * image by the loads themselves, no im2col buffer.
 *   out[y*W + x][n] = sum_{tap, c} in[(y+dy) >> up][(x+dx) >> up][c] * wt[n][tap][c]
 * with tap = 3 (dy + 1) + (dx + 1), then the epilogue (F32 / BF16 with bias,
 * or ADD: out f32 += conv + bias). in bf16 NHWC [H'][W'][cin] (H' = H/2 for
 * up 1, 2H for up 2, else H),
 * cin a power of two >= 64; wt bf16 [cout][9][cin]; out [H*W][ldo].
 * up = 1 reads the input through a nearest-neighbour 2x upsample
 * (iris_upsample_nearest followed by the conv, iris_vae.c:957-965); up = 2
 * is the encoder's downsample: stride 2 over a (2H) x (2W) input zero-padded
 * on the right and bottom only, out[y][x] = sum in[2y + ky][2x + kx]
 * (vae_pad_right_bottom + the stride-2 conv, iris_vae.c:172-193, :407-418).
 * splits > 1 splits K over blocks into the f32 workspace ws (splits * H*W *
 * cout floats) and reduces in order (deterministic). */
typedef struct {
    const uint16_t *in;
    const uint16_t *wt;
    void *out;
    const float *bias;
    int H, W, cin, cout, up, ldo, epi;
    int splits;
    float *ws;
    size_t ws_bytes;
    /* GroupNorm statistics of the output (iris_group_norm's sums,
     * iris_kernels.c:542), computed in the epilogue; gn_part NULL: none.
     * Without split-K only. For each row tile t of 256 output pixels and
     * each of gn_groups groups of cout / gn_groups channels (a multiple of
     * 4), the sum and the sum of squares of the f32 values written (with
     * IRIS_EPI_ADD the updated stream, with IRIS_EPI_BF16 the values before
     * rounding), summed in a fixed order, at gn_part[(t * gn_groups + g) * 2]
     * and [.. + 1]: the layout and block count (ceil(H * W / 256)) that
     * iris_hip_gn_finalize takes. */
    double *gn_part;
    int gn_groups;
} iris_conv3x3_t;
int iris_hip_conv3x3(const iris_conv3x3_t *c);

/* ---- VAE decoder kernels (vae.hip), channels-last (NHWC) activations ---- */
/* GroupNorm (iris_group_norm, iris_kernels.c:542) in three launches:
 * per-block float64 group sums of x (f32, or bf16 if is_bf16) over
 * `pixels` rows of C channels into part (>= nblk * groups * 2 doubles;
 * returns the number of blocks used, < 0 on error), per-group finalize into
 * ab[2][C] = (gamma / std, beta - mean * gamma / std), and the apply pass
 * y = act(x * ab[0][c] + ab[1][c]) in bf16 with act = swish
 * (iris_vae.c:195) or identity; raw, if not NULL, receives x in bf16. */
int iris_hip_gn_stats(const void *d_x, int is_bf16, int pixels, int C, int groups, double *d_part, int nblk);
int iris_hip_gn_finalize(const double *d_part, int nblk, int pixels, int C, int groups, const float *d_gamma,
                         const float *d_beta, float eps, float *d_ab);
int iris_hip_gn_apply(const void *d_x, int is_bf16, const float *d_ab, int pixels, int C, int swish, uint16_t *d_y,
                      uint16_t *d_raw);
/* Latent [4z][h][w] f32 -> bf16 [2h][2w][64]: denormalize (x * sc + sh, or
 * x / sc + sh if divide), unpatchify 2x2, 1x1 post_quant_conv (pqw [z][z],
 * NULL to skip), channels z..63 zero (iris_vae.c:860-897). z <= 32. */
int iris_hip_vae_front(uint16_t *d_out, const float *d_latent, int z, int h, int w, const float *d_sc,
                       const float *d_sh, int divide, const float *d_pqw, const float *d_pqb);
/* Encoder input: image [3][H][W] f32 -> bf16 [H][W][64] (channels 3..63 zero). */
int iris_hip_vae_img_in(uint16_t *d_out, const float *d_img, int H, int W);
/* Encoder output (iris_vae.c:440-482): moments [h][w][2z] f32 -> 1x1
 * quant_conv (qw [2z][2z], NULL to skip) -> mean (first z) -> patchify 2x2
 * -> (x - sh[c]) * sc[c] per latent channel -> latent [4z][h/2][w/2] f32. */
int iris_hip_vae_enc_out(float *d_latent, const float *d_moments, int z, int h, int w, const float *d_qw,
                         const float *d_qb, const float *d_sc, const float *d_sh);
/* Row softmax, f32 scores [rows][ld_s] -> bf16 [rows][ld_p], columns
 * cols..cols_pad-1 zeroed (iris_softmax in attnblock_forward, iris_vae.c:335). */
int iris_hip_softmax_bf16(uint16_t *d_p, int ld_p, int cols_pad, const float *d_s, int ld_s, int rows, int cols);
/* The same softmax over the scaled products of one attention head, with no
 * f32 score matrix (the scores of attnblock_forward, iris_vae.c:320-335):
 * s[m][n] = scale * q[m] . k[n] over d (q [M][ld_q], k [N][ld_k] bf16,
 * d % 64 == 0), p[m][n] = exp(s - max_n s) / sum_n exp(s - max_n s) in bf16
 * into p [M][ld_p], columns N..pad_n-1 zeroed (pad_n <= N rounded up to 256).
 * Two passes over the products: the first writes each 256-column tile's row
 * (max, sum) into stat (M * ceil(N / 256) float pairs) and merges them per
 * row into row (M float pairs), the second writes p. */
int iris_hip_softmax_scores(const uint16_t *d_q, int ld_q, const uint16_t *d_k, int ld_k, int M, int N, int d,
                            float scale, uint16_t *d_p, int ld_p, int pad_n, float *d_stat, float *d_row);
/* dst[c][r] = src[r][c] (bf16), rows..rows_pad-1 zero-filled; rows_pad % 64 == 0 */
int iris_hip_transpose_bf16(uint16_t *d_dst, int ld_dst, int rows_pad, const uint16_t *d_src, int ld_src, int rows,
                            int cols);
/* conv_out 3x3 cin -> 3 plus the [-1,1] -> uint8 conversion (iris_vae.c:968-994):
 * g bf16 [H][W][cin], wt f32 [9][cin][4], bias f32[3]; rgb uint8 [H][W][3];
 * f32 (or NULL) receives the conv output as [3][H][W]. */
int iris_hip_vae_conv_out(uint8_t *d_rgb, float *d_f32, const uint16_t *d_g, int H, int W, int cin,
                          const float *d_wt, const float *d_bias);

/* y[n] = act_out( sum_k W[n][k] * act_in(x[k]) + bias[n] ), W bf16 [N][K], x f32.
 * act_in: 0 none, 1 SiLU (expf). Used for the timestep MLP and modulation. */
int iris_hip_gemv(float *d_y, const uint16_t *d_W, const float *d_x, const float *d_bias,
                  int N, int K, int act_in);

/* ---- row normalisations (one row of `cols` per block) ---- */
enum {
    IRIS_NORM_LN_MOD = 0,    /* LayerNorm (no affine) then (1 + scale) * n + shift     */
    IRIS_NORM_LN_SCALE = 1,  /* LayerNorm (no affine) then n * scale                   */
    IRIS_NORM_RMS = 2,       /* x * rsqrt(mean(x^2) + eps) * w, then * scale if given  */
};
typedef struct {
    const float *x; int ldx;          /* f32 input rows */
    void *out; int ldo; int out_bf16; /* output rows    */
    int rows, cols, mode;
    float eps;
    int split;                        /* (row % period) < split: set A, else set B */
    int period;                       /* 0: no period (row itself)                 */
    const float *shiftA, *scaleA, *wA;
    const float *shiftB, *scaleB, *wB;
} iris_norm_args_t;
int iris_hip_rownorm(const iris_norm_args_t *a);

/* Z-Image gated residual: x[r,:] += g[:] * RMSNorm(y[r,:]) * w[:] with
 * g = gate (gate_tanh 0), tanh(gate) (gate_tanh 1), or 1 when gate is NULL. */
int iris_hip_rms_gated_add(float *d_x, const float *d_y, const float *d_w, const float *d_gate,
                           int rows, int cols, float eps, int gate_tanh);

/* ---- attention pieces ---- */
/* Per (row, head) RMSNorm of Q and K (x w_q / w_k, rows < split use set A) and
 * rotary embedding from per-row cos/sin tables [rows][128] (pairs 2i, 2i+1).
 * qkv: bf16 rows holding Q at column 0, K at col_k, V at col_v (ld_qkv).
 * Writes Q' as bf16 [rows][heads*128], K' as [rows][kv_heads*128] and V
 * transposed to vt[kv head][d][ld_vt] (columns rows..ld_vt-1 zero-filled).
 * kv_heads 0 means heads (no grouped-query attention). */
typedef struct {
    const uint16_t *qkv; int ld_qkv, col_k, col_v;
    uint16_t *q_out, *k_out, *vt_out; int ld_vt;
    int rows, heads;
    const float *wqA, *wkA, *wqB, *wkB; int split;
    const float *cos_t, *sin_t;       /* [rows][128]; NULL = no rotation */
    int period;                       /* 0: none; else split and table row use row % period */
    float eps;
    int kv_heads;                     /* K / V heads; 0: same as heads */
    const float *kcos_t, *ksin_t;     /* K-side tables [rows][128]; NULL: the Q tables (SREF RoPE
                                         band control scales the reference rows' K bands,
                                         iris_transformer_flux.c:1272-1321) */
} iris_qkprep_args_t;
int iris_hip_qk_prepare(const iris_qkprep_args_t *a);
/* The K and V half of iris_hip_qk_prepare (q_out, wqA and wqB unused): K'
 * and V^T in one pass, for attention calls that normalise and rotate Q in
 * their own prologue (iris_attn_args_t.qn_wA). */
int iris_hip_kv_prepare(const iris_qkprep_args_t *a);

/* Flash attention over head_dim 128: O = softmax(Q K^T * scale) V per head.
 * Q [sq][ld_q], K [sk][ld_k] (head h at column h*128), Vt [h][128][ld_vt],
 * O [sq][ld_o]. Keys outside [kv_lo0, kv_hi0) U [kv_lo1, kv_hi1) are masked
 * (pass 0, sk, 0, 0 for none); with causal set, so are keys after the query's
 * own index. Query head h reads K / V head h / kv_group (grouped-query
 * attention; 0 means 1). batch / *_bstride run independent sequences. A query
 * with no unmasked key gets zeros. */
typedef struct {
    const uint16_t *q; const uint16_t *k; const uint16_t *vt; uint16_t *o;
    int ld_q, ld_k, ld_vt, ld_o;
    int sq, sk, heads, batch;
    long long q_bstride, k_bstride, vt_bstride, o_bstride;
    float scale;
    int kv_lo0, kv_hi0, kv_lo1, kv_hi1;
    int causal;                       /* 1: key j is masked for query i < j */
    int kv_group;                     /* query heads per K / V head; 0: 1 */
    int bias_from;                    /* keys >= bias_from get key_bias added to their logits */
    float key_bias;                   /* (SREF strength: log gamma on the reference keys,
                                         iris_transformer_flux.c:1328-1338); 0: none */
    /* Q prologue (apply_qk_norm + apply_rope_2d on Q, iris_transformer_flux.c:
     * 1464-1518, :1026-1048): when qn_wA is set, q holds the raw projection and
     * each (query, head) row is RMS-normalised (eps qn_eps) times qn_wA
     * (queries < qn_split) or qn_wB, then its pairs (2i, 2i+1) are rotated by
     * the per-pair tables rope_cos / rope_sin [sq][64] (entry i rotates dims
     * 2i, 2i+1; NULL: no rotation), before the product. Causal masking and
     * key_bias do not combine. */
    const float *qn_wA, *qn_wB;
    int qn_split;
    float qn_eps;
    const float *rope_cos, *rope_sin;
    /* Optional workspace (NULL: one block per 256 queries of a head). When
     * those blocks need two or more rounds of blocks (one per compute unit)
     * that are on average less than 80 % full and causal is 0, the key tiles of all
     * (query block, head) units are dealt out in equal ranges, one per
     * compute unit, and the partial softmax states of a unit done by several
     * blocks are merged by the last of them (deterministic order). At least
     * iris_hip_attention_workspace_bytes(), 256-byte aligned, zeroed once
     * before first use (calls leave it zeroed); calls sharing one workspace
     * must not overlap. */
    void *ws;
    size_t ws_bytes;
    /* Factored RoPE for the Q prologue, used instead of rope_cos / rope_sin
     * when rope_pos is set: pair i of a head belongs to axis i / 16 (four
     * axes of 16 pairs with one frequency table, as Flux's), query q sits at
     * position rope_pos[4 q + i / 16] on it, and the pair's cos and sin are
     * rope_axis[16 p + i % 16] and rope_axis[16 (rope_axis_len + p) + i % 16]
     * for that position p (0 <= p < rope_axis_len). The same values as the
     * per-query tables, from 8 bytes per query instead of 512. */
    const int16_t *rope_pos;
    const float *rope_axis;
    int rope_axis_len;
} iris_attn_args_t;
size_t iris_hip_attention_workspace_bytes(void);
int iris_hip_attention(const iris_attn_args_t *a);

/* ---- layout and conversion ---- */
/* NCHW f32 latent [C][hw] -> token rows bf16 out[row0 + p][C] (ld = C) */
int iris_hip_nchw_to_tokens(uint16_t *d_out, const float *d_latent, int C, int hw);
int iris_hip_f32_to_bf16(uint16_t *d_out, const float *d_in, size_t n);
int iris_hip_bf16_to_f32(float *d_out, const uint16_t *d_in, size_t n);
/* z += dt * v  (sign -1: z += dt * (-v)); with v2: v = v + g * (v2 - v) first (CFG) */
int iris_hip_euler(float *d_z, const float *d_v, const float *d_v2, float g, float dt, float sign,
                   size_t n);
/* Z-Image (ph, pw, c) patchify of [C][H][W] f32 -> bf16 rows [n_patch][ps*ps*C], and back */
int iris_hip_patchify(uint16_t *d_out, const float *d_latent, int C, int H, int W, int ps);
int iris_hip_unpatchify(float *d_latent, const float *d_patches, int C, int H, int W, int ps);
/* copy one f32 row vector into rows [r0, r1) of a [*, cols] matrix */
int iris_hip_fill_rows(float *d_x, const float *d_row, int r0, int r1, int cols);
/* x[r][c0 + j] = tanh(x[r][c0 + j]) for r < rows, j < len ([rows][ld] f32):
 * the gate columns of Z-Image's modulation vectors once per step (tanh(gate)
 * of zi_block_forward, iris_transformer_zimage.c:818-836), so the gated
 * residual adds take them with gate_tanh 0. */
int iris_hip_tanh_cols(float *d_x, int rows, int ld, int c0, int len);
/* out[r][c] = table[ids[r]][c] (bf16 table [vocab][cols] -> f32), zeros for
 * ids outside [0, vocab) */
int iris_hip_embed_rows(float *d_out, const uint16_t *d_table, const int *d_ids, int rows, int cols, int vocab);
/* f32 block copy: dst[r][c] = src[r][c] for r < rows, c < cols */
int iris_hip_copy_rows(float *d_dst, int ld_dst, const float *d_src, int ld_src, int rows, int cols);

/* ---- f32 kernel API support (iris_kernels.h) ---- */
/* f32 -> bf16 hi/lo split for f32-accurate GEMMs: the destination row holds
 * nseg (1..3) segments of K_pad columns (zero padded past the data), segment s
 * = lo(x) if bit s of lo_mask is set else hi(x), hi = bf16(x), lo = bf16(x - hi).
 * A = [hi|hi|lo] (mask 4) against W = [hi|lo|hi] (mask 2) over K = 3 * K_pad
 * sums Ahi.Whi + Ahi.Wlo + Alo.Whi in one GEMM. */
int iris_hip_split_rows(uint16_t *d_dst, const float *d_src, int rows, int cols, int ld_src, int K_pad, int nseg,
                        int lo_mask);
/* src [K][N] -> dst [N][nseg * K_pad] (transposed) */
int iris_hip_split_transpose(uint16_t *d_dst, const float *d_src, int K, int N, int K_pad, int nseg, int lo_mask);
/* bf16 [rows][cols] -> nseg zero-padded copies side by side [rows][nseg * K_pad] */
int iris_hip_pad_bf16(uint16_t *d_dst, const uint16_t *d_src, int rows, int cols, int K_pad, int nseg);
/* im2col rows for output pixels [pix0, pix0 + npix) of one [C][H][W] image,
 * columns (ic, kh, kw), split as above into [npix][nseg * K_pad] */
int iris_hip_im2col_split(uint16_t *d_dst, const float *d_in, int C, int H, int W, int kH, int kW, int stride,
                          int pad, int outW, int pix0, int npix, int K_pad, int nseg, int lo_mask);
/* op: 0 out = a + b, 1 out = a * b, 2 out = a + s * b, 3 out = silu(a), 4 out = silu(a) * b */
int iris_hip_elementwise(int op, float *d_out, const float *d_a, const float *d_b, float s, size_t n);
/* out[r][c] += bias[r] for c < cols */
int iris_hip_add_row_bias(float *d_out, const float *d_bias, int rows, int cols, int ld);
int iris_hip_rms_rows(float *d_out, const float *d_x, const float *d_w, int rows, int cols, float eps);
int iris_hip_softmax_rows(float *d_x, int rows, int cols);
/* x [batch][channels][spatial]; gamma / beta [channels] */
int iris_hip_group_norm(float *d_out, const float *d_x, const float *d_gamma, const float *d_beta, int batch,
                        int channels, int spatial, int groups, float eps);
int iris_hip_batch_norm(float *d_out, const float *d_x, const float *d_mean, const float *d_var,
                        const float *d_gamma, const float *d_beta, int batch, int channels, int spatial, float eps);
int iris_hip_upsample_nearest(float *d_out, const float *d_in, int planes, int H, int W, int sh, int sw);
/* [B][C][H][W] <-> [B][C*p*p][H/p][W/p], channel c*p*p + pi*p + pj = pixel (ph*p + pi, pw*p + pj) */
int iris_hip_space_to_depth(float *d_out, const float *d_in, int batch, int C, int H, int W, int p, int inverse);
/* f32 attention for head_dim <= 512, keys <= 12288: row r of q / o for
 * (batch b, head h) at b*q_sb + h*q_sh + r*ld, of k / v at b*k_sb + h*k_sh + r*ld */
int iris_hip_attention_f32(float *d_o, const float *d_q, const float *d_k, const float *d_v, int batch, int heads,
                           int sq, int sk, int hd, float scale, long long q_sb, long long q_sh, long long k_sb,
                           long long k_sh, int ld);

#ifdef __cplusplus
}
#endif
#endif
