/*
 * iris_qwen3.h - Qwen3 text encoder on the HIP layer.
 *
 * Mirrors the model half of the reference's iris_qwen3.h (constants :20-30,
 * model API :83-105): a decoder-only Qwen3 (RMSNorm, GQA attention with
 * per-head QK-RMSNorm and rotary embedding, SwiGLU MLP) whose hidden states
 * after layers 8, 17 and 26 are concatenated into the [seq, 3*hidden] text
 * embedding Flux consumes, or whose layer num_layers-2 output is Z-Image's
 * [seq, hidden] caption embedding. Weights stay resident in HBM as bf16; the
 * forward runs on the library stream with the same GEMM, norm and attention
 * kernels as the denoiser. The tokenizer half (qwen3_tokenizer_*,
 * qwen3_encoder_*, qwen3_encode_text*) is host string processing and is not
 * part of this library.
 */
#ifndef IRIS_QWEN3_H
#define IRIS_QWEN3_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QWEN3_VOCAB_SIZE       151936
#define QWEN3_MAX_SEQ_LEN      512
#define QWEN3_RMS_NORM_EPS     1e-6f
#define QWEN3_ROPE_THETA       1000000.0f
/* hidden states captured after these layers (0-indexed) for Flux */
#define QWEN3_OUTPUT_LAYER_1   8
#define QWEN3_OUTPUT_LAYER_2   17
#define QWEN3_OUTPUT_LAYER_3   26

typedef struct qwen3_model qwen3_model_t;

/* Loads config.json and the bf16 safetensors shards of a HuggingFace Qwen3
 * directory (model.safetensors.index.json, else model-00001-of-00002 and
 * model-00002-of-00002, else model.safetensors) and uploads the weights.
 * Replaces qwen3_model_load (iris_qwen3.c:1578-1660). NULL on failure. */
qwen3_model_t *qwen3_model_load(const char *model_dir);

/* Replaces qwen3_model_free (iris_qwen3.c). */
void qwen3_model_free(qwen3_model_t *model);

/* Embeds input_ids[seq_len] and runs the layers up to the last extracted one.
 * attention_mask (1 real, 0 padding; NULL = all real) must be a run of ones
 * followed by zeros, as qwen3_pad_tokens makes it; keys at padding positions
 * and keys after the query are masked. Returns malloc'd f32
 * [seq_len][text_dim] (3*hidden in Flux mode, hidden in Z-Image mode), NULL on
 * error. Replaces qwen3_forward (iris_qwen3.c:1072-1200). */
float *qwen3_forward(qwen3_model_t *model, const int *input_ids, const int *attention_mask, int seq_len);

/* No counterpart in the reference, which sets the mode through its encoder
 * (qwen3_set_extraction_mode, iris_qwen3.h:128-134): 0 = Flux (layers 8, 17,
 * 26 -> [seq, 3*hidden], the default), 1 = Z-Image (layer num_layers-2 ->
 * [seq, hidden]). */
void qwen3_model_set_extraction_mode(qwen3_model_t *model, int mode);
int qwen3_model_text_dim(const qwen3_model_t *model);

/* No counterpart in the reference: a random-init model of the given
 * architecture (head_dim 128, rope theta 1e6) with the seeded generator of
 * iris_synth.h, for benchmarks. Weights ~ N(0, 0.02), norm weights
 * 1 + N(0, 0.02). */
qwen3_model_t *qwen3_model_create_synthetic(int hidden, int intermediate, int heads, int kv_heads, int layers,
                                            int vocab, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif
