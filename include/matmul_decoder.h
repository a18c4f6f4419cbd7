/*
 * matmul_decoder.h — public C ABI of the decoder, served on one MI355X (gfx950).
 *
 * Drop-in replacement for the reference header of the same name
 * (reference: include/matmul_decoder.h:1-474).  Every struct layout, enum
 * value and prototype below is ABI-identical to the reference so that C
 * callers compiled against the reference header, and the `static inline`
 * config helpers they inline, keep working unchanged.  The implementation
 * behind it is device resident: weights, KV cache and scratch live in one
 * HBM arena and each projection is a hand-written HIP kernel.
 *
 * Threading: a context is not thread safe; every entry point is synchronous
 * on return (the device stream is drained before control comes back).
 */
#ifndef MATMUL_DECODER_H
#define MATMUL_DECODER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MATMUL_DECODER_VERSION_MAJOR 1
#define MATMUL_DECODER_VERSION_MINOR 0
#define MATMUL_DECODER_VERSION_PATCH 0

/* Return codes (reference: include/matmul_decoder.h:30-37).
 * MATMUL_DECODER_ERR_RKNN keeps its value for ABI compatibility; here it
 * reports a HIP runtime / device failure. */
typedef enum {
    MATMUL_DECODER_OK = 0,
    MATMUL_DECODER_ERR_INVALID_ARG = -1,
    MATMUL_DECODER_ERR_MEMORY = -2,
    MATMUL_DECODER_ERR_FILE_IO = -3,
    MATMUL_DECODER_ERR_RKNN = -4,
    MATMUL_DECODER_ERR_UNSUPPORTED = -5,
} MatmulDecoderError;

/* Execution mode (reference: include/matmul_decoder.h:41-44).  Stored and
 * reported; on one GPU both values run the same kernels. */
typedef enum {
    EXEC_SINGLE_CORE = 0,
    EXEC_DUAL_CORE = 1,
} ExecutionMode;

/* Model architecture (reference: include/matmul_decoder.h:52-114).
 * Field order and types are part of the ABI. */
typedef struct {
    const char* name;           /* borrowed, for logging only */
    int hidden_dim;
    int num_q_heads;
    int num_kv_heads;           /* GQA: num_q_heads % num_kv_heads == 0 */
    int head_dim;
    int ffn_dim;
    int num_layers;
    int vocab_size;
    int max_seq_len;
    float rms_eps;
    float rope_theta;
    int tie_word_embeddings;

    float rope_scaling_factor;  /* stored, not applied (as in the reference) */
    int rope_scaling_type;

    int norm_type;              /* 0 = RMSNorm (the only one applied) */

    int rope_style;             /* 0 = interleaved pairs (2i,2i+1); 1 = split halves (i,i+d/2) */

    int ffn_act_type;           /* 0 = SwiGLU (the only one applied) */

    int has_qk_norm;            /* per-head RMSNorm on q and k after projection */

    int num_lm_heads;           /* > 1 selects the multi-head step_head path */
    int lm_head_vocab_size;     /* vocab of each head when num_lm_heads > 1 */

    int context_pool_mode;      /* accepted for compatibility; one arena serves all modes */

    int iommu_domain_id;        /* accepted for compatibility; unused on the GPU */

    ExecutionMode exec_mode;

    int disable_npu_lm_head;    /* 1 = fp16-weight lm_head with fp32 activations instead of INT8 */

    int max_batch_prefill;      /* prefill chunk size, 0 = 64 */
} MatmulDecoderConfig;

/* Qwen3-0.6B defaults (reference: include/matmul_decoder.h:119-144). */
static inline MatmulDecoderConfig matmul_decoder_config_qwen3_0_6b(void) {
    MatmulDecoderConfig c;
    c.name = "qwen3-asr-0.6b";
    c.hidden_dim = 1024;
    c.num_q_heads = 16;
    c.num_kv_heads = 8;
    c.head_dim = 128;
    c.ffn_dim = 3072;
    c.num_layers = 28;
    c.vocab_size = 151936;
    c.max_seq_len = 4096;
    c.rms_eps = 1e-6f;
    c.rope_theta = 1000000.0f;
    c.tie_word_embeddings = 1;
    c.rope_scaling_factor = 1.0f;
    c.rope_scaling_type = 0;
    c.norm_type = 0;
    c.rope_style = 0;
    c.ffn_act_type = 0;
    c.has_qk_norm = 1;
    c.num_lm_heads = 0;
    c.lm_head_vocab_size = 0;
    c.context_pool_mode = 0;
    c.iommu_domain_id = 1;
    c.exec_mode = EXEC_DUAL_CORE;
    c.disable_npu_lm_head = 0;
    c.max_batch_prefill = 64;
    return c;
}

/* Reference: include/matmul_decoder.h:149-153. */
static inline MatmulDecoderConfig matmul_decoder_config_qwen3_0_6b_single_core(void) {
    MatmulDecoderConfig c = matmul_decoder_config_qwen3_0_6b();
    c.exec_mode = EXEC_SINGLE_CORE;
    return c;
}

/* Code-predictor shape: 5 layers, 15 heads of 2048 (reference:
 * include/matmul_decoder.h:159-184). */
static inline MatmulDecoderConfig matmul_decoder_config_qwen3_tts_cp(void) {
    MatmulDecoderConfig c = matmul_decoder_config_qwen3_0_6b();
    c.name = "qwen3-tts-cp";
    c.num_layers = 5;
    c.vocab_size = 2048;
    c.max_seq_len = 20;
    c.tie_word_embeddings = 0;
    c.num_lm_heads = 15;
    c.lm_head_vocab_size = 2048;
    return c;
}

/* Weight quantisation of the layer projections (reference:
 * include/matmul_decoder.h:188-193).  QUANT_INT4 and QUANT_INT4_G128 both
 * load one scale per output column, as the reference loader does. */
typedef enum {
    QUANT_FP16 = 0,
    QUANT_INT8 = 1,
    QUANT_INT4 = 2,
    QUANT_INT4_G128 = 3,
} QuantizationType;

/* Reference: include/matmul_decoder.h:201-207. */
typedef struct {
    void* data;
    float* scales;
    int K;
    int N;
    QuantizationType quant_type;
} ProjectionWeight;

/* Reference: include/matmul_decoder.h:212-232. */
typedef struct {
    ProjectionWeight q_proj;
    ProjectionWeight k_proj;
    ProjectionWeight v_proj;
    ProjectionWeight o_proj;
    ProjectionWeight gate_proj;
    ProjectionWeight up_proj;
    ProjectionWeight down_proj;
    float* input_norm_weight;
    float* post_attn_norm_weight;
    float* q_norm_weight;
    float* k_norm_weight;
} LayerWeights;

/* Standalone KV cache object (reference: src/matmul_decoder.c:449-502).
 * Host-side fp32 [layer][max_seq][kv_head][head_dim], as in the reference;
 * the decoder's own cache is fp16 in the device arena. */
typedef struct MatmulKVCache MatmulKVCache;

MatmulKVCache* matmul_kv_cache_create(int num_layers, int num_kv_heads,
                                      int head_dim, int max_seq_len);
void matmul_kv_cache_clear(MatmulKVCache* cache);
int matmul_kv_cache_get_seq_len(const MatmulKVCache* cache);
void matmul_kv_cache_destroy(MatmulKVCache* cache);

typedef struct MatmulDecoderContext MatmulDecoderContext;

/* Load a model directory in the reference on-disk format (reference:
 * src/matmul_decoder.c:830-1309).  `config` NULL reads model_dir/config.json.
 * Returns NULL on failure with a diagnostic on stderr. */
MatmulDecoderContext* matmul_decoder_create(const char* model_dir,
                                            const MatmulDecoderConfig* config,
                                            QuantizationType quant_type,
                                            int max_seq_len);

/* Build a decoder from caller memory (reference: src/matmul_decoder.c:1311).
 * Projection data follows the on-disk formats: fp16 [K,N], int8 [K,N] plus
 * fp32 scales[N], or int4 [K,N/2] plus scales[N]. */
MatmulDecoderContext* matmul_decoder_create_from_weights(
    const MatmulDecoderConfig* config,
    const float* embeddings,
    const LayerWeights* layers,
    const float* lm_head,
    QuantizationType quant_type,
    int max_seq_len);

/* One greedy token (reference: src/matmul_decoder.c:1430-1634).
 * output_logits == NULL is prefill mode: no lm_head, returns 0. */
int matmul_decoder_step(MatmulDecoderContext* ctx,
                        int token_id,
                        const float* embedding,
                        float* output_logits);

/* Declared but never defined by the reference (include/matmul_decoder.h:320);
 * defined here as step() with a required logits buffer. */
int matmul_decoder_step_get_logits(MatmulDecoderContext* ctx,
                                   int token_id,
                                   const float* embedding,
                                   float* logits_out);

/* Reference: src/matmul_decoder.c:1636-1742. */
int matmul_decoder_step_head(MatmulDecoderContext* ctx,
                             int token_id,
                             const float* embedding,
                             int lm_head_idx,
                             float* output_logits);

/* Reference: src/matmul_decoder.c:1901-2065. */
int matmul_decoder_prefill_batch(MatmulDecoderContext* ctx,
                                 const float* embeddings, int M);

void matmul_decoder_clear_kv_cache(MatmulDecoderContext* ctx);
int matmul_decoder_get_seq_len(const MatmulDecoderContext* ctx);
const MatmulDecoderConfig* matmul_decoder_get_config(const MatmulDecoderContext* ctx);

/* Reference: include/matmul_decoder.h:372-382, filled by step() as in
 * src/matmul_decoder.c:1551-1560, 1616-1623 (prefill_batch and step_head
 * leave them alone).  On the GPU, device times come from events on the
 * step's stream:
 *   total_ms    host wall time of the call;
 *   matmul_ms   the projections (with the norm, residual and SwiGLU they
 *               carry).  A step whose layers and lm_head are one launch
 *               counts that whole launch here, unless MDX_PROFILE=1;
 *   lm_head_ms  the lm_head when it is a kernel of its own (0 in prefill
 *               mode and inside the one launch unless MDX_PROFILE=1);
 *   cpu_ops_ms  QK-norm, RoPE, KV append and attention (0 unless
 *               MDX_PROFILE=1: they are fused into the same launch);
 *   rebind_ms   time the one launch's stages wait for each other's results
 *               (0 unless MDX_PROFILE=1; there are no B buffers to rebind);
 *   convert_ms  total_ms minus the device times above (uploads, copies of
 *               the logits, launch and synchronisation).
 * MDX_PROFILE=1 at creation times every stage of the one launch
 * (per-workgroup timestamps, medians over workgroups, scaled to the launch's
 * event time), at the cost of a 0.9 MB copy per step. */
typedef struct {
    float total_ms;
    float matmul_ms;
    float rebind_ms;
    float convert_ms;
    float cpu_ops_ms;
    float lm_head_ms;
    int n_steps;
} MatmulDecoderStats;

void matmul_decoder_get_stats(const MatmulDecoderContext* ctx, MatmulDecoderStats* stats);
void matmul_decoder_destroy(MatmulDecoderContext* ctx);

/* Reference: include/matmul_decoder.h:391-412. */
typedef struct {
    int top_k;
    float top_p;
    float temperature;
    float repeat_penalty;
    const int* repeat_tokens;
    int n_repeat_tokens;
} SamplingParams;

static inline SamplingParams sampling_params_greedy(void) {
    SamplingParams p;
    p.top_k = 1;
    p.top_p = 1.0f;
    p.temperature = 1.0f;
    p.repeat_penalty = 1.0f;
    p.repeat_tokens = NULL;
    p.n_repeat_tokens = 0;
    return p;
}

/* Greedy regardless of top_k, as in the reference (src/matmul_decoder.c:2316-2324). */
int matmul_sample_token(const float* logits, int vocab_size, SamplingParams* params);

typedef void (*GenerateCallback)(int token_id, const char* token_text, void* user_data);

/* Declared but never defined by the reference (include/matmul_decoder.h:448);
 * defined here: feeds the prompt in prefill mode, then samples up to
 * max_new_tokens, calling `callback` (token_text NULL) after each token. */
int matmul_decoder_generate(MatmulDecoderContext* ctx,
                            const int* prompt_tokens,
                            int n_prompt,
                            int max_new_tokens,
                            SamplingParams* params,
                            GenerateCallback callback,
                            void* user_data);

/* Reference: src/matmul_decoder.c:2182-2312.  Numbers are parsed with strtod,
 * so exponents such as 1e-06 are honoured; "rope_style" and
 * "max_batch_prefill" are read in addition to the reference's keys. */
int matmul_decoder_load_config(const char* json_path, MatmulDecoderConfig* config);

/* Declared but never defined by the reference (include/matmul_decoder.h:467).
 * Converts a local HuggingFace checkpoint (config.json + *.safetensors, F32/
 * F16/BF16, sharded or not) into the on-disk format the loader reads, with
 * the projections as fp16 [K,N] (QUANT_FP16) or quantised files (QUANT_INT8,
 * QUANT_INT4); the file layout follows the reference exporter
 * examples/qwen3_asr/export_weights.py:128-216.  Returns 0 or a negative
 * MatmulDecoderError. */
int matmul_decoder_export_hf_model(const char* hf_model_path,
                                   const char* output_dir,
                                   QuantizationType quant_type);

#ifdef __cplusplus
}
#endif

#endif /* MATMUL_DECODER_H */
