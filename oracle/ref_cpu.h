/*
 * ref_cpu.h — the oracle: a scalar C restatement of the reference decoder's
 * CPU path (reference: src/cpu_ops.c, src/matmul_decoder.c).
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker or as the timed CPU baseline.  The product (the HIP decoder under
 * rknn-matmul-parallel_amd/) never links or calls it.
 *
 * Every function names the reference file:line it follows.  Arithmetic is
 * plain fp32 C compiled with -ffp-contract=off: every multiply and add rounds
 * separately, except where the reference uses a fused NEON intrinsic
 * (vfmaq_f32), which is restated with fmaf().  NEON lane orders are
 * reproduced where the reference's result depends on them (four partial
 * sums reduced as (l0+l1)+(l2+l3), the vaddvq_f32 order).
 *
 * Projections go through the NPU in the reference; the NPU's accumulation
 * order is not published (include/rknn_matmul_api.h:72,76 give only the type
 * names).  The oracle defines it as: every product fp16(x)*w is exact in fp32
 * and is added to an fp32 accumulator in increasing k.
 */
#ifndef MDX_ORACLE_REF_CPU_H
#define MDX_ORACLE_REF_CPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 <-> fp32, round to nearest even (reference: src/cpu_ops.c:383-406,
 *      vcvt_f16_f32 under the default FPCR rounding mode) ---- */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_vec_f32_to_f16(uint16_t* dst, const float* src, size_t n);
void orc_vec_f16_to_f32(float* dst, const uint16_t* src, size_t n);

/* ---- generator restatement: SplitMix64 + Box-Muller, chunked streams ---- */
uint64_t orc_seed_for(uint64_t base, const char* name);
void orc_fill_normal_f32(float* out, size_t n, uint64_t seed, double mean, double std);

/* ---- element-wise and reduction ops (reference: src/cpu_ops.c) ---- */
void orc_rms_norm(float* out, const float* x, const float* w, int dim, float eps);
void orc_rope_tables(float* cos_t, float* sin_t, int max_seq, int head_dim, float theta);
void orc_apply_rope(float* x, const float* cos_row, const float* sin_row,
                    int num_heads, int head_dim, int rope_style);
void orc_apply_rope_batch(float* x, int M, int start_pos, int num_heads, int head_dim,
                          float theta, int rope_style);
void orc_attention(float* out, const float* q, const float* k_cache, const float* v_cache,
                   int num_q_heads, int num_kv_heads, int head_dim, int seq_len);
void orc_attention_batch_causal(float* out, const float* q_batch, const float* k_batch,
                                const float* v_batch, const float* k_cache,
                                const float* v_cache, int M, int num_q_heads,
                                int num_kv_heads, int head_dim, int cache_seq_len);
void orc_silu_mul(float* out, const float* gate, const float* up, int dim);
void orc_vec_add(float* dst, const float* src, int n);
int orc_argmax(const float* x, int n);
/* Top-k sampling with a given uniform (src/cpu_ops.c:593-648); see ref_cpu.c. */
int orc_sample_topk(float* x, int vocab_size, const int* rep, int n_rep, float penalty, int k,
                    float temperature, float top_p, float u, int* top_idx, float* top_val, int* kept);

/* ---- projections on the reference weight layout W[K,N] row-major ---- */
/* Projection accumulation order: 0 increasing k (default), 1 four
 * interleaved sums combined (s0+s1)+(s2+s3), used only to measure the
 * order sensitivity of end-to-end results. */
void orc_set_accum_order(int order);
/* y[m,n] = sum_k fp16(x[m,k]) * W[k,n]                      (NPU type 1) */
void orc_matmul_f16(float* y, const float* x, const uint16_t* w, int M, int K, int N);
/* y[m,n] = scale[n] * sum_k fp16(x[m,k]) * q[k,n]           (NPU type 5) */
void orc_matmul_i8(float* y, const float* x, const int8_t* q, const float* scale,
                   int M, int K, int N);
/* INT4: byte (k, n/2) holds column n even in its low nibble, n odd in its
 * high nibble, two's complement in [-8,7]; y as for INT8.  scale may be NULL
 * (unscaled), as may the INT8 one. */
void orc_matmul_i4(float* y, const float* x, const uint8_t* q, const float* scale,
                   int M, int K, int N);
/* CPU lm_head fallback, W[N,K] rows, fp32 x (reference:
 * src/matmul_decoder.c:572-616 and :511-566). */
void orc_gemv_rows_f16(float* out, const float* x, const uint16_t* w, int N, int K);
void orc_gemv_rows_f32(float* out, const float* x, const float* w, int N, int K);

/* INT8 lm_head quantiser (reference: src/matmul_decoder.c:1216-1244).
 * lm_head_f16 is [V,K] fp16; q is written [V,K] (row per vocab entry). */
void orc_quantize_lm_head(int8_t* q, float* scales, const uint16_t* lm_head_f16, int V, int K);

/* ---- the decoder (reference: src/matmul_decoder.c:830-2065) ---- */
typedef struct orc_model orc_model;

typedef struct {
    int hidden_dim, num_q_heads, num_kv_heads, head_dim, ffn_dim, num_layers, vocab_size;
    float rms_eps, rope_theta;
    int tie_word_embeddings, rope_style, has_qk_norm;
    int num_lm_heads, lm_head_vocab_size;
    int disable_npu_lm_head, max_batch_prefill;
} orc_config;

/* quant: 0 fp16, 1 int8, 2 int4.  kv_fp16: 1 rounds K/V to fp16 when they
 * are written (as the GPU decoder's fp16 cache does), 0 keeps fp32 (the
 * reference). */
orc_model* orc_model_open(const char* dir, const orc_config* cfg, int quant, int max_seq,
                          int kv_fp16);
void orc_model_close(orc_model* m);
int orc_model_step(orc_model* m, int token_id, const float* embedding, float* logits);
int orc_model_step_head(orc_model* m, int token_id, const float* embedding, int head,
                        float* logits);
int orc_model_prefill_batch(orc_model* m, const float* embeddings, int M);
int orc_model_seq_len(const orc_model* m);
void orc_model_set_seq_len(orc_model* m, int n);
/* KV test hook: positions [0,n_pos) of every layer from N(0,1) streams
 * named "kv/k/LL" and "kv/v/LL", then seq_len = n_pos. */
int orc_model_kv_fill_normal(orc_model* m, int n_pos, uint64_t seed);
/* Copies of the cache rows (fp32 view) and of the last hidden state. */
int orc_model_kv_read(const orc_model* m, int layer, int pos0, int n, float* k, float* v);
void orc_model_last_normed(const orc_model* m, float* out);
/* The lm_head the model holds, for bit-exact comparison. */
const int8_t* orc_model_lm_q(const orc_model* m);
const float* orc_model_lm_scales(const orc_model* m);

#ifdef __cplusplus
}
#endif

#endif
