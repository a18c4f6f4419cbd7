/*
 * mdx_ext.h — additive C entry points of the MI355X decoder library.
 *
 * None of these exist in the reference; they sit beside the drop-in ABI
 * (matmul_decoder.h, rknn_matmul_parallel.h) and never change its
 * behaviour.  They serve three groups of callers:
 *   - test hooks the reference API lacks (KV fill/read, last-token logits
 *     after a batch prefill);
 *   - single-kernel entry points so parity tests can check one projection,
 *     one attention call or one GEMM against the oracle;
 *   - device-resident loops and timers for measurement (greedy decode with
 *     the token fed back on the device, GEMV bandwidth timing).
 * Every function returns 0 (or a token id) on success and a negative
 * MatmulDecoderError code on failure.
 */
#ifndef MDX_EXT_H
#define MDX_EXT_H

#include <stddef.h>
#include <stdint.h>

#include "matmul_decoder.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Library build information: "<version> gfx950". */
const char* mdx_version(void);
/* Number of visible GPUs (0 when the HIP runtime finds none). */
int mdx_device_count(void);
/* Last HIP runtime message recorded by the library (thread-local). */
const char* mdx_last_error(void);
/* `iters` device-to-device copies of `bytes` (a plain copy kernel of known
 * traffic: the calibration run for HBM byte counters). */
int mdx_copy_probe(size_t bytes, int iters);

/* Decode path of a context:
 *   1  a step is one launch of the whole model (the 0.6B layer shape with one
 *      weight kind and the single INT8 lm_head);
 *   2  the layers are one launch and the lm_head a per-stage kernel after it
 *      (the same layer shape with several lm_heads or the fp16 lm_head);
 *   0  the per-stage kernel sequence.
 * MDX_PERSIST=0 in the environment at creation selects 0.  The launch is an
 * ordinary one; if its waits time out (grid not co-resident) the step is run
 * again as a cooperative launch, and the context keeps launching
 * cooperatively. */
int mdx_decode_path(const MatmulDecoderContext* ctx);
/* Test hook: the next one-launch step polls each exchange at most `rounds`
 * times before giving up (0: the default), which forces the timeout-and-retry
 * path without any workgroup waiting long. */
int mdx_debug_persist_spin_limit(MatmulDecoderContext* ctx, unsigned rounds);
/* Test hook: how the one-launch step reads the K/V rows.  -1 (the default):
 * with non-temporal loads once the cache holds more than 96 MB, so that a long
 * context does not evict the lm_head from the last-level cache; 0 / 1: always
 * ordinary / always non-temporal.  The results are the same either way. */
int mdx_debug_persist_kv_stream(MatmulDecoderContext* ctx, int mode);
/* Test hook: where the one-launch step's per-head exchanges (qkv rows to
 * attention, partial records to the merge) travel.  -1 (the default): in the
 * L2 of the XCD that the KV head's workgroups share, through a cacheable word
 * buffer, until a step times out, then through the uncached words like the
 * other exchanges; 0 / 1: always through the uncached words / always local.
 * The results are the same bits either way.  Returns
 * MATMUL_DECODER_ERR_UNSUPPORTED when the context has no local buffer. */
int mdx_debug_persist_local_exchange(MatmulDecoderContext* ctx, int mode);
/* Test hook: before the next cooperative retry, leave exchange words tagged
 * with the epoch that retry would accept first (what a workgroup of the
 * timed-out launch that started late could have written); the retry must
 * clear them and still produce the undisturbed result. */
int mdx_debug_persist_poison_retry(MatmulDecoderContext* ctx);
/* Test hook (process-wide): on != 0 makes the batch-prefill projections use
 * the GEMM that loads its activation fragments per wave in rounds instead of
 * the one that stages the block's activation panel in LDS (same sums, bit for
 * bit); takes effect for graphs captured afterwards.  Returns the previous
 * setting. */
int mdx_debug_gemm_rounds(int on);
/* The K-split count of a batch-prefill projection that is split over blocks
 * (kind MDX_W_F16/I8/I4, N outputs, K inputs), with the K-blocks per split in
 * *per_split (may be NULL): split s covers K-blocks [s*per, (s+1)*per), and
 * no split is empty.  Host arithmetic only (no device call); -1 for invalid
 * arguments. */
int mdx_debug_gemm_splits(int kind, int N, int K, int* per_split);
/* Host enumeration of the K/V cache rows the one-launch decode step reads,
 * with the kernel's own split and row functions: every position
 * 0 <= pos < max_seq, every attention split, every round of k_passes (4 or
 * 5) 16-position passes the step requests.  Returns the number of rows
 * outside [0, pos] (0 when every address lies in the cache rows written so
 * far), -1 for invalid arguments; *n_checked (may be NULL) receives the
 * number of row addresses checked.  No device call. */
long long mdx_debug_persist_kv_rows(int max_seq, int k_passes, long long* n_checked);

/* One decode step of the one-launch path with per-workgroup timestamps
 * (100 MHz device clock) at every stage boundary: out[256][E] with E
 * events per workgroup: 16 per layer, 3 for the lm_head, then the
 * workgroup's XCD index.  Returns E, or
 * MATMUL_DECODER_ERR_UNSUPPORTED unless the decode path is 1. */
int mdx_trace_step(MatmulDecoderContext* ctx, int token_id, unsigned long long* out, int cap);

/* matmul_decoder_step with the lm_head and argmax but without copying the
 * logits to the host (the pybind step_get_token path). */
int mdx_step_token(MatmulDecoderContext* ctx, int token_id, const float* embedding);

/* ---- test hooks on a decoder context ---- */

/* Fill KV rows [0, n_pos) of every layer with N(0,1) values rounded to fp16
 * (streams "kv/k/LL" and "kv/v/LL" of mdx_synth_fill_normal, seed `seed`)
 * and set the sequence length to n_pos. */
int mdx_kv_fill_normal(MatmulDecoderContext* ctx, int n_pos, uint64_t seed);
/* Read KV rows [pos0, pos0+n) of one layer as fp32 [n][kv_heads*head_dim]. */
int mdx_kv_read(const MatmulDecoderContext* ctx, int layer, int pos0, int n, float* k, float* v);
/* Batch prefill of M rows, then final norm + lm_head on the last row only.
 * Writes logits when non-NULL and returns the argmax. */
int mdx_prefill_logits(MatmulDecoderContext* ctx, const float* embeddings, int M, float* logits);
/* n_steps greedy tokens starting from token `first_token`, with each argmax
 * fed back on the device (no host round trip between steps).  Tokens go to
 * out_tokens[n_steps]; *device_ms (optional) receives the GPU time of the
 * whole loop.  Equivalent to n_steps calls of matmul_decoder_step with the
 * previous result as token_id. */
int mdx_generate_greedy(MatmulDecoderContext* ctx, int first_token, int n_steps, int* out_tokens,
                        float* device_ms);
/* Average device microseconds of one launch of a layer projection kernel
 * ("qkv", "o", "gate_up", "down", "lm_head"), or of the four launches that
 * make one layer's seven projections with their RMSNorms ("layer"), timed
 * with HIP events over `iters` repetitions cycling through all layers
 * (distinct weights).  *bytes receives the algorithmic HBM bytes of one
 * repetition. */
int mdx_time_projection(MatmulDecoderContext* ctx, const char* which, int iters, float* avg_us,
                        double* bytes);
/* Device milliseconds of one M-row batch prefill through all layers (timed
 * with HIP events, KV position restored afterwards). */
int mdx_time_prefill(MatmulDecoderContext* ctx, const float* embeddings, int M, int iters,
                     float* avg_ms);

/* Average device microseconds of one GEMV y = fp16(x) . W (x per-column
 * scale) with kind 1 (int8) or 0 (fp16) weights of [K,N], timed with HIP
 * events over `iters` back-to-back launches that cycle through `copies`
 * distinct weight buffers (enough copies defeat the device caches), issued
 * from a captured graph of one launch per copy when iters is a multiple of
 * copies (MDX_GRAPHS=0: one by one).  The buffers hold a fixed pattern; the
 * kernel is the decoder's per-stage GEMV. */
int mdx_time_gemv(int kind, int K, int N, int copies, int iters, float* avg_us);

/* ---- single-kernel entry points (weights in the on-disk layout) ---- */

/* kind: 0 fp16 [K,N] (uint16 bits), 1 int8 [K,N], 2 int4 [K,N/2] (byte
 * (k,j): column 2j in the low nibble, 2j+1 in the high nibble), 3 fp32
 * rows [N,K] with fp32 x (the CPU GEMV), 4 fp16 rows [N,K] with fp32 x.
 * scales[N] may be NULL.  y[N] fp32 = fp16(x) . W (x scale). */
int mdx_debug_gemv(int kind, int K, int N, const void* w, const float* scales, const float* x,
                   float* y);
/* M-row MFMA projection, M <= 64: y[M,N] = fp16(x[M,K]) . W (x scale). */
/* One residual projection of the batch prefill (the o and down stages):
 * hidden[M][N] += fp16(x) . W (x scale), then x16_out[M][N] =
 * fp16((hidden * rms) * norm_w) per row when norm_w is given.  kind and the
 * weight / scale formats as mdx_debug_gemm; hidden is updated in place. */
int mdx_debug_gemm_residual(int kind, int M, int K, int N, const void* w, const float* scales,
                            const float* x, float* hidden, const float* norm_w, float eps,
                            uint16_t* x16_out);
int mdx_debug_gemm(int kind, int M, int K, int N, const void* w, const float* scales,
                   const float* x, float* y);
/* One decode attention layer at position pos: qkv fp32 [nq*hd + 2*nkv*hd]
 * (the projection output, before QK-norm and RoPE), cache rows fp16 bits
 * [pos][nkv*hd] for positions < pos; q_norm/k_norm [hd] may be NULL.
 * Returns out fp32 [nq*hd] (the fp16 value the kernel stores, widened) and
 * the appended fp16 K/V row of position pos. */
int mdx_debug_attn_decode(int nq, int nkv, int hd, int pos, int rope_style, float theta, float eps,
                          const float* q_norm, const float* k_norm, const float* qkv,
                          const uint16_t* k16, const uint16_t* v16, float* out, uint16_t* k_new,
                          uint16_t* v_new);
/* Causal batch attention of M query rows at positions S..S+M-1 over cache
 * rows [0, S+M) (the batch's own K/V already appended). */
int mdx_debug_attn_prefill(int nq, int nkv, int hd, int S, int M, const float* q,
                           const uint16_t* k16, const uint16_t* v16, float* out);
/* QK-norm + RoPE + KV append of one token at position pos through the
 * batch-prefill kernel: qkv fp32 [nq*hd + 2*nkv*hd]; returns q fp32 and
 * the fp16 k,v rows. */
int mdx_debug_qk_rope(int nq, int nkv, int hd, int pos, int rope_style, float theta, float eps,
                      const float* q_norm, const float* k_norm, const float* qkv, float* q_out,
                      uint16_t* k16, uint16_t* v16);
/* Fused RMSNorm + lm_head + argmax on one hidden vector; lm_kind as
 * mdx_debug_gemv's 1 (int8 rows [N,K] + scales), 3 or 4.  Returns the
 * argmax and writes logits[N]. */
int mdx_debug_lmhead(int lm_kind, int K, int N, const void* w_rows, const float* scales,
                     const float* hidden, const float* norm_w, float eps, float* logits);

/* Runs the sampler of matmul_decoder_step_sample on host logits[V]
 * (uploaded, penalised, sampled, copied back).  out[0] = token, out[1] =
 * candidates kept after top-p; top_idx/top_val (may be NULL) receive the k
 * candidates, k = clamp(top_k, 1, V), by descending tempered value.
 * Returns 0 or a negative error. */
int mdx_debug_sample(const float* logits, int V, const SamplingParams* params, float uniform,
                     int* out, int* top_idx, float* top_val);

/* ---- device-side sampling ---------------------------------------------- */

#define MDX_SAMPLE_MAX_REPEAT 4096

/* One decode step (as matmul_decoder_step with a logits buffer) followed by
 * sampling on the device from the logits it leaves in HBM, so non-greedy
 * decoding copies no logits to the host (output_logits may be NULL; when
 * given it receives the step's logits before the penalty).  Reference:
 * src/cpu_ops.c:593-648 (top_k_sample_f32) and the SamplingParams of
 * include/matmul_decoder.h:391-398, with these definitions:
 *   - repeat_penalty p != 1: each distinct listed token's logit l becomes
 *     l / p if l > 0, else l * p (the reference declares the field and
 *     applies it nowhere);
 *   - temperature T: v = l / T when T != 1, as the reference divides;
 *   - top_k k = clamp(top_k, 1, V), at most MDX_SAMPLE_MAX_TOP_K: the k
 *     largest v, ties to the lower index, in descending order;
 *     e_j = expf(v_j - v_0), summed in that order;
 *   - top_p < 1: only the shortest prefix whose running sum reaches
 *     top_p * sum is kept (the reference's top_p_sample_f32 returns the
 *     argmax instead);
 *   - uniform u in [0,1] replaces rand() / RAND_MAX: r = u * sum, the token
 *     is the first candidate whose running sum exceeds r, else the last.
 * top_k <= 1 gives the argmax of the penalised, tempered logits.  Returns
 * the token, or a negative error (INVALID_ARG for out-of-range parameters
 * or repeat tokens, more than MDX_SAMPLE_MAX_REPEAT of them, or a bad
 * token/full cache as matmul_decoder_step; UNSUPPORTED for a context with
 * several lm_heads).  Not part of the reference ABI. */
int matmul_decoder_step_sample(MatmulDecoderContext* ctx, int token_id, const float* embedding,
                               const SamplingParams* params, float uniform, float* output_logits);

/* No counterpart in the reference: the device sampler for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid hipMalloc).  A variant of mdx_debug_sample without the repetition
 * penalty that takes device pointers: logits[V] (read only), out[2] (token,
 * candidates kept after top-p), top_idx/top_val[top_k] (may be NULL); k =
 * top_k must be in [1, min(V, MDX_SAMPLE_MAX_TOP_K)] (larger k is rejected
 * with a message: the scratch holds 1024 candidates).  Enqueued on `stream`
 * (NULL: the default stream); returns without synchronising.  It calls no
 * allocator: its 141 KB of scratch is a static device array of the library,
 * one per GPU, held until the process ends.  The first call on each device
 * looks up that array's device address (hipGetSymbolAddress), so make it
 * outside stream capture; later calls can be captured (they launch kernels
 * only, no memset nodes).  Calls that overlap on one GPU
 * share that scratch and race; serialise them.  Returns 0, -1 for bad
 * arguments, -4 on a HIP failure. */
int mdx_sample_topk_noalloc(const float* logits, int V, float temperature, int top_k, float top_p,
                            float uniform, int* out, int* top_idx, float* top_val, void* stream);

/* Device memory and synchronous copies on the current device, for callers
 * and tests that hand device pointers to the device-pointer entry points.
 * Return 0 or a negative error. */
int mdx_device_malloc(void** ptr, size_t bytes);
int mdx_device_free(void* ptr);
int mdx_memcpy_h2d(void* dst, const void* src, size_t bytes);
int mdx_memcpy_d2h(void* dst, const void* src, size_t bytes);
int mdx_device_synchronize(void);

/* ---- host helpers shared with tools (no GPU needed) ---- */

/* INT8 lm_head quantiser of the reference (per vocab row of the fp16 copy):
 * scale = max|v|/127, q = clamp((int)roundf(v * (127/max)), -128, 127). */
void mdx_quantize_lm_head(int8_t* q, float* scales, const uint16_t* lm_f16, int V, int K);
/* Round-to-nearest-even fp32 -> fp16 bits, and back. */
uint16_t mdx_f32_to_f16(float f);
float mdx_f16_to_f32(uint16_t h);
/* SplitMix64 + Box-Muller N(mean, std) stream, in chunks of 2^20 values,
 * seeded per tensor with mdx_synth_seed(base, name). */
uint64_t mdx_synth_seed(uint64_t base, const char* name);
void mdx_synth_fill_normal(float* out, size_t n, uint64_t seed, double mean, double std);

/* Write a synthetic model directory in the reference on-disk format:
 * config.json, embeddings.bin ~N(0, 0.02) fp32, layers/layer_LL/ with norm
 * weights 1.0 and projections ~N(0, 0.02): quant 0 writes fp16 [K,N]
 * <proj>.bin; quant 1 quantises per column (scale = max|col|/127) into
 * <proj>_weight.bin int8 [K,N] + <proj>_scales.bin fp32; quant 2 writes
 * int4 [K,N/2] (column 2j low nibble) with fp16-representable scales
 * max|col|/7.  The lm_head is tied to the embeddings.  Returns 0. */
int mdx_synth_write_model(const char* dir, const MatmulDecoderConfig* cfg, int quant,
                          uint64_t seed);

#ifdef __cplusplus
}
#endif

#endif
