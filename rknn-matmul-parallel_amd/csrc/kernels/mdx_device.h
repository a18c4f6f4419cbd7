/*
 * mdx_device.h — the thin C ABI between the host C runtime and the HIP
 * kernels for gfx950.  Plain C types only: device pointers are `void*`,
 * streams and graphs are opaque handles.  Every launcher returns 0 or a
 * negative MatmulDecoderError code and never synchronises.
 *
 * Device weight layout (all projections): W^T, one row per output column
 * n, K contiguous.  fp16 rows are K*2 bytes, int8 rows K bytes, int4 rows
 * K/2 bytes made of 32-bit words of 8 consecutive k: bits [4i+3:4i] hold
 * k=2i and bits [4i+19:4i+16] hold k=2i+1 (i = 0..3), two's complement
 * [-8,7].  fp32 rows (multi-head lm_heads) are K*4 bytes.  Optional fp32
 * per-row scales [N].
 */
#ifndef MDX_DEVICE_H
#define MDX_DEVICE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { MDX_W_F16 = 0, MDX_W_I8 = 1, MDX_W_I4 = 2, MDX_W_F32 = 3 };

/* One (possibly merged) projection resident in HBM. */
typedef struct {
    const void* w;          /* [N][K] in the layout above */
    const float* scale;     /* [N] or NULL */
    int kind;               /* MDX_W_* */
    int K, N;
} mdx_wdesc;

/* Per-context decode state, resident in device memory. */
typedef struct {
    int pos;                /* position being written (KV rows [0,pos) are valid) */
    int token;              /* input token when mode == 0; argmax output feeds it */
    int mode;               /* 0 = gather embeddings[token], 1 = use the uploaded embedding */
    int argmax;             /* last lm_head argmax */
    int n_out;              /* tokens appended to the greedy output list */
    int pad[3];
} mdx_state;

/* ---- runtime wrappers (mdx_rt.hip) ---- */
int mdxrt_device_count(void);
const char* mdxrt_last_error(void);
int mdxrt_malloc(void** p, size_t bytes);
int mdxrt_free(void* p);
int mdxrt_host_alloc(void** p, size_t bytes);     /* pinned */
/* Uncached device memory from a process-lifetime pool (never freed: a
 * released buffer goes back to the pool).  Not cleared: the caller clears it
 * on its stream. */
int mdxrt_uc_acquire(void** p, size_t bytes);
int mdxrt_uc_release(void* p);
int mdxrt_host_free(void* p);
int mdxrt_h2d(void* dst, const void* src, size_t bytes);
int mdxrt_d2h(void* dst, const void* src, size_t bytes);
int mdxrt_h2d_async(void* dst, const void* src, size_t bytes, void* stream);
int mdxrt_d2h_async(void* dst, const void* src, size_t bytes, void* stream);
int mdxrt_d2d_async(void* dst, const void* src, size_t bytes, void* stream);
int mdxrt_stream_create(void** stream);
int mdxrt_stream_destroy(void* stream);
int mdxrt_stream_sync(void* stream);
int mdxrt_device_sync(void);
int mdxrt_graph_begin(void* stream);
int mdxrt_graph_end(void* stream, void** exec);
int mdxrt_graph_launch(void* exec, void* stream);
int mdxrt_graph_destroy(void* exec);
int mdxrt_event_create(void** ev);
int mdxrt_event_destroy(void* ev);
int mdxrt_event_record(void* ev, void* stream);
int mdxrt_event_elapsed_ms(void* start, void* stop, float* ms);
/* Fill `n` 32-bit words with `value` on the stream (a kernel, never a
 * memset node, so it is safe inside captured graphs). */
int mdxrt_fill_u32(void* dst, uint32_t value, size_t n, void* stream);

/* ---- decode (M = 1) kernels ---- */

/* Fused RMSNorm + projection: x16 = fp16((hidden*rms)*norm_w), y = x16 . W^T
 * (x scale).  epilogue: 0 store y fp32, 1 SwiGLU over rows [0,N/2) and
 * [N/2,N) writing act fp16 [N/2]. */
int mdx_launch_norm_gemv(const float* hidden, const float* norm_w, float eps,
                         const mdx_wdesc* w, int epilogue, void* out, void* stream);

/* First projection of a step: the input row is embeddings[state->token]
 * (state->mode 0) or emb_in (mode 1); it is copied to hidden[d] and then
 * RMSNorm + projection as mdx_launch_norm_gemv, storing y fp32. */
int mdx_launch_embed_norm_gemv(const mdx_state* state, const float* emb_table, const float* emb_in,
                               int vocab, float* hidden, const float* norm_w, float eps,
                               const mdx_wdesc* w, float* out, void* stream);

/* y = fp16 x . W^T (x scale); out[n] += y[n] (residual add, fp32). */
int mdx_launch_gemv_add(const uint16_t* x16, const mdx_wdesc* w, float* out, void* stream);

/* y = x16 . W^T (x scale), fp16 input already rounded, fp32 output. */
int mdx_launch_gemv_f16in(const uint16_t* x16, const mdx_wdesc* w, float* y, void* stream);

/* Plain projection with fp32 output: y = x . W^T.  For MDX_W_F16/I8/I4 the
 * fp32 x is rounded to fp16 (the NPU input); for MDX_W_F32 and when
 * x_fp32_exact != 0 with MDX_W_F16 it is used as fp32 (the CPU GEMVs). */
int mdx_launch_gemv(const float* x, const mdx_wdesc* w, int x_fp32_exact, float* y,
                    void* stream);

/* One decode attention layer: QK-norm (q_norm/k_norm may be NULL) + RoPE at
 * row state->pos of the tables, append of the new K/V (fp16) at that row
 * of the layer cache [max_seq][nkv*hd], split-K GQA attention over rows
 * [0, state->pos] and the merge of the splits; writes the fp16 attention
 * output [nq*hd].  qkv is the fp32 [q|k|v] projection output.  scratch:
 * mdx_attn_decode_scratch_bytes() bytes whose last nkv words are zero
 * between launches (the kernel leaves them zero). */
int mdx_attn_max_splits(int max_seq);
size_t mdx_attn_decode_scratch_bytes(int nq, int nkv, int hd, int max_splits);
int mdx_launch_attn_decode(const mdx_state* state, const float* qkv, const float* q_norm,
                           const float* k_norm, float eps, const float* cos_t, const float* sin_t,
                           int rope_style, int nq, int nkv, int hd, int max_seq, int max_splits,
                           uint16_t* k_cache, uint16_t* v_cache, void* scratch, uint16_t* attn_out16,
                           void* stream);

/* Final RMSNorm + lm_head writing logits fp32 [N], with the argmax (lowest
 * index on ties) fused: the last block to finish stores it in
 * state->argmax and state->token, appends it to out_tokens[state->n_out++]
 * when out_tokens != NULL and advances state->pos by `advance`.
 * w->kind: MDX_W_I8 (fp16 activations, the NPU path), MDX_W_F16 with fp32
 * activations (the CPU fp16 GEMV), MDX_W_F32 (fp32 rows).  scratch:
 * mdx_lmhead_scratch_bytes() zero bytes (left zero by the kernel). */
size_t mdx_lmhead_scratch_bytes(void);
int mdx_launch_lmhead(const float* hidden, const float* norm_w, float eps, const mdx_wdesc* w,
                      float* logits, void* scratch, mdx_state* state, int* out_tokens, int advance,
                      void* stream);
/* state->pos += advance (prefill-mode steps). */
int mdx_launch_advance(mdx_state* state, int advance, void* stream);

/* ---- whole decode step in one cooperative launch (mdx_persist.hip) ---- */

/* Per-layer device pointers of the persistent step (all projections of one
 * kind, W^T rows as above; scales may be NULL; q_norm/k_norm may be NULL). */
typedef struct {
    const void* wqkv;  const float* sqkv;    /* [q | k | v] rows */
    const void* wo;    const float* so;
    const void* wgu;   const float* sgu;     /* [gate | up] rows */
    const void* wdown; const float* sdown;
    const float* in_norm;
    const float* post_norm;
    const float* q_norm;
    const float* k_norm;
    uint16_t* kc;      /* [max_seq][nkv*hd] fp16 */
    uint16_t* vc;
} mdx_persist_layer;

typedef struct {
    int kind;              /* MDX_W_F16 / MDX_W_I8 / MDX_W_I4 for every projection */
    int n_layers, vocab, max_seq, rope_style;
    int head;              /* 1: final norm + INT8 lm_head + argmax; 0: layers only */
    int advance;           /* state->pos += advance at the end of the step */
    int cooperative;       /* 1: hipLaunchCooperativeKernel (guaranteed co-residency);
                              0: ordinary launch of the same grid (less launch latency;
                              if the grid is not co-resident the waits time out and the
                              step reports the failure in state->pad[1]) */
    float eps;
    mdx_state* state;
    mdx_persist_layer l0;              /* layer 0; layer l's pointers are l0's plus
                                          l * layer_stride bytes, its KV caches
                                          l0.kc/vc plus l * kv_stride elements */
    long long layer_stride;
    long long kv_stride;
    const float* emb_table;            /* [vocab][d] fp32 */
    const float* emb_in;               /* [d], used when state->mode == 1 */
    const float* cos_t;
    const float* sin_t;
    const float* final_norm;
    const int8_t* lm_w;                /* [vocab][d] int8 */
    const float* lm_scale;             /* [vocab] */
    float* logits;                     /* [vocab] */
    float* hidden_out;                 /* [d] final hidden (before the final norm) */
    void* xbuf;                        /* mdx_persist_xbuf_bytes(), zeroed once at creation */
    int* out_tokens;                   /* optional greedy output list (state->n_out) */
    unsigned long long* trace;         /* optional [256][trace_stride] timestamps */
    int trace_stride;                  /* >= mdx_persist_trace_events(n_layers) */
    unsigned spin_limit;               /* polling rounds before a wait gives up; 0: default */
    int kv_stream;                     /* 1: read the K/V rows with non-temporal loads (a
                                          cache too large to stay in the last-level cache
                                          next to the lm_head) */
    int k_passes;                      /* 16-position K/V passes per round, 4 or 5: see
                                          mdx_persist_k_passes (int8 and int4 layers; fp16
                                          layers always take 4) */
    int in_args;                       /* 1: the step's position, token and mode come from
                                          the three fields below instead of the device
                                          state (which the step still updates) */
    int in_pos, in_token, in_mode;
    float* logits_host;                /* optional (head only, vocab <= 256 * 1024): the
                                          logits written to this mapped host buffer instead
                                          of logits */
    int* res_host;                     /* optional mapped host words: [0] <- the argmax,
                                          [1] <- 1 when a wait timed out */
    void* xbl;                         /* optional: cacheable words (mdx_persist_xbuf_bytes(),
                                          zeroed) for the exchanges among one KV head's
                                          workgroups, which share an XCD; NULL: those go
                                          through xbuf like the others */
} mdx_persist_args;

/* 1 when (d, nq, nkv, hd, F) is the shape the persistent step is built for. */
int mdx_persist_shape_ok(int d, int nq, int nkv, int hd, int F);
/* 1 when the current device can hold the whole grid co-resident. */
int mdx_persist_usable(int kind);
size_t mdx_persist_xbuf_bytes(void);
/* K/V passes per round for a step that attends over n_pos positions: 5 when
 * rounds of 64 positions per split would take three or more rounds and rounds
 * of 80 take fewer (the first two rounds are requested together; each later
 * one is a dependent load round trip), else 4. */
int mdx_persist_k_passes(int n_pos);
/* Events per workgroup of a traced step: 16 per layer (stage starts, waits
 * done, outputs written), 3 for the lm_head and the workgroup's XCD index. */
int mdx_persist_trace_events(int n_layers);
/* One decode step (all layers, and the lm_head when head != 0).  A wait that
 * times out sets state->pad[1] = 1; the caller treats that as a failure. */
int mdx_launch_persist_step(const mdx_persist_args* a, void* stream);
/* Test hook: leaves hidden-state exchange words tagged with the epoch the next
 * launch's first inter-layer wait accepts (stale data a late workgroup of a
 * timed-out launch could have written). */
int mdx_persist_debug_poison(void* xbuf, int n_layers, void* stream);

/* ---- batch prefill (M <= 64) kernels ---- */

/* x16[m][d] = fp16((x[m]*rms)*w) for m < M. */
int mdx_launch_rmsnorm_rows(const float* x, const float* w, float eps, int M, int d,
                            uint16_t* x16, void* stream);
/* x16[m][k] = fp16(x[m][k]). */
int mdx_launch_to_f16(const float* x, int n, uint16_t* x16, void* stream);

/* Y = X16[M][K] . W^T on MFMA, M <= 64.  epilogue: 0 store fp32 y[M][N],
 * 1 add into y[M][N], 2 SwiGLU (rows [0,N/2) gate, [N/2,N) up) -> fp16
 * act[M][N/2].  `scratch` is not used (kept for the signature). */
int mdx_launch_gemm(const uint16_t* x16, int M, const mdx_wdesc* w, int epilogue, void* out,
                    float* scratch, void* stream);
/* Residual projection with the next RMSNorm fused: hidden[M][N] += X16 . W^T
 * (x scale), then x16_out[M][N] = fp16((hidden * rms) * norm_w) per row
 * (norm_w NULL: no norm).  K is split over blocks; scratch holds the split
 * partials: mdx_gemm_scratch_floats(M, N, K) floats. */
size_t mdx_gemm_scratch_floats(int M, int N, int K);
int mdx_launch_gemm_residual_norm(const uint16_t* x16, int M, const mdx_wdesc* w, float* hidden,
                                  const float* norm_w, float eps, uint16_t* x16_out, float* scratch,
                                  void* stream);

/* QK-norm + RoPE for rows t < M at positions start+t, appending k,v fp16
 * at cache rows start+t; q written fp32 [M][nq*hd].  `start` is read from
 * state->pos. */
int mdx_launch_qk_rope_append_rows(const mdx_state* state, const float* qkv, int M,
                                   const float* q_norm, const float* k_norm, float eps,
                                   const float* cos_t, const float* sin_t, int nq, int nkv,
                                   int hd, int rope_style, float* q_out, uint16_t* k_cache,
                                   uint16_t* v_cache, void* stream);

/* The qkv projection and the launch above in one call: X16 . W^T as K-split
 * partials in scratch (mdx_gemm_scratch_floats(M, N, K) floats, about 256
 * blocks so every CU takes a share), which the QK-norm/RoPE/append kernel
 * sums in split order and scales per column as it reads the rows. */
int mdx_launch_qkv_rope_append_rows(const uint16_t* x16, int M, const mdx_wdesc* w, float* scratch,
                                    const mdx_state* state, const float* q_norm, const float* k_norm,
                                    float eps, const float* cos_t, const float* sin_t, int nq, int nkv,
                                    int hd, int rope_style, float* q_out, uint16_t* k_cache,
                                    uint16_t* v_cache, void* stream);

/* Causal attention for query rows t < M at positions state->pos + t over
 * cache rows [0, state->pos + t]; output fp16 [M][nq*hd]. */
int mdx_launch_attn_prefill(const mdx_state* state, const float* q, int M,
                            const uint16_t* k_cache, const uint16_t* v_cache, int nq, int nkv,
                            int hd, uint16_t* out16, void* stream);

/* Copy row M-1 of x[M][d] to dst[d] (last-token hidden after prefill). */
int mdx_launch_copy_row(const float* x, int row, int d, float* dst, void* stream);

/* ---- sampling (mdx_sample.hip) ---- */

#define MDX_SAMPLE_MAX_TOP_K 1024

/* logits[t] = logits[t] > 0 ? logits[t] / penalty : logits[t] * penalty for
 * each of the n tokens, which must be distinct and in range. */
int mdx_launch_repeat_penalty(float* logits, const int* tokens, int n, float penalty, void* stream);

/* Device scratch of mdx_launch_topk_sample (cleared by the launch itself). */
size_t mdx_sample_scratch_bytes(void);

/* Temperature, top-k (1 <= k <= min(V, MDX_SAMPLE_MAX_TOP_K); ties to the
 * lower index), top-p over the candidates when top_p < 1, and the draw at
 * uniform in [0,1].  out[0] = token, out[1] = candidates kept after top-p.
 * top_idx/top_val (k each, may be NULL) receive the candidates by descending
 * tempered value.  Calls sharing one scratch must not overlap. */
int mdx_launch_topk_sample(const float* logits, int V, float temperature, int k, float top_p,
                           float uniform, void* scratch, int* out, int* top_idx, float* top_val,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif
