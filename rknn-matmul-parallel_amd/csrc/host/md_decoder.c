/*
 * md_decoder.c — the decoder context behind matmul_decoder.h, on one GPU.
 *
 * Replaces the reference engine (src/matmul_decoder.c): instead of an NPU
 * context pool with a B-buffer rebind per projection, every weight, the fp16
 * KV cache, the RoPE tables and all scratch live in one device arena that is
 * sized and filled at create time.  A decode step is one pre-captured HIP
 * graph whose position and input token are read from device memory, so the
 * host only uploads the 4 KiB embedding (or nothing), launches, and reads
 * back the argmax (and the logits when the caller asks for them).
 */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include "md_internal.h"

enum { P_Q = 0, P_K, P_V, P_O, P_GATE, P_UP, P_DOWN, P_COUNT };
static const char* const kProjNames[P_COUNT] = {"q_proj", "k_proj", "v_proj", "o_proj",
                                                "gate_proj", "up_proj", "down_proj"};

typedef struct {
    mdx_wdesc qkv, o, gu, down;
    float *in_norm, *post_norm, *q_norm, *k_norm;
    uint16_t *kc, *vc;
} md_layer;

typedef struct {
    int M;
    void* exec;
} md_pgraph;

struct MatmulDecoderContext {
    MatmulDecoderConfig config;
    QuantizationType quant_type;
    int max_seq, seq_len;
    int d, nq, nkv, hd, qd, kvd, F, V, L;
    int n_lm, lm_vocab, max_m, max_splits;
    void* stream;
    uint8_t* arena;
    size_t arena_size, arena_used;
    mdx_state* d_state;
    float* d_emb;
    mdx_wdesc lm;
    mdx_wdesc* lm_heads;
    float* d_final_norm;
    md_layer* layers;
    uint16_t *d_kc, *d_vc;
    float *d_cos, *d_sin;
    float *d_hidden, *d_emb_in, *d_qkv, *d_logits, *d_tmp;
    void* d_sscr;                /* sampler scratch */
    void* d_part;            /* attention split partials + merge counters */
    uint16_t *d_attn16, *d_act16;
    void* d_partial;         /* lm_head argmax key + completion counter */
    int* d_tokens;
    int tokens_cap;
    float *d_bhidden, *d_bqkv, *d_bq, *d_gscr;
    uint16_t *d_bx16, *d_battn16, *d_bact16;
    void *g_layers, *g_head, *g_adv, *g_greedy;
    int graphs_ready;
    md_pgraph pgraphs[4];
    int pgraph_next;
    int capture_M;
    int use_graphs;          /* 0 when MDX_GRAPHS=0: same kernels, launched one by one */
    int persist;             /* 1: the layers of a decode step run as one launch */
    int persist_head;        /* 1: that launch also runs the INT8 lm_head and the argmax */
    int persist_coop;        /* 1: launch it cooperatively (after an ordinary launch timed out) */
    unsigned spin_once;      /* test hook: spin limit of the next one-launch step (0: default) */
    int poison_retry;        /* test hook: plant stale exchange words before the next retry */
    int kv_stream_force;     /* test hook: -1 decide per launch; 0 / 1 force the K/V load policy */
    int profile;             /* MDX_PROFILE=1: per-stage stats from device timestamps */
    unsigned long long* d_trace;   /* [256][trace_ev] timestamps of the profiled step */
    unsigned long long* h_trace;
    int trace_ev;
    void* d_xbuf;            /* exchange words of the persistent step */
    void* uc_xbuf;           /* the same in uncached memory from the runtime's pool (or NULL:
                                the arena's words are used) */
    void* lx_buf;            /* the arena's words, for the per-head exchanges in the L2 when the
                                uncached words serve the others (or NULL) */
    int lx_off;              /* set after a timed-out step: per-head exchanges through xbuf */
    int lx_force;            /* test hook: -1 default, 0 / 1 force them off / on */
    mdx_persist_args pargs;
    mdx_state* h_state;
    float* h_io;
    int* h_samp;                 /* pinned: sampler tokens, then {token, kept} */
    int* h_res;                  /* pinned: a host-fed step's {argmax, timeout flag} */
    size_t h_io_floats;
    void *ev0, *ev1, *ev2;
    MatmulDecoderStats stats;
};

/* ------------------------------------------------------------------------ */
/* Arena                                                                     */
/* ------------------------------------------------------------------------ */

static void* carve(MatmulDecoderContext* c, size_t bytes) {
    size_t off = (c->arena_used + MD_ALIGN - 1) & ~(size_t)(MD_ALIGN - 1);
    c->arena_used = off + bytes;
    if (!c->arena) return (void*)(uintptr_t)(off + MD_ALIGN); /* sizing pass: non-NULL marker */
    if (c->arena_used > c->arena_size) return NULL;
    return c->arena + off;
}

/* ------------------------------------------------------------------------ */
/* Weight sources                                                            */
/* ------------------------------------------------------------------------ */

typedef struct {
    md_host_proj p[P_COUNT];
    float *in_norm, *post_norm, *q_norm, *k_norm;
    int owned;           /* 1: buffers were read from files and are freed */
} md_host_layer;

typedef struct {
    const char* model_dir;               /* file source, or */
    const LayerWeights* mem_layers;      /* caller memory source */
} md_source;

static int qkind_of(QuantizationType q) {
    switch (q) {
        case QUANT_INT8: return 1;
        case QUANT_INT4:
        case QUANT_INT4_G128: return 2;
        default: return 0;
    }
}

static void proj_shapes(const MatmulDecoderContext* c, int* K, int* N) {
    K[P_Q] = c->d; N[P_Q] = c->qd;
    K[P_K] = c->d; N[P_K] = c->kvd;
    K[P_V] = c->d; N[P_V] = c->kvd;
    K[P_O] = c->qd; N[P_O] = c->d;
    K[P_GATE] = c->d; N[P_GATE] = c->F;
    K[P_UP] = c->d; N[P_UP] = c->F;
    K[P_DOWN] = c->F; N[P_DOWN] = c->d;
}

static void layer_dir(const char* model_dir, int l, char* out, size_t n) {
    struct stat st;
    snprintf(out, n, "%s/layers/layer_%02d", model_dir, l);
    if (stat(out, &st) == 0 && S_ISDIR(st.st_mode)) return;
    snprintf(out, n, "%s/layer_%02d", model_dir, l);
}

static long file_size(const char* path) {
    struct stat st;
    if (stat(path, &st) != 0) return -1;
    return (long)st.st_size;
}

/* Which kind each projection will have once loaded (reference fallbacks:
 * src/matmul_decoder.c:778-813): quantised file, else the fp16 file, else
 * zeros of the requested kind. */
static int planned_kind(const MatmulDecoderContext* c, const md_source* s, int l, int p) {
    int K[P_COUNT], N[P_COUNT];
    proj_shapes(c, K, N);
    const int qk = qkind_of(c->quant_type);
    if (s->mem_layers) {
        const ProjectionWeight* pw = &(&s->mem_layers[l].q_proj)[p];
        return pw->data ? qkind_of(pw->quant_type) : qk;
    }
    char dir[900], path[1024];
    layer_dir(s->model_dir, l, dir, sizeof dir);
    const size_t kn = (size_t)K[p] * N[p];
    if (qk) {
        snprintf(path, sizeof path, "%s/%s_weight.bin", dir, kProjNames[p]);
        if (file_size(path) >= (long)(qk == 2 ? kn / 2 : kn)) return qk;
        snprintf(path, sizeof path, "%s/%s.bin", dir, kProjNames[p]);
        if (file_size(path) >= (long)(kn * 2)) return 0;
        return qk;
    }
    return 0;
}

static void free_host_layer(md_host_layer* h) {
    if (!h->owned) return;
    for (int p = 0; p < P_COUNT; p++) {
        free(h->p[p].data);
        free(h->p[p].scale);
    }
    free(h->in_norm);
    free(h->post_norm);
    free(h->q_norm);
    free(h->k_norm);
}

static int read_host_layer(const MatmulDecoderContext* c, const md_source* s, int l,
                           md_host_layer* h) {
    int K[P_COUNT], N[P_COUNT];
    proj_shapes(c, K, N);
    memset(h, 0, sizeof *h);
    if (s->mem_layers) {
        const LayerWeights* lw = &s->mem_layers[l];
        const ProjectionWeight* pws = &lw->q_proj;
        for (int p = 0; p < P_COUNT; p++) {
            h->p[p].K = K[p];
            h->p[p].N = N[p];
            h->p[p].kind = pws[p].data ? qkind_of(pws[p].quant_type) : qkind_of(c->quant_type);
            h->p[p].data = pws[p].data;
            h->p[p].scale = pws[p].scales;
            if (pws[p].data && (pws[p].K != K[p] || pws[p].N != N[p])) {
                fprintf(stderr, "[MatmulDecoder] layer %d %s: shape %dx%d, expected %dx%d\n", l,
                        kProjNames[p], pws[p].K, pws[p].N, K[p], N[p]);
                return MATMUL_DECODER_ERR_INVALID_ARG;
            }
        }
        h->in_norm = lw->input_norm_weight;
        h->post_norm = lw->post_attn_norm_weight;
        h->q_norm = lw->q_norm_weight;
        h->k_norm = lw->k_norm_weight;
        h->owned = 0;
        if (!h->in_norm || !h->post_norm) return MATMUL_DECODER_ERR_INVALID_ARG;
        return MATMUL_DECODER_OK;
    }
    h->owned = 1;
    char dir[900], path[1024];
    layer_dir(s->model_dir, l, dir, sizeof dir);
    static const char* const in_names[] = {"input_norm.bin", "input_norm_weight.bin", NULL};
    static const char* const post_names[] = {"post_attn_norm.bin", "post_norm.bin",
                                             "post_attn_norm_weight.bin", NULL};
    static const char* const qn_names[] = {"q_norm.bin", "q_norm_weight.bin", NULL};
    static const char* const kn_names[] = {"k_norm.bin", "k_norm_weight.bin", NULL};
    h->in_norm = md_read_f32_first(dir, in_names, (size_t)c->d);
    h->post_norm = md_read_f32_first(dir, post_names, (size_t)c->d);
    if (!h->in_norm || !h->post_norm) {
        fprintf(stderr, "[MatmulDecoder] missing norm weights in %s\n", dir);
        return MATMUL_DECODER_ERR_FILE_IO;
    }
    if (c->config.has_qk_norm) {
        h->q_norm = md_read_f32_first(dir, qn_names, (size_t)c->hd);
        h->k_norm = md_read_f32_first(dir, kn_names, (size_t)c->hd);
        if (!h->q_norm || !h->k_norm) {
            fprintf(stderr, "[MatmulDecoder] missing QK norm weights in %s\n", dir);
            return MATMUL_DECODER_ERR_FILE_IO;
        }
    }
    const int qk = qkind_of(c->quant_type);
    for (int p = 0; p < P_COUNT; p++) {
        md_host_proj* hp = &h->p[p];
        hp->K = K[p];
        hp->N = N[p];
        const size_t kn = (size_t)K[p] * N[p];
        if (qk) {
            snprintf(path, sizeof path, "%s/%s_weight.bin", dir, kProjNames[p]);
            hp->data = md_read_file(path, qk == 2 ? kn / 2 : kn);
            if (hp->data) {
                hp->kind = qk;
                snprintf(path, sizeof path, "%s/%s_scales.bin", dir, kProjNames[p]);
                hp->scale = (float*)md_read_file(path, (size_t)N[p] * sizeof(float));
                if (!hp->scale)
                    fprintf(stderr, "[MatmulDecoder] warning: no scales for %s/%s, unscaled\n", dir,
                            kProjNames[p]);
                continue;
            }
        }
        snprintf(path, sizeof path, "%s/%s.bin", dir, kProjNames[p]);
        hp->data = md_read_file(path, kn * 2);
        hp->kind = 0;
        if (!hp->data) {
            fprintf(stderr, "[MatmulDecoder] warning: failed to load %s/%s, using zeros\n", dir,
                    kProjNames[p]);
            hp->kind = qk;
            hp->data = calloc(qk == 2 ? kn / 2 : (qk == 1 ? kn : kn * 2), 1);
            if (!hp->data) return MATMUL_DECODER_ERR_MEMORY;
        }
    }
    return MATMUL_DECODER_OK;
}

/* ------------------------------------------------------------------------ */
/* Layout                                                                    */
/* ------------------------------------------------------------------------ */

static int dev_kind_of(int host_kind) {
    return host_kind == 1 ? MDX_W_I8 : (host_kind == 2 ? MDX_W_I4 : MDX_W_F16);
}

/* Device kind and scale need of a merged group of projections. */
static void group_kind(const int* kinds, int n, int* dev_kind, int* has_scale) {
    int same = 1;
    for (int i = 1; i < n; i++) same &= kinds[i] == kinds[0];
    *dev_kind = same ? dev_kind_of(kinds[0]) : MDX_W_F16;
    *has_scale = 0;
    for (int i = 0; i < n; i++) *has_scale |= kinds[i] != 0;
}

static int carve_wdesc(MatmulDecoderContext* c, mdx_wdesc* w, int dev_kind, int has_scale, int K,
                       int N) {
    w->kind = dev_kind;
    w->K = K;
    w->N = N;
    w->w = carve(c, md_row_bytes(dev_kind, K) * (size_t)N);
    w->scale = has_scale ? (const float*)carve(c, (size_t)N * 4) : NULL;
    return w->w && (!has_scale || w->scale) ? 0 : -1;
}

static int layer_kinds(const MatmulDecoderContext* c, const md_source* s, int l, int* kinds) {
    for (int p = 0; p < P_COUNT; p++) kinds[p] = planned_kind(c, s, l, p);
    return 0;
}

static size_t lm_rows_bytes(const MatmulDecoderContext* c) {
    if (c->n_lm > 1) return 0;
    return c->config.disable_npu_lm_head ? (size_t)c->V * c->d * 2 : (size_t)c->V * c->d;
}

/* One pass over the arena layout; with c->arena == NULL it only sizes. */
static int layout(MatmulDecoderContext* c, const md_source* s) {
    c->arena_used = 0;
    int fail = 0;
#define CARVE(ptr, bytes) do { *(void**)&(ptr) = carve(c, (bytes)); fail |= (ptr) == NULL; } while (0)
    CARVE(c->d_state, sizeof(mdx_state));
    CARVE(c->d_emb, (size_t)c->V * c->d * 4);
    if (c->n_lm > 1) {
        for (int i = 0; i < c->n_lm; i++) {
            c->lm_heads[i].kind = MDX_W_F32;
            c->lm_heads[i].K = c->d;
            c->lm_heads[i].N = c->lm_vocab;
            c->lm_heads[i].scale = NULL;
            c->lm_heads[i].w = carve(c, (size_t)c->lm_vocab * c->d * 4);
            fail |= c->lm_heads[i].w == NULL;
        }
    } else {
        c->lm.K = c->d;
        c->lm.N = c->V;
        c->lm.kind = c->config.disable_npu_lm_head ? MDX_W_F16 : MDX_W_I8;
        c->lm.w = carve(c, lm_rows_bytes(c));
        c->lm.scale = c->config.disable_npu_lm_head ? NULL : (const float*)carve(c, (size_t)c->V * 4);
        fail |= c->lm.w == NULL;
    }
    CARVE(c->d_final_norm, (size_t)c->d * 4);
    for (int l = 0; l < c->L; l++) {
        md_layer* ly = &c->layers[l];
        int kinds[P_COUNT];
        layer_kinds(c, s, l, kinds);
        int dk, hs;
        group_kind(kinds, 3, &dk, &hs);
        fail |= carve_wdesc(c, &ly->qkv, dk, hs, c->d, c->qd + 2 * c->kvd);
        group_kind(&kinds[P_O], 1, &dk, &hs);
        fail |= carve_wdesc(c, &ly->o, dk, hs, c->qd, c->d);
        group_kind(&kinds[P_GATE], 2, &dk, &hs);
        fail |= carve_wdesc(c, &ly->gu, dk, hs, c->d, 2 * c->F);
        group_kind(&kinds[P_DOWN], 1, &dk, &hs);
        fail |= carve_wdesc(c, &ly->down, dk, hs, c->F, c->d);
        CARVE(ly->in_norm, (size_t)c->d * 4);
        CARVE(ly->post_norm, (size_t)c->d * 4);
        if (c->config.has_qk_norm) {
            CARVE(ly->q_norm, (size_t)c->hd * 4);
            CARVE(ly->k_norm, (size_t)c->hd * 4);
        } else {
            ly->q_norm = ly->k_norm = NULL;
        }
    }
    const size_t kv_bytes = (size_t)c->L * c->max_seq * c->kvd * 2;
    CARVE(c->d_kc, kv_bytes);
    CARVE(c->d_vc, kv_bytes);
    for (int l = 0; l < c->L; l++) {
        if (!c->arena) continue;
        c->layers[l].kc = c->d_kc + (size_t)l * c->max_seq * c->kvd;
        c->layers[l].vc = c->d_vc + (size_t)l * c->max_seq * c->kvd;
    }
    CARVE(c->d_cos, (size_t)c->max_seq * (c->hd / 2) * 4);
    CARVE(c->d_sin, (size_t)c->max_seq * (c->hd / 2) * 4);
    const int nlog = c->V > c->lm_vocab ? c->V : c->lm_vocab;
    const int widest = c->qd + 2 * c->kvd > 2 * c->F ? c->qd + 2 * c->kvd : 2 * c->F;
    CARVE(c->d_hidden, (size_t)c->d * 4);
    CARVE(c->d_emb_in, (size_t)c->d * 4);
    CARVE(c->d_qkv, (size_t)(c->qd + 2 * c->kvd) * 4);
    CARVE(c->d_part, mdx_attn_decode_scratch_bytes(c->nq, c->nkv, c->hd, c->max_splits));
    CARVE(c->d_logits, (size_t)nlog * 4);
    CARVE(c->d_sscr, mdx_sample_scratch_bytes());
    CARVE(c->d_tmp, (size_t)(widest > c->d ? widest : c->d) * 4);
    CARVE(c->d_attn16, (size_t)c->qd * 2);
    CARVE(c->d_act16, (size_t)c->F * 2);
    CARVE(c->d_partial, mdx_lmhead_scratch_bytes());
    CARVE(c->d_xbuf, mdx_persist_xbuf_bytes());
    const int mm = c->max_m;
    const int kmax = c->F > c->qd ? (c->F > c->d ? c->F : c->d) : (c->qd > c->d ? c->qd : c->d);
    CARVE(c->d_bhidden, (size_t)mm * c->d * 4);
    CARVE(c->d_bqkv, (size_t)mm * (c->qd + 2 * c->kvd) * 4);
    CARVE(c->d_bq, (size_t)mm * c->qd * 4);
    CARVE(c->d_bx16, (size_t)mm * kmax * 2);
    CARVE(c->d_battn16, (size_t)mm * c->qd * 2);
    CARVE(c->d_bact16, (size_t)mm * c->F * 2);
    {
        size_t g = mdx_gemm_scratch_floats(mm, c->qd + 2 * c->kvd, c->d);
        size_t t;
        t = mdx_gemm_scratch_floats(mm, c->d, c->qd); if (t > g) g = t;
        t = mdx_gemm_scratch_floats(mm, 2 * c->F, c->d); if (t > g) g = t;
        t = mdx_gemm_scratch_floats(mm, c->d, c->F); if (t > g) g = t;
        CARVE(c->d_gscr, g * 4);
    }
#undef CARVE
    return fail ? -1 : 0;
}

/* ------------------------------------------------------------------------ */
/* Upload                                                                    */
/* ------------------------------------------------------------------------ */

static int upload_group(const md_host_proj* const* ps, int n, const mdx_wdesc* w) {
    const size_t rb = md_row_bytes(w->kind, w->K);
    uint8_t* rows = (uint8_t*)malloc(rb * (size_t)w->N);
    float* sc = w->scale ? (float*)malloc((size_t)w->N * 4) : NULL;
    if (!rows || (w->scale && !sc)) {
        free(rows);
        free(sc);
        return MATMUL_DECODER_ERR_MEMORY;
    }
    int row0 = 0, rc = 0;
    for (int i = 0; i < n && rc == 0; i++) {
        rc = md_repack_rows(ps[i], w->kind, rows, sc, row0);
        row0 += ps[i]->N;
    }
    if (rc == 0) rc = mdxrt_h2d((void*)w->w, rows, rb * (size_t)w->N);
    if (rc == 0 && sc) rc = mdxrt_h2d((void*)w->scale, sc, (size_t)w->N * 4);
    free(rows);
    free(sc);
    return rc ? (rc == -1 ? MATMUL_DECODER_ERR_UNSUPPORTED : rc) : 0;
}

static int upload_layers(MatmulDecoderContext* c, const md_source* s, float** last_post_norm) {
    for (int l = 0; l < c->L; l++) {
        md_host_layer h;
        int rc = read_host_layer(c, s, l, &h);
        if (rc) {
            free_host_layer(&h);
            return rc;
        }
        md_layer* ly = &c->layers[l];
        const md_host_proj* qkv[3] = {&h.p[P_Q], &h.p[P_K], &h.p[P_V]};
        const md_host_proj* o[1] = {&h.p[P_O]};
        const md_host_proj* gu[2] = {&h.p[P_GATE], &h.p[P_UP]};
        const md_host_proj* dn[1] = {&h.p[P_DOWN]};
        rc = upload_group(qkv, 3, &ly->qkv);
        if (!rc) rc = upload_group(o, 1, &ly->o);
        if (!rc) rc = upload_group(gu, 2, &ly->gu);
        if (!rc) rc = upload_group(dn, 1, &ly->down);
        if (!rc) rc = mdxrt_h2d(ly->in_norm, h.in_norm, (size_t)c->d * 4);
        if (!rc) rc = mdxrt_h2d(ly->post_norm, h.post_norm, (size_t)c->d * 4);
        if (!rc && c->config.has_qk_norm) {
            if (h.q_norm && h.k_norm) {
                rc = mdxrt_h2d(ly->q_norm, h.q_norm, (size_t)c->hd * 4);
                if (!rc) rc = mdxrt_h2d(ly->k_norm, h.k_norm, (size_t)c->hd * 4);
            } else {
                ly->q_norm = ly->k_norm = NULL;   /* reference skips QK-norm without weights */
            }
        }
        if (!rc && l == c->L - 1 && last_post_norm) {
            *last_post_norm = (float*)malloc((size_t)c->d * 4);
            if (*last_post_norm) memcpy(*last_post_norm, h.post_norm, (size_t)c->d * 4);
        }
        free_host_layer(&h);
        if (rc) return rc;
    }
    return MATMUL_DECODER_OK;
}

/* RoPE tables with the reference formula and libm calls (reference:
 * src/matmul_decoder.c:620-631), so the values match the host exactly. */
static int upload_rope(MatmulDecoderContext* c) {
    const int half = c->hd / 2;
    const size_t n = (size_t)c->max_seq * half;
    float* ct = (float*)malloc(n * 4);
    float* st = (float*)malloc(n * 4);
    if (!ct || !st) {
        free(ct);
        free(st);
        return MATMUL_DECODER_ERR_MEMORY;
    }
    for (int pos = 0; pos < c->max_seq; pos++) {
        for (int i = 0; i < half; i++) {
            const float freq = 1.0f / powf(c->config.rope_theta, (2.0f * i) / c->hd);
            const float angle = pos * freq;
            ct[(size_t)pos * half + i] = cosf(angle);
            st[(size_t)pos * half + i] = sinf(angle);
        }
    }
    int rc = mdxrt_h2d(c->d_cos, ct, n * 4);
    if (!rc) rc = mdxrt_h2d(c->d_sin, st, n * 4);
    free(ct);
    free(st);
    return rc;
}

static int upload_lm_single(MatmulDecoderContext* c, const float* lm32) {
    const size_t n = (size_t)c->V * c->d;
    uint16_t* lm16 = (uint16_t*)malloc(n * 2);
    if (!lm16) return MATMUL_DECODER_ERR_MEMORY;
    for (size_t i = 0; i < n; i++) lm16[i] = mdx_f32_to_f16(lm32[i]);
    int rc;
    if (c->config.disable_npu_lm_head) {
        rc = mdxrt_h2d((void*)c->lm.w, lm16, n * 2);
    } else {
        int8_t* q = (int8_t*)malloc(n);
        float* sc = (float*)malloc((size_t)c->V * 4);
        if (!q || !sc) {
            free(q);
            free(sc);
            free(lm16);
            return MATMUL_DECODER_ERR_MEMORY;
        }
        mdx_quantize_lm_head(q, sc, lm16, c->V, c->d);
        rc = mdxrt_h2d((void*)c->lm.w, q, n);
        if (!rc) rc = mdxrt_h2d((void*)c->lm.scale, sc, (size_t)c->V * 4);
        free(q);
        free(sc);
    }
    free(lm16);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* Launch sequences                                                          */
/* ------------------------------------------------------------------------ */

static int run_layers(MatmulDecoderContext* c, void* s) {
    const float eps = c->config.rms_eps;
    int rc = 0;
    for (int l = 0; l < c->L && rc == 0; l++) {
        md_layer* ly = &c->layers[l];
        if (l == 0)
            rc = mdx_launch_embed_norm_gemv(c->d_state, c->d_emb, c->d_emb_in, c->V, c->d_hidden,
                                            ly->in_norm, eps, &ly->qkv, c->d_qkv, s);
        else
            rc = mdx_launch_norm_gemv(c->d_hidden, ly->in_norm, eps, &ly->qkv, 0, c->d_qkv, s);
        if (!rc)
            rc = mdx_launch_attn_decode(c->d_state, c->d_qkv, ly->q_norm, ly->k_norm, eps, c->d_cos,
                                        c->d_sin, c->config.rope_style, c->nq, c->nkv, c->hd,
                                        c->max_seq, c->max_splits, ly->kc, ly->vc, c->d_part,
                                        c->d_attn16, s);
        if (!rc) rc = mdx_launch_gemv_add(c->d_attn16, &ly->o, c->d_hidden, s);
        if (!rc) rc = mdx_launch_norm_gemv(c->d_hidden, ly->post_norm, eps, &ly->gu, 1, c->d_act16, s);
        if (!rc) rc = mdx_launch_gemv_add(c->d_act16, &ly->down, c->d_hidden, s);
    }
    return rc;
}

static int run_head(MatmulDecoderContext* c, const mdx_wdesc* lm, int* out_tokens, int advance,
                    void* s) {
    return mdx_launch_lmhead(c->d_hidden, c->d_final_norm, c->config.rms_eps, lm, c->d_logits,
                             c->d_partial, c->d_state, out_tokens, advance, s);
}

static int run_prefill(MatmulDecoderContext* c, int M, void* s) {
    const float eps = c->config.rms_eps;
    /* the first layer's input norm; every later norm is fused into the
     * residual projection before it */
    int rc = mdx_launch_rmsnorm_rows(c->d_bhidden, c->layers[0].in_norm, eps, M, c->d, c->d_bx16, s);
    for (int l = 0; l < c->L && rc == 0; l++) {
        md_layer* ly = &c->layers[l];
        const float* next_norm = l + 1 < c->L ? c->layers[l + 1].in_norm : NULL;
        /* qkv as K-split partials, summed by the RoPE/append kernel */
        rc = mdx_launch_qkv_rope_append_rows(c->d_bx16, M, &ly->qkv, c->d_gscr, c->d_state, ly->q_norm,
                                             ly->k_norm, eps, c->d_cos, c->d_sin, c->nq, c->nkv, c->hd,
                                             c->config.rope_style, c->d_bq, ly->kc, ly->vc, s);
        if (!rc)
            rc = mdx_launch_attn_prefill(c->d_state, c->d_bq, M, ly->kc, ly->vc, c->nq, c->nkv,
                                         c->hd, c->d_battn16, s);
        if (!rc)
            rc = mdx_launch_gemm_residual_norm(c->d_battn16, M, &ly->o, c->d_bhidden, ly->post_norm,
                                               eps, c->d_bx16, c->d_gscr, s);
        if (!rc) rc = mdx_launch_gemm(c->d_bx16, M, &ly->gu, 2, c->d_bact16, c->d_gscr, s);
        if (!rc)
            rc = mdx_launch_gemm_residual_norm(c->d_bact16, M, &ly->down, c->d_bhidden, next_norm,
                                               eps, c->d_bx16, c->d_gscr, s);
    }
    if (!rc) rc = mdx_launch_advance(c->d_state, M, s);
    return rc;
}

typedef int (*md_seq_fn)(MatmulDecoderContext*, void*);

static int capture(MatmulDecoderContext* c, md_seq_fn fn, void** exec) {
    int rc = mdxrt_graph_begin(c->stream);
    if (rc) return rc;
    int rc2 = fn(c, c->stream);
    rc = mdxrt_graph_end(c->stream, exec);
    return rc2 ? rc2 : rc;
}

static int seq_layers(MatmulDecoderContext* c, void* s) { return run_layers(c, s); }
static int seq_head(MatmulDecoderContext* c, void* s) { return run_head(c, &c->lm, NULL, 1, s); }
static int seq_adv(MatmulDecoderContext* c, void* s) { return mdx_launch_advance(c->d_state, 1, s); }
static int seq_greedy(MatmulDecoderContext* c, void* s) {
    int rc = run_layers(c, s);
    if (!rc) rc = run_head(c, &c->lm, c->d_tokens, 1, s);
    return rc;
}

/* Launches a captured sequence, or issues its kernels directly when graphs
 * are switched off. */
static int launch_seq(MatmulDecoderContext* c, void* exec, md_seq_fn fn) {
    return c->use_graphs ? mdxrt_graph_launch(exec, c->stream) : fn(c, c->stream);
}

static int ensure_graphs(MatmulDecoderContext* c) {
    if (c->graphs_ready) return 0;
    if (!c->use_graphs) {
        c->graphs_ready = 1;
        return 0;
    }
    int rc = capture(c, seq_layers, &c->g_layers);
    if (!rc && c->n_lm <= 1) rc = capture(c, seq_head, &c->g_head);
    if (!rc) rc = capture(c, seq_adv, &c->g_adv);
    if (rc) {
        fprintf(stderr, "[MatmulDecoder] graph capture failed: %s\n", mdxrt_last_error());
        return MATMUL_DECODER_ERR_RKNN;
    }
    c->graphs_ready = 1;
    return 0;
}

static int seq_prefill(MatmulDecoderContext* c, void* s) { return run_prefill(c, c->capture_M, s); }

static void* prefill_graph(MatmulDecoderContext* c, int M) {
    if (!c->use_graphs) return NULL;
    for (int i = 0; i < 4; i++)
        if (c->pgraphs[i].exec && c->pgraphs[i].M == M) return c->pgraphs[i].exec;
    md_pgraph* slot = &c->pgraphs[c->pgraph_next];
    c->pgraph_next = (c->pgraph_next + 1) % 4;
    if (slot->exec) mdxrt_graph_destroy(slot->exec);
    slot->exec = NULL;
    c->capture_M = M;
    if (capture(c, seq_prefill, &slot->exec) != 0) {
        slot->exec = NULL;
        return NULL;
    }
    slot->M = M;
    return slot->exec;
}

/* ------------------------------------------------------------------------ */
/* Persistent step                                                           */
/* ------------------------------------------------------------------------ */

static int at_stride(const void* p0, const void* pl, int l, long long stride) {
    if (!p0 || !pl) return p0 == pl;
    return (const char*)pl - (const char*)p0 == (long long)l * stride;
}

/* The layers of a step become one launch when the model has the shape that
 * kernel is built for, one weight kind throughout, and layers laid out at a
 * constant stride in the arena (always true for the arena layout, checked
 * anyway).  With the single INT8 lm_head the same launch also runs the head
 * and the argmax; multi-head models and the fp16 lm_head run their head as a
 * per-stage kernel after it.  MDX_PERSIST=0 keeps the per-kernel path. */
static void setup_persist(MatmulDecoderContext* c) {
    c->persist = 0;
    c->persist_head = 0;
    const char* e = getenv("MDX_PERSIST");
    if (e && e[0] == '0') return;
    if (c->L < 1) return;
    if (!mdx_persist_shape_ok(c->d, c->nq, c->nkv, c->hd, c->F)) return;
    const md_layer* l0 = &c->layers[0];
    const int kind = l0->qkv.kind;
    if (kind != MDX_W_F16 && kind != MDX_W_I8 && kind != MDX_W_I4) return;
    const long long stride = c->L > 1 ? (const char*)c->layers[1].qkv.w - (const char*)l0->qkv.w : 0;
    for (int l = 0; l < c->L; l++) {
        const md_layer* ly = &c->layers[l];
        if (ly->qkv.kind != kind || ly->o.kind != kind || ly->gu.kind != kind || ly->down.kind != kind)
            return;
        if (!at_stride(l0->qkv.w, ly->qkv.w, l, stride) || !at_stride(l0->qkv.scale, ly->qkv.scale, l, stride) ||
            !at_stride(l0->o.w, ly->o.w, l, stride) || !at_stride(l0->o.scale, ly->o.scale, l, stride) ||
            !at_stride(l0->gu.w, ly->gu.w, l, stride) || !at_stride(l0->gu.scale, ly->gu.scale, l, stride) ||
            !at_stride(l0->down.w, ly->down.w, l, stride) ||
            !at_stride(l0->down.scale, ly->down.scale, l, stride) ||
            !at_stride(l0->in_norm, ly->in_norm, l, stride) ||
            !at_stride(l0->post_norm, ly->post_norm, l, stride) ||
            !at_stride(l0->q_norm, ly->q_norm, l, stride) || !at_stride(l0->k_norm, ly->k_norm, l, stride) ||
            ly->kc != l0->kc + (size_t)l * c->max_seq * c->kvd ||
            ly->vc != l0->vc + (size_t)l * c->max_seq * c->kvd)
            return;
    }
    if (!mdx_persist_usable(kind)) return;
    mdx_persist_args* a = &c->pargs;
    memset(a, 0, sizeof *a);
    a->kind = kind;
    a->n_layers = c->L;
    a->vocab = c->V;
    a->max_seq = c->max_seq;
    a->rope_style = c->config.rope_style;
    a->eps = c->config.rms_eps;
    a->state = c->d_state;
    a->l0.wqkv = l0->qkv.w;
    a->l0.sqkv = l0->qkv.scale;
    a->l0.wo = l0->o.w;
    a->l0.so = l0->o.scale;
    a->l0.wgu = l0->gu.w;
    a->l0.sgu = l0->gu.scale;
    a->l0.wdown = l0->down.w;
    a->l0.sdown = l0->down.scale;
    a->l0.in_norm = l0->in_norm;
    a->l0.post_norm = l0->post_norm;
    a->l0.q_norm = l0->q_norm;
    a->l0.k_norm = l0->k_norm;
    a->l0.kc = l0->kc;
    a->l0.vc = l0->vc;
    a->layer_stride = stride;
    a->kv_stride = (long long)c->max_seq * c->kvd;
    a->emb_table = c->d_emb;
    a->emb_in = c->d_emb_in;
    a->cos_t = c->d_cos;
    a->sin_t = c->d_sin;
    a->final_norm = c->d_final_norm;
    if (c->n_lm <= 1 && !c->config.disable_npu_lm_head && c->V >= 256 && c->lm.kind == MDX_W_I8) {
        a->lm_w = (const int8_t*)c->lm.w;
        a->lm_scale = c->lm.scale;
        c->persist_head = 1;
    }
    a->logits = c->d_logits;
    a->hidden_out = c->d_hidden;
    /* The exchange words in uncached memory: the stores and polls then skip
     * the L2 (fp16 layers at KV 512: 465.3 -> 443.8 us/token).  The arena's
     * words stay the fallback if that allocation fails. */
    c->lx_buf = NULL;
    if (mdxrt_uc_acquire(&c->uc_xbuf, mdx_persist_xbuf_bytes()) == 0) {
        /* a pooled buffer holds the words of an earlier context: start from
         * zero words (epoch 0 is never valid) */
        if (mdxrt_fill_u32(c->uc_xbuf, 0u, mdx_persist_xbuf_bytes() / 4, c->stream) ||
            mdxrt_stream_sync(c->stream)) {
            mdxrt_uc_release(c->uc_xbuf);
            c->uc_xbuf = NULL;
        } else {
            /* the arena's (zeroed) words carry the per-head exchanges */
            c->lx_buf = c->d_xbuf;
            c->d_xbuf = c->uc_xbuf;
        }
    } else {
        c->uc_xbuf = NULL;
    }
    a->xbuf = c->d_xbuf;
    c->persist = 1;
}

/* pos: the position the launch processes (it attends over pos + 1) */
static int launch_persist(MatmulDecoderContext* c, int head, int* out_tokens, int pos) {
    if (head && !c->persist_head) return MATMUL_DECODER_ERR_INVALID_ARG;
    c->pargs.head = head;
    c->pargs.advance = 1;
    c->pargs.out_tokens = out_tokens;
    c->pargs.cooperative = c->persist_coop;
    c->pargs.spin_limit = c->spin_once;
    c->spin_once = 0;
    /* K/V rows of a long context are streamed past the last-level cache
     * (256 MB), which then keeps the 156 MB INT8 lm_head from step to step;
     * a short context's rows (read again every step) stay cached */
    const double kv_bytes = 2.0 * c->L * (double)(pos + 1) * c->kvd * 2.0;
    c->pargs.kv_stream = c->kv_stream_force >= 0 ? c->kv_stream_force : kv_bytes > 96.0 * 1024 * 1024;
    c->pargs.k_passes = mdx_persist_k_passes(pos + 1);
    /* the per-head exchanges in the XCD's L2 (fp16 KV 512: 453.0 -> 448.1
     * us/token for the qkv exchange alone), unless a step has timed out */
    c->pargs.xbl = c->lx_buf && (c->lx_force >= 0 ? c->lx_force : !c->lx_off) ? c->lx_buf : NULL;
    return mdx_launch_persist_step(&c->pargs, c->stream);
}

/* One-launch steps of different contexts in this process never run at the
 * same time: an ordinary launch relies on its grid being co-resident, which
 * two concurrent grids of 256 CU-filling workgroups would not be.  (A grid of
 * another process can still crowd one out; the step then times out and is
 * retried as a cooperative launch, see persist_retry.) */
static pthread_mutex_t g_persist_mu = PTHREAD_MUTEX_INITIALIZER;

/* After a timed-out ordinary launch: switch the context to cooperative
 * launches.  Returns 1 when the caller should run the step again (the state
 * is uploaded again; the K/V rows the failed step wrote are rewritten). */
static int persist_retry(MatmulDecoderContext* c) {
    if (!c->persist || c->persist_coop) return 0;
    c->persist_coop = 1;
    if (c->poison_retry) {
        c->poison_retry = 0;
        if (mdx_persist_debug_poison(c->d_xbuf, c->L, c->stream)) return 0;
    }
    /* A workgroup of the timed-out launch that started late (crowded out by
     * another grid) read the step counter after workgroup 0 had advanced it,
     * and published words tagged with the epochs the retry would use.  Zeroing
     * the exchange words, the counter with them, leaves no word the retry can
     * accept before its own writer stores it (epoch 0 is never valid).  The
     * stream is synchronised, so no workgroup of that launch is still running. */
    if (mdxrt_fill_u32(c->d_xbuf, 0u, mdx_persist_xbuf_bytes() / 4, c->stream) ||
        (c->lx_buf && mdxrt_fill_u32(c->lx_buf, 0u, mdx_persist_xbuf_bytes() / 4, c->stream)) ||
        mdxrt_stream_sync(c->stream))
        return 0;
    /* The per-head exchanges stay in an XCD's L2 only while each KV head's
     * workgroups share an XCD; after a timeout they go through memory like
     * the others. */
    c->lx_off = 1;
    fprintf(stderr, "[MatmulDecoder] one-launch step timed out; retrying with cooperative launches\n");
    return 1;
}

/* ------------------------------------------------------------------------ */
/* Create / destroy                                                          */
/* ------------------------------------------------------------------------ */

static int check_config(const MatmulDecoderConfig* cfg, int max_seq_len) {
    if (cfg->hidden_dim <= 0 || cfg->num_q_heads <= 0 || cfg->num_kv_heads <= 0 ||
        cfg->head_dim <= 0 || cfg->ffn_dim <= 0 || cfg->num_layers <= 0 || cfg->vocab_size <= 0 ||
        max_seq_len <= 0) {
        fprintf(stderr, "[MatmulDecoder] invalid model dimensions\n");
        return MATMUL_DECODER_ERR_INVALID_ARG;
    }
    const int G = cfg->num_q_heads % cfg->num_kv_heads ? 0 : cfg->num_q_heads / cfg->num_kv_heads;
    const int hd = cfg->head_dim;
    if (!(hd == 64 || hd == 128 || hd == 256) || !(G == 1 || G == 2 || G == 4 || G == 8) ||
        (hd == 256 && G == 8)) {
        fprintf(stderr, "[MatmulDecoder] unsupported head layout: head_dim=%d group=%d\n", hd, G);
        return MATMUL_DECODER_ERR_UNSUPPORTED;
    }
    if (cfg->hidden_dim % 32 || (cfg->num_q_heads * hd) % 32 || cfg->ffn_dim % 32) {
        fprintf(stderr, "[MatmulDecoder] hidden, q and ffn dims must be multiples of 32\n");
        return MATMUL_DECODER_ERR_UNSUPPORTED;
    }
    if (cfg->hidden_dim * 4 > 64 * 1024 || cfg->ffn_dim * 2 > 64 * 1024 ||
        cfg->num_q_heads * hd * 2 > 64 * 1024) {
        fprintf(stderr, "[MatmulDecoder] dimensions exceed the LDS activation buffer\n");
        return MATMUL_DECODER_ERR_UNSUPPORTED;
    }
    return 0;
}

static MatmulDecoderContext* create_common(const MatmulDecoderConfig* config,
                                           QuantizationType quant, int max_seq_len,
                                           const md_source* src, const float* embeddings,
                                           const float* lm_head) {
    if (check_config(config, max_seq_len) != 0) return NULL;
    if (mdxrt_device_count() <= 0) {
        fprintf(stderr, "[MatmulDecoder] no GPU visible to the HIP runtime\n");
        return NULL;
    }
    MatmulDecoderContext* c = (MatmulDecoderContext*)calloc(1, sizeof *c);
    if (!c) return NULL;
    c->config = *config;
    c->quant_type = quant;
    c->max_seq = max_seq_len;
    c->d = config->hidden_dim;
    c->nq = config->num_q_heads;
    c->nkv = config->num_kv_heads;
    c->hd = config->head_dim;
    c->qd = c->nq * c->hd;
    c->kvd = c->nkv * c->hd;
    c->F = config->ffn_dim;
    c->V = config->vocab_size;
    c->L = config->num_layers;
    c->n_lm = config->num_lm_heads > 1 ? config->num_lm_heads : 0;
    c->lm_vocab = c->n_lm ? (config->lm_head_vocab_size > 0 ? config->lm_head_vocab_size : c->V)
                          : c->V;
    int mm = config->max_batch_prefill > 0 ? config->max_batch_prefill : 64;
    c->max_m = mm > 64 ? 64 : mm;
    c->max_splits = mdx_attn_max_splits(max_seq_len);
    {
        const char* e = getenv("MDX_GRAPHS");
        c->use_graphs = !(e && e[0] == '0');
    }
    c->layers = (md_layer*)calloc((size_t)c->L, sizeof(md_layer));
    if (c->n_lm) c->lm_heads = (mdx_wdesc*)calloc((size_t)c->n_lm, sizeof(mdx_wdesc));
    if (!c->layers || (c->n_lm && !c->lm_heads)) goto fail;

    if (mdxrt_stream_create(&c->stream) || mdxrt_event_create(&c->ev0) ||
        mdxrt_event_create(&c->ev1) || mdxrt_event_create(&c->ev2))
        goto fail;

    /* size, allocate, then lay out for real */
    if (layout(c, src) != 0) goto fail;
    c->arena_size = c->arena_used;
    if (mdxrt_malloc((void**)&c->arena, c->arena_size) != 0) {
        fprintf(stderr, "[MatmulDecoder] arena of %zu bytes: %s\n", c->arena_size, mdxrt_last_error());
        c->arena = NULL;
        goto fail;
    }
    if (layout(c, src) != 0) goto fail;
    if (md_verbose())
        printf("[MatmulDecoder] arena %.1f MiB, %d layers, max_seq %d\n",
               c->arena_size / 1048576.0, c->L, c->max_seq);

    /* zero everything once (KV cache, scratch, state) */
    if (mdxrt_fill_u32(c->arena, 0u, c->arena_size / 4, c->stream) || mdxrt_stream_sync(c->stream))
        goto fail;

    if (mdxrt_h2d(c->d_emb, embeddings, (size_t)c->V * c->d * 4)) goto fail;
    if (c->n_lm) {
        for (int i = 0; i < c->n_lm; i++) {
            char path[1024];
            snprintf(path, sizeof path, "%s/lm_head_%02d.bin", src->model_dir ? src->model_dir : ".", i);
            float* h = src->model_dir ? (float*)md_read_file(path, (size_t)c->lm_vocab * c->d * 4) : NULL;
            if (!h) {
                fprintf(stderr, "[MatmulDecoder] failed to load %s\n", path);
                goto fail;
            }
            int rc = mdxrt_h2d((void*)c->lm_heads[i].w, h, (size_t)c->lm_vocab * c->d * 4);
            free(h);
            if (rc) goto fail;
        }
    } else {
        if (upload_lm_single(c, lm_head ? lm_head : embeddings)) goto fail;
    }
    {
        float* last_post = NULL;
        int rc = upload_layers(c, src, &last_post);
        if (rc) {
            free(last_post);
            goto fail;
        }
        float* fn = NULL;
        if (src->model_dir) {
            static const char* const names[] = {"final_norm.bin", "model_norm.bin", NULL};
            fn = md_read_f32_first(src->model_dir, names, (size_t)c->d);
        }
        if (!fn) {
            if (src->model_dir)
                fprintf(stderr, "[MatmulDecoder] warning: final_norm.bin not found, using the last "
                                "layer's post-attention norm\n");
            fn = last_post;
            last_post = NULL;
        }
        rc = fn ? mdxrt_h2d(c->d_final_norm, fn, (size_t)c->d * 4) : MATMUL_DECODER_ERR_FILE_IO;
        free(fn);
        free(last_post);
        if (rc) goto fail;
    }
    if (upload_rope(c)) goto fail;
    if (mdxrt_host_alloc((void**)&c->h_state, sizeof(mdx_state))) goto fail;
    c->h_io_floats = (size_t)(c->V > c->lm_vocab ? c->V : c->lm_vocab);
    if ((size_t)c->max_m * c->d > c->h_io_floats) c->h_io_floats = (size_t)c->max_m * c->d;
    if (mdxrt_host_alloc((void**)&c->h_io, c->h_io_floats * 4)) goto fail;
    if (mdxrt_host_alloc((void**)&c->h_samp, (MDX_SAMPLE_MAX_REPEAT + 64) * sizeof(int))) goto fail;
    if (mdxrt_host_alloc((void**)&c->h_res, 4 * sizeof(int))) goto fail;
    memset(c->h_state, 0, sizeof(mdx_state));
    setup_persist(c);
    {
        const char* e = getenv("MDX_PROFILE");
        c->profile = e && e[0] == '1';
        c->kv_stream_force = -1;
        c->lx_force = -1;
    }
    if (c->profile && c->persist) {
        c->trace_ev = mdx_persist_trace_events(c->L);
        const size_t n = (size_t)256 * c->trace_ev;
        c->h_trace = (unsigned long long*)malloc(n * 8);
        if (!c->h_trace || mdxrt_malloc((void**)&c->d_trace, n * 8)) goto fail;
    }
    if (md_verbose())
        printf("[MatmulDecoder] decode step: %s\n",
               c->persist ? (c->persist_head ? "one launch" : "layers in one launch, per-stage lm_head")
                          : "per-stage kernels");
    return c;
fail:
    fprintf(stderr, "[MatmulDecoder] create failed%s%s\n", mdxrt_last_error()[0] ? ": " : "",
            mdxrt_last_error());
    matmul_decoder_destroy(c);
    return NULL;
}

MatmulDecoderContext* matmul_decoder_create(const char* model_dir, const MatmulDecoderConfig* config,
                                            QuantizationType quant_type, int max_seq_len) {
    if (!model_dir) return NULL;
    MatmulDecoderConfig loaded;
    char path[1024];
    if (!config) {
        snprintf(path, sizeof path, "%s/config.json", model_dir);
        if (matmul_decoder_load_config(path, &loaded) != 0) {
            fprintf(stderr, "[MatmulDecoder] failed to load config from %s\n", path);
            return NULL;
        }
        config = &loaded;
    }
    if (check_config(config, max_seq_len) != 0) return NULL;
    snprintf(path, sizeof path, "%s/embeddings.bin", model_dir);
    float* emb = (float*)md_read_file(path, (size_t)config->vocab_size * config->hidden_dim * 4);
    if (!emb) {
        fprintf(stderr, "[MatmulDecoder] failed to load embeddings from %s\n", path);
        return NULL;
    }
    float* lm = NULL;
    if (config->num_lm_heads <= 1) {
        snprintf(path, sizeof path, "%s/lm_head.bin", model_dir);
        lm = (float*)md_read_file(path, (size_t)config->vocab_size * config->hidden_dim * 4);
        if (!lm && !config->tie_word_embeddings) {
            fprintf(stderr, "[MatmulDecoder] failed to load lm_head from %s\n", path);
            free(emb);
            return NULL;
        }
    }
    md_source src = {model_dir, NULL};
    MatmulDecoderContext* c = create_common(config, quant_type, max_seq_len, &src, emb, lm);
    free(emb);
    free(lm);
    return c;
}

MatmulDecoderContext* matmul_decoder_create_from_weights(const MatmulDecoderConfig* config,
                                                         const float* embeddings,
                                                         const LayerWeights* layers,
                                                         const float* lm_head,
                                                         QuantizationType quant_type,
                                                         int max_seq_len) {
    if (!config || !embeddings || !layers) return NULL;
    if (config->num_lm_heads > 1) {
        fprintf(stderr, "[MatmulDecoder] create_from_weights takes a single lm_head\n");
        return NULL;
    }
    if (!lm_head && !config->tie_word_embeddings) {
        fprintf(stderr, "[MatmulDecoder] lm_head is required when embeddings are not tied\n");
        return NULL;
    }
    md_source src = {NULL, layers};
    return create_common(config, quant_type, max_seq_len, &src, embeddings, lm_head);
}

void matmul_decoder_destroy(MatmulDecoderContext* c) {
    if (!c) return;
    if (c->stream) mdxrt_stream_sync(c->stream);
    mdxrt_graph_destroy(c->g_layers);
    mdxrt_graph_destroy(c->g_head);
    mdxrt_graph_destroy(c->g_adv);
    mdxrt_graph_destroy(c->g_greedy);
    for (int i = 0; i < 4; i++) mdxrt_graph_destroy(c->pgraphs[i].exec);
    mdxrt_free(c->d_tokens);
    mdxrt_free(c->d_trace);
    free(c->h_trace);
    mdxrt_free(c->arena);
    mdxrt_uc_release(c->uc_xbuf);
    mdxrt_host_free(c->h_state);
    mdxrt_host_free(c->h_io);
    mdxrt_host_free(c->h_samp);
    mdxrt_host_free(c->h_res);
    mdxrt_event_destroy(c->ev0);
    mdxrt_event_destroy(c->ev1);
    mdxrt_event_destroy(c->ev2);
    mdxrt_stream_destroy(c->stream);
    free(c->layers);
    free(c->lm_heads);
    free(c);
}

/* ------------------------------------------------------------------------ */
/* Steps                                                                     */
/* ------------------------------------------------------------------------ */

static int set_state(MatmulDecoderContext* c, int token_id, const float* embedding) {
    memset(c->h_state, 0, sizeof(mdx_state));
    c->h_state->pos = c->seq_len;
    c->h_state->token = embedding ? 0 : token_id;
    c->h_state->mode = embedding ? 1 : 0;
    int rc = 0;
    if (embedding) {
        memcpy(c->h_io, embedding, (size_t)c->d * 4);
        rc = mdxrt_h2d_async(c->d_emb_in, c->h_io, (size_t)c->d * 4, c->stream);
    }
    if (!rc) rc = mdxrt_h2d_async(c->d_state, c->h_state, sizeof(mdx_state), c->stream);
    return rc;
}

/* Shared by step and step_head: validation order of the reference
 * (src/matmul_decoder.c:1447-1462). */
static int step_checks(MatmulDecoderContext* c, int token_id, const float* embedding) {
    if (!embedding && (token_id < 0 || token_id >= c->V)) return MATMUL_DECODER_ERR_INVALID_ARG;
    if (c->seq_len >= c->max_seq) {
        fprintf(stderr, "[MatmulDecoder] KV cache full: seq_len=%d >= max=%d\n", c->seq_len,
                c->max_seq);
        return MATMUL_DECODER_ERR_INVALID_ARG;
    }
    return 0;
}

/* One decode step.  want_head selects the lm_head (the reference's
 * output_logits != NULL); logits_out may be NULL with want_head set when
 * only the token is needed. */
/* A device-side draw appended to a step (matmul_decoder_step_sample): the n
 * distinct penalised tokens are in c->h_samp[0..n). */
typedef struct {
    const SamplingParams* p;
    int k, n;
    float u;
} md_sample_req;

/* ---- MDX_PROFILE=1: the stats breakdown of a one-launch step ----------- */

static int cmp_u64(const void* a, const void* b) {
    const unsigned long long x = *(const unsigned long long*)a, y = *(const unsigned long long*)b;
    return x < y ? -1 : (x > y);
}

/* Median over the 256 workgroups of the time between events e0 and e1 of the
 * traced step (100 MHz ticks). */
static double seg_median(const MatmulDecoderContext* c, int e0, int e1, unsigned long long* tmp) {
    int n = 0;
    for (int b = 0; b < 256; b++) {
        const unsigned long long* r = c->h_trace + (size_t)b * c->trace_ev;
        if (r[e0] && r[e1]) tmp[n++] = r[e1] > r[e0] ? r[e1] - r[e0] : 0;
    }
    if (!n) return 0.0;
    qsort(tmp, (size_t)n, sizeof *tmp, cmp_u64);
    return (double)tmp[n / 2];
}

/* Splits the device time of a traced one-launch step over the reference's
 * categories (src/matmul_decoder.c:1616-1623): matmul_ms the projection
 * stages (with the norm / residual / SwiGLU they carry), cpu_ops_ms what
 * cpu_ops.c does there (QK-norm, RoPE, the KV append, attention and the merge
 * of its splits), lm_head_ms the lm_head with its argmax, rebind_ms the waits
 * for other workgroups' results (the one-launch step's data movement between
 * stages, where the reference rebinds B buffers).  Each category is the sum
 * over layers of the per-segment medians over workgroups, scaled so that the
 * four add up to the measured device time. */
static void profile_split(MatmulDecoderContext* c, float dev_ms, int head, MatmulDecoderStats* st) {
    static const int mm_seg[][2] = {{1, 2}, {6, 7}, {8, 9}, {9, 15}, {10, 11}};
    static const int ops_seg[][2] = {{3, 12}, {12, 13}, {13, 4}};
    static const int wait_seg[][2] = {{0, 1}, {2, 3}, {4, 5}, {5, 6}, {7, 8}, {15, 10}};
    unsigned long long tmp[256];
    double mm = 0, ops = 0, wait = 0, lm = 0;
    for (int l = 0; l < c->L; l++) {
        const int b = 16 * l;
        for (size_t i = 0; i < sizeof mm_seg / sizeof mm_seg[0]; i++)
            mm += seg_median(c, b + mm_seg[i][0], b + mm_seg[i][1], tmp);
        for (size_t i = 0; i < sizeof ops_seg / sizeof ops_seg[0]; i++)
            ops += seg_median(c, b + ops_seg[i][0], b + ops_seg[i][1], tmp);
        for (size_t i = 0; i < sizeof wait_seg / sizeof wait_seg[0]; i++)
            wait += seg_median(c, b + wait_seg[i][0], b + wait_seg[i][1], tmp);
    }
    if (head) {
        const int e = 16 * c->L;
        wait += seg_median(c, e - 16 + 11, e + 0, tmp);
        lm += seg_median(c, e + 0, e + 1, tmp);
        /* workgroup 0's reduction of the 256 keys */
        const unsigned long long* r0 = c->h_trace;
        if (r0[e + 2] > r0[e + 1]) lm += (double)(r0[e + 2] - r0[e + 1]);
    }
    const double sum = mm + ops + wait + lm;
    const double k = sum > 0 ? (double)dev_ms / sum : 0.0;
    st->matmul_ms = (float)(mm * k);
    st->cpu_ops_ms = (float)(ops * k);
    st->rebind_ms = (float)(wait * k);
    st->lm_head_ms = (float)(lm * k);
}

static int trace_arm(MatmulDecoderContext* c) {
    c->pargs.trace = c->d_trace;
    c->pargs.trace_stride = c->trace_ev;
    return mdxrt_fill_u32(c->d_trace, 0u, (size_t)256 * c->trace_ev * 2, c->stream);
}

static int do_step(MatmulDecoderContext* c, int token_id, const float* embedding,
                   float* output_logits, int want_head, const md_sample_req* sr) {
    if (!c) return MATMUL_DECODER_ERR_INVALID_ARG;
    const double t0 = md_now_ms();
    int rc = step_checks(c, token_id, embedding);
    if (rc) return rc;
    if (ensure_graphs(c)) return MATMUL_DECODER_ERR_RKNN;
    if (c->n_lm > 1 && want_head) {
        /* multi-head model: the reference step() has no single lm_head
         * either; use head 0 like step_head(…, 0, …) */
        return matmul_decoder_step_head(c, token_id, embedding, 0, output_logits);
    }
    const int prof = c->profile && c->persist && c->d_trace;
    const int one_launch_head = c->persist && c->persist_head && want_head;
    /* A step with the head in the one launch is host-fed: the position, token
     * and mode go in as kernel arguments, and the kernel writes the argmax,
     * the timeout flag and (for a plain step) the logits to mapped host
     * memory, so no copy runs before or after it.  A sampling step keeps its
     * logits on the device for the sampler (and copies them out when asked);
     * a profiling step keeps every copy. */
    const int host_fed = one_launch_head && !prof && (long long)c->V <= 256LL * 1024;
    const int host_logits = host_fed && !sr && output_logits;
    if (c->persist) pthread_mutex_lock(&g_persist_mu);
    if (host_fed) {
        c->h_res[0] = -1;
        c->h_res[1] = 0;
        c->pargs.in_args = 1;
        c->pargs.in_pos = c->seq_len;
        c->pargs.in_token = embedding ? 0 : token_id;
        c->pargs.in_mode = embedding ? 1 : 0;
        c->pargs.res_host = c->h_res;
        c->pargs.logits_host = host_logits ? c->h_io : NULL;
        rc = 0;
        if (embedding) {
            memcpy(c->h_io, embedding, (size_t)c->d * 4);
            rc = mdxrt_h2d_async(c->d_emb_in, c->h_io, (size_t)c->d * 4, c->stream);
        }
    } else {
        rc = set_state(c, token_id, embedding);
    }
    if (!rc && prof) rc = trace_arm(c);
    if (!rc) rc = mdxrt_event_record(c->ev0, c->stream);
    if (c->persist && (c->persist_head || !want_head)) {
        if (!rc) rc = launch_persist(c, want_head, NULL, c->seq_len);
        if (!rc) rc = mdxrt_event_record(c->ev1, c->stream);
    } else if (c->persist) {
        /* the fp16 lm_head: layers in one launch (which advances the
         * position), then the per-stage head */
        if (!rc) rc = launch_persist(c, 0, NULL, c->seq_len);
        if (!rc) rc = mdxrt_event_record(c->ev1, c->stream);
        if (!rc) rc = run_head(c, &c->lm, NULL, 0, c->stream);
    } else {
        if (!rc) rc = launch_seq(c, c->g_layers, seq_layers);
        if (!rc) rc = mdxrt_event_record(c->ev1, c->stream);
        if (!rc) rc = launch_seq(c, want_head ? c->g_head : c->g_adv, want_head ? seq_head : seq_adv);
    }
    if (!rc) rc = mdxrt_event_record(c->ev2, c->stream);
    if (!rc && output_logits && !host_logits)
        rc = mdxrt_d2h_async(c->h_io, c->d_logits, (size_t)c->V * 4, c->stream);
    if (!rc && sr) {
        /* penalty and draw on the logits just copied out; the kernels read
         * the tokens from and write {token, kept} to pinned host memory */
        if (sr->n)
            rc = mdx_launch_repeat_penalty(c->d_logits, c->h_samp, sr->n, sr->p->repeat_penalty, c->stream);
        if (!rc)
            rc = mdx_launch_topk_sample(c->d_logits, c->V, sr->p->temperature, sr->k, sr->p->top_p, sr->u,
                                        c->d_sscr, c->h_samp + MDX_SAMPLE_MAX_REPEAT, NULL, NULL,
                                        c->stream);
    }
    if (!rc && !host_fed) rc = mdxrt_d2h_async(c->h_state, c->d_state, sizeof(mdx_state), c->stream);
    if (!rc && prof)
        rc = mdxrt_d2h_async(c->h_trace, c->d_trace, (size_t)256 * c->trace_ev * 8, c->stream);
    if (!rc) rc = mdxrt_stream_sync(c->stream);
    c->pargs.trace = NULL;
    c->pargs.trace_stride = 0;
    c->pargs.in_args = 0;
    c->pargs.res_host = NULL;
    c->pargs.logits_host = NULL;
    if (host_fed && !rc) {
        c->h_state->pad[1] = c->h_res[1];
        c->h_state->argmax = c->h_res[0];
    }
    if (c->persist) pthread_mutex_unlock(&g_persist_mu);
    if (rc) {
        fprintf(stderr, "[MatmulDecoder] step failed: %s\n", mdxrt_last_error());
        return MATMUL_DECODER_ERR_RKNN;
    }
    if (c->h_state->pad[1]) {
        if (persist_retry(c)) return do_step(c, token_id, embedding, output_logits, want_head, sr);
        fprintf(stderr, "[MatmulDecoder] step failed: a workgroup timed out waiting for another\n");
        return MATMUL_DECODER_ERR_RKNN;
    }
    float layers_ms = 0.0f, head_ms = 0.0f;
    mdxrt_event_elapsed_ms(c->ev0, c->ev1, &layers_ms);
    mdxrt_event_elapsed_ms(c->ev1, c->ev2, &head_ms);
    c->seq_len++;
    int tok = 0;
    if (output_logits) memcpy(output_logits, c->h_io, (size_t)c->V * 4);
    if (want_head) tok = c->h_state->argmax;
    if (sr) tok = c->h_samp[MDX_SAMPLE_MAX_REPEAT];
    const float total = (float)(md_now_ms() - t0);
    /* Device times from events on the step's stream: layers_ms is the layers
     * launch (with the lm_head too when it runs inside it), head_ms the
     * separate head kernels.  Without MDX_PROFILE the one launch is not split:
     * it all counts as matmul_ms. */
    c->stats.total_ms = total;
    c->stats.matmul_ms = layers_ms;
    c->stats.rebind_ms = 0.0f;
    c->stats.cpu_ops_ms = 0.0f;
    c->stats.lm_head_ms = want_head && !one_launch_head ? head_ms : 0.0f;
    if (prof) {
        profile_split(c, layers_ms, one_launch_head, &c->stats);
        if (want_head && !one_launch_head) c->stats.lm_head_ms = head_ms;
    }
    c->stats.convert_ms = total - c->stats.matmul_ms - c->stats.cpu_ops_ms - c->stats.rebind_ms -
                          c->stats.lm_head_ms;
    if (c->stats.convert_ms < 0) c->stats.convert_ms = 0;
    c->stats.n_steps++;
    return tok;
}

int matmul_decoder_step(MatmulDecoderContext* c, int token_id, const float* embedding,
                        float* output_logits) {
    return do_step(c, token_id, embedding, output_logits, output_logits != NULL, NULL);
}

int mdx_step_token(MatmulDecoderContext* c, int token_id, const float* embedding) {
    return do_step(c, token_id, embedding, NULL, 1, NULL);
}

int matmul_decoder_step_get_logits(MatmulDecoderContext* c, int token_id, const float* embedding,
                                   float* logits_out) {
    if (!logits_out) return MATMUL_DECODER_ERR_INVALID_ARG;
    return matmul_decoder_step(c, token_id, embedding, logits_out);
}

int matmul_decoder_step_head(MatmulDecoderContext* c, int token_id, const float* embedding,
                             int lm_head_idx, float* output_logits) {
    if (!c) return MATMUL_DECODER_ERR_INVALID_ARG;
    if (c->n_lm <= 1) return matmul_decoder_step(c, token_id, embedding, output_logits);
    if (lm_head_idx < 0 || lm_head_idx >= c->n_lm) return MATMUL_DECODER_ERR_INVALID_ARG;
    int rc = step_checks(c, token_id, embedding);
    if (rc) return rc;
    if (ensure_graphs(c)) return MATMUL_DECODER_ERR_RKNN;
    if (c->persist) pthread_mutex_lock(&g_persist_mu);
    rc = set_state(c, token_id, embedding);
    if (c->persist) {
        /* the one launch advances the position; the head does not */
        if (!rc) rc = launch_persist(c, 0, NULL, c->seq_len);
        if (!rc) rc = run_head(c, &c->lm_heads[lm_head_idx], NULL, 0, c->stream);
    } else {
        if (!rc) rc = launch_seq(c, c->g_layers, seq_layers);
        if (!rc) rc = run_head(c, &c->lm_heads[lm_head_idx], NULL, 1, c->stream);
    }
    if (!rc && output_logits)
        rc = mdxrt_d2h_async(c->h_io, c->d_logits, (size_t)c->lm_vocab * 4, c->stream);
    if (!rc) rc = mdxrt_d2h_async(c->h_state, c->d_state, sizeof(mdx_state), c->stream);
    if (!rc) rc = mdxrt_stream_sync(c->stream);
    if (c->persist) pthread_mutex_unlock(&g_persist_mu);
    if (rc) return MATMUL_DECODER_ERR_RKNN;
    if (c->h_state->pad[1]) {
        if (persist_retry(c)) return matmul_decoder_step_head(c, token_id, embedding, lm_head_idx, output_logits);
        fprintf(stderr, "[MatmulDecoder] step failed: a workgroup timed out waiting for another\n");
        return MATMUL_DECODER_ERR_RKNN;
    }
    c->seq_len++;
    if (output_logits) memcpy(output_logits, c->h_io, (size_t)c->lm_vocab * 4);
    return c->h_state->argmax;
}

static int prefill_chunk(MatmulDecoderContext* c, const float* emb, int M) {
    memcpy(c->h_io, emb, (size_t)M * c->d * 4);
    memset(c->h_state, 0, sizeof(mdx_state));
    c->h_state->pos = c->seq_len;
    int rc = mdxrt_h2d_async(c->d_bhidden, c->h_io, (size_t)M * c->d * 4, c->stream);
    if (!rc) rc = mdxrt_h2d_async(c->d_state, c->h_state, sizeof(mdx_state), c->stream);
    void* g = rc ? NULL : prefill_graph(c, M);
    if (!rc) rc = g ? mdxrt_graph_launch(g, c->stream) : run_prefill(c, M, c->stream);
    if (!rc) rc = mdxrt_stream_sync(c->stream);
    if (rc) {
        fprintf(stderr, "[BatchPrefill] failed: %s\n", mdxrt_last_error());
        return MATMUL_DECODER_ERR_RKNN;
    }
    c->seq_len += M;
    return 0;
}

int matmul_decoder_prefill_batch(MatmulDecoderContext* c, const float* embeddings, int M) {
    if (!c || !embeddings || M <= 0) return MATMUL_DECODER_ERR_INVALID_ARG;
    if (c->seq_len + M > c->max_seq) {
        fprintf(stderr, "[BatchPrefill] KV cache overflow: seq_len=%d + M=%d > max=%d\n", c->seq_len,
                M, c->max_seq);
        return MATMUL_DECODER_ERR_INVALID_ARG;
    }
    for (int off = 0; off < M; off += c->max_m) {
        const int n = M - off < c->max_m ? M - off : c->max_m;
        int rc = prefill_chunk(c, embeddings + (size_t)off * c->d, n);
        if (rc) return rc;
    }
    return MATMUL_DECODER_OK;
}

void matmul_decoder_clear_kv_cache(MatmulDecoderContext* c) {
    if (c) c->seq_len = 0;
}

int matmul_decoder_get_seq_len(const MatmulDecoderContext* c) { return c ? c->seq_len : 0; }

const MatmulDecoderConfig* matmul_decoder_get_config(const MatmulDecoderContext* c) {
    return c ? &c->config : NULL;
}

void matmul_decoder_get_stats(const MatmulDecoderContext* c, MatmulDecoderStats* stats) {
    if (c && stats) *stats = c->stats;
}

/* Reference: src/matmul_decoder.c:2316-2324 (greedy whatever top_k says). */
int matmul_sample_token(const float* logits, int vocab_size, SamplingParams* params) {
    (void)params;
    if (!logits || vocab_size <= 0) return MATMUL_DECODER_ERR_INVALID_ARG;
    float best = logits[0];
    int idx = 0;
    for (int i = 1; i < vocab_size; i++)
        if (logits[i] > best) {
            best = logits[i];
            idx = i;
        }
    return idx;
}

int matmul_decoder_generate(MatmulDecoderContext* c, const int* prompt_tokens, int n_prompt,
                            int max_new_tokens, SamplingParams* params, GenerateCallback callback,
                            void* user_data) {
    if (!c || (n_prompt > 0 && !prompt_tokens) || n_prompt < 0 || max_new_tokens < 0)
        return MATMUL_DECODER_ERR_INVALID_ARG;
    if (n_prompt == 0) return 0;
    for (int i = 0; i < n_prompt - 1; i++) {
        int rc = matmul_decoder_step(c, prompt_tokens[i], NULL, NULL);
        if (rc < 0) return rc;
    }
    float* logits = (float*)malloc((size_t)c->V * 4);
    if (!logits) return MATMUL_DECODER_ERR_MEMORY;
    int tok = prompt_tokens[n_prompt - 1], n = 0;
    for (; n < max_new_tokens; n++) {
        int next = matmul_decoder_step(c, tok, NULL, logits);
        if (next < 0) {
            free(logits);
            return n > 0 ? n : next;
        }
        if (params && params->top_k > 1) next = matmul_sample_token(logits, c->V, params);
        if (callback) callback(next, NULL, user_data);
        tok = next;
    }
    free(logits);
    return n;
}

/* ------------------------------------------------------------------------ */
/* Additive entry points (mdx_ext.h)                                         */
/* ------------------------------------------------------------------------ */

static int int_cmp(const void* a, const void* b) {
    const int x = *(const int*)a, y = *(const int*)b;
    return (x > y) - (x < y);
}

int md_sample_prepare(const SamplingParams* p, int V, float uniform, int* k_out, int** toks,
                      int* n_toks) {
    *toks = NULL;
    *n_toks = 0;
    if (!p || V <= 0 || !(uniform >= 0.0f && uniform <= 1.0f) || !(p->temperature > 0.0f) ||
        !isfinite(p->temperature) || !(p->repeat_penalty > 0.0f) || !isfinite(p->repeat_penalty) ||
        p->top_p != p->top_p || p->n_repeat_tokens < 0 || p->n_repeat_tokens > MDX_SAMPLE_MAX_REPEAT ||
        (p->n_repeat_tokens > 0 && !p->repeat_tokens))
        return MATMUL_DECODER_ERR_INVALID_ARG;
    const int k = p->top_k <= 1 ? 1 : (p->top_k > V ? V : p->top_k);
    if (k > MDX_SAMPLE_MAX_TOP_K) return MATMUL_DECODER_ERR_INVALID_ARG;
    for (int i = 0; i < p->n_repeat_tokens; i++)
        if (p->repeat_tokens[i] < 0 || p->repeat_tokens[i] >= V) return MATMUL_DECODER_ERR_INVALID_ARG;
    *k_out = k;
    if (p->repeat_penalty == 1.0f || p->n_repeat_tokens == 0) return 0;
    /* once per distinct token */
    int* t = (int*)malloc((size_t)p->n_repeat_tokens * sizeof(int));
    if (!t) return MATMUL_DECODER_ERR_MEMORY;
    memcpy(t, p->repeat_tokens, (size_t)p->n_repeat_tokens * sizeof(int));
    qsort(t, (size_t)p->n_repeat_tokens, sizeof(int), int_cmp);
    int n = 0;
    for (int i = 0; i < p->n_repeat_tokens; i++)
        if (n == 0 || t[i] != t[n - 1]) t[n++] = t[i];
    *toks = t;
    *n_toks = n;
    return 0;
}

int matmul_decoder_step_sample(MatmulDecoderContext* c, int token_id, const float* embedding,
                               const SamplingParams* params, float uniform, float* output_logits) {
    if (!c) return MATMUL_DECODER_ERR_INVALID_ARG;
    if (c->n_lm > 1) return MATMUL_DECODER_ERR_UNSUPPORTED;
    md_sample_req sr = {params, 1, 0, uniform};
    int* toks = NULL;
    int rc = md_sample_prepare(params, c->V, uniform, &sr.k, &toks, &sr.n);
    if (rc) return rc;
    if (sr.n) memcpy(c->h_samp, toks, (size_t)sr.n * sizeof(int));
    free(toks);
    return do_step(c, token_id, embedding, output_logits, 1, &sr);
}

int mdx_kv_fill_normal(MatmulDecoderContext* c, int n_pos, uint64_t seed) {
    if (!c || n_pos < 0 || n_pos > c->max_seq) return MATMUL_DECODER_ERR_INVALID_ARG;
    const size_t n = (size_t)n_pos * c->kvd;
    float* f = (float*)malloc(n * 4 + 4);
    uint16_t* h = (uint16_t*)malloc(n * 2 + 2);
    if (!f || !h) {
        free(f);
        free(h);
        return MATMUL_DECODER_ERR_MEMORY;
    }
    char name[64];
    int rc = 0;
    for (int l = 0; l < c->L && !rc; l++) {
        for (int which = 0; which < 2 && !rc; which++) {
            snprintf(name, sizeof name, which ? "kv/v/%02d" : "kv/k/%02d", l);
            mdx_synth_fill_normal(f, n, mdx_synth_seed(seed, name), 0.0, 1.0);
            for (size_t i = 0; i < n; i++) h[i] = mdx_f32_to_f16(f[i]);
            rc = mdxrt_h2d(which ? (void*)c->layers[l].vc : (void*)c->layers[l].kc, h, n * 2);
        }
    }
    free(f);
    free(h);
    if (rc) return MATMUL_DECODER_ERR_RKNN;
    c->seq_len = n_pos;
    return 0;
}

int mdx_kv_read(const MatmulDecoderContext* c, int layer, int pos0, int n, float* k, float* v) {
    if (!c || layer < 0 || layer >= c->L || pos0 < 0 || n < 0 || pos0 + n > c->max_seq || !k || !v)
        return MATMUL_DECODER_ERR_INVALID_ARG;
    const size_t cnt = (size_t)n * c->kvd;
    uint16_t* h = (uint16_t*)malloc(cnt * 2 + 2);
    if (!h) return MATMUL_DECODER_ERR_MEMORY;
    int rc = mdxrt_d2h(h, c->layers[layer].kc + (size_t)pos0 * c->kvd, cnt * 2);
    for (size_t i = 0; !rc && i < cnt; i++) k[i] = mdx_f16_to_f32(h[i]);
    if (!rc) rc = mdxrt_d2h(h, c->layers[layer].vc + (size_t)pos0 * c->kvd, cnt * 2);
    for (size_t i = 0; !rc && i < cnt; i++) v[i] = mdx_f16_to_f32(h[i]);
    free(h);
    return rc ? MATMUL_DECODER_ERR_RKNN : 0;
}

int mdx_prefill_logits(MatmulDecoderContext* c, const float* embeddings, int M, float* logits) {
    if (!c || c->n_lm > 1) return MATMUL_DECODER_ERR_INVALID_ARG;
    int rc = matmul_decoder_prefill_batch(c, embeddings, M);
    if (rc) return rc;
    const int last = (M - 1) % c->max_m;
    rc = mdx_launch_copy_row(c->d_bhidden, last, c->d, c->d_hidden, c->stream);
    if (!rc) rc = run_head(c, &c->lm, NULL, 0, c->stream);
    if (!rc && logits) rc = mdxrt_d2h_async(c->h_io, c->d_logits, (size_t)c->V * 4, c->stream);
    if (!rc) rc = mdxrt_d2h_async(c->h_state, c->d_state, sizeof(mdx_state), c->stream);
    if (!rc) rc = mdxrt_stream_sync(c->stream);
    if (rc) return MATMUL_DECODER_ERR_RKNN;
    if (logits) memcpy(logits, c->h_io, (size_t)c->V * 4);
    return c->h_state->argmax;
}

int mdx_generate_greedy(MatmulDecoderContext* c, int first_token, int n_steps, int* out_tokens,
                        float* device_ms) {
    if (!c || c->n_lm > 1 || n_steps <= 0 || !out_tokens || first_token < 0 || first_token >= c->V)
        return MATMUL_DECODER_ERR_INVALID_ARG;
    if (c->seq_len + n_steps > c->max_seq) return MATMUL_DECODER_ERR_INVALID_ARG;
    if (ensure_graphs(c)) return MATMUL_DECODER_ERR_RKNN;
    if (c->tokens_cap < n_steps) {
        /* the greedy graph bakes in the token buffer address: rebuild it */
        mdxrt_graph_destroy(c->g_greedy);
        c->g_greedy = NULL;
        mdxrt_free(c->d_tokens);
        c->d_tokens = NULL;
        int cap = n_steps < 1024 ? 1024 : n_steps;
        if (mdxrt_malloc((void**)&c->d_tokens, (size_t)cap * 4)) return MATMUL_DECODER_ERR_MEMORY;
        c->tokens_cap = cap;
    }
    if (!c->persist && c->use_graphs && !c->g_greedy && capture(c, seq_greedy, &c->g_greedy))
        return MATMUL_DECODER_ERR_RKNN;
    if (c->persist) pthread_mutex_lock(&g_persist_mu);
    memset(c->h_state, 0, sizeof(mdx_state));
    c->h_state->pos = c->seq_len;
    c->h_state->token = first_token;
    int rc = mdxrt_h2d_async(c->d_state, c->h_state, sizeof(mdx_state), c->stream);
    if (!rc) rc = mdxrt_event_record(c->ev0, c->stream);
    for (int i = 0; i < n_steps && !rc; i++) {
        if (!c->persist) {
            rc = launch_seq(c, c->g_greedy, seq_greedy);
        } else if (c->persist_head) {
            rc = launch_persist(c, 1, c->d_tokens, c->seq_len + i);
        } else {
            rc = launch_persist(c, 0, NULL, c->seq_len + i);
            if (!rc) rc = run_head(c, &c->lm, c->d_tokens, 0, c->stream);
        }
    }
    if (!rc) rc = mdxrt_event_record(c->ev1, c->stream);
    if (!rc) rc = mdxrt_d2h_async(c->h_state, c->d_state, sizeof(mdx_state), c->stream);
    if (!rc) rc = mdxrt_stream_sync(c->stream);
    if (c->persist) pthread_mutex_unlock(&g_persist_mu);
    if (!rc) rc = mdxrt_d2h(out_tokens, c->d_tokens, (size_t)n_steps * 4);
    if (rc) return MATMUL_DECODER_ERR_RKNN;
    if (c->h_state->pad[1]) {
        if (persist_retry(c)) return mdx_generate_greedy(c, first_token, n_steps, out_tokens, device_ms);
        fprintf(stderr, "[MatmulDecoder] generate failed: a workgroup timed out waiting for another\n");
        return MATMUL_DECODER_ERR_RKNN;
    }
    if (device_ms) mdxrt_event_elapsed_ms(c->ev0, c->ev1, device_ms);
    c->seq_len += n_steps;
    return 0;
}

static int time_projection_launch(MatmulDecoderContext* c, int sel, int l, const mdx_wdesc* w0,
                                  float eps);
static int time_projection_bytes(const MatmulDecoderContext* c, int sel, double* bytes);

int mdx_time_projection(MatmulDecoderContext* c, const char* which, int iters, float* avg_us,
                        double* bytes) {
    if (!c || !which || iters <= 0) return MATMUL_DECODER_ERR_INVALID_ARG;
    int sel = -1;
    if (!strcmp(which, "qkv")) sel = 0;
    else if (!strcmp(which, "o")) sel = 1;
    else if (!strcmp(which, "gate_up")) sel = 2;
    else if (!strcmp(which, "down")) sel = 3;
    else if (!strcmp(which, "lm_head")) sel = 4;
    else if (!strcmp(which, "layer")) sel = 5;
    if (sel < 0 || (sel == 4 && c->n_lm > 1)) return MATMUL_DECODER_ERR_INVALID_ARG;
    const float eps = c->config.rms_eps;
    const mdx_wdesc* w0 = sel == 4 ? &c->lm : NULL;
    /* the per-layer selections replay a captured graph of one pass over the
     * layers when iters is a multiple of the layer count, so the host's launch
     * overhead is not what is timed */
    const int use_graph = c->use_graphs && sel != 4 && iters % c->L == 0;
    void* g = NULL;
    int rc = 0;
    if (use_graph) {
        rc = mdxrt_graph_begin(c->stream);
        int rc2 = 0;
        for (int l = 0; l < c->L && !rc2; l++) rc2 = time_projection_launch(c, sel, l, w0, eps);
        if (!rc) rc = mdxrt_graph_end(c->stream, &g);
        if (rc2) rc = rc2;
        if (!rc) rc = mdxrt_graph_launch(g, c->stream);   /* warm-up */
    }
    if (!rc) rc = mdxrt_event_record(c->ev0, c->stream);
    for (int i = 0; i < iters / c->L && !rc && use_graph; i++) rc = mdxrt_graph_launch(g, c->stream);
    for (int i = 0; i < iters && !rc && !use_graph; i++) rc = time_projection_launch(c, sel, i % c->L, w0, eps);
    if (!rc) rc = mdxrt_event_record(c->ev1, c->stream);
    if (!rc) rc = mdxrt_stream_sync(c->stream);
    if (g) mdxrt_graph_destroy(g);
    if (rc) return MATMUL_DECODER_ERR_RKNN;
    float ms = 0.0f;
    mdxrt_event_elapsed_ms(c->ev0, c->ev1, &ms);
    if (avg_us) *avg_us = ms * 1000.0f / iters;
    return time_projection_bytes(c, sel, bytes);
}

static int time_projection_launch(MatmulDecoderContext* c, int sel, int l, const mdx_wdesc* w0,
                                  float eps) {
    int rc = 0;
    md_layer* ly = &c->layers[l];
    switch (sel) {
        case 0: rc = mdx_launch_norm_gemv(c->d_hidden, ly->in_norm, eps, &ly->qkv, 0, c->d_tmp, c->stream); break;
        case 1: rc = mdx_launch_gemv_add(c->d_attn16, &ly->o, c->d_tmp, c->stream); break;
        case 2: rc = mdx_launch_norm_gemv(c->d_hidden, ly->post_norm, eps, &ly->gu, 1, c->d_act16, c->stream); break;
        case 3: rc = mdx_launch_gemv_add(c->d_act16, &ly->down, c->d_tmp, c->stream); break;
        case 5:
            /* the seven projections of one layer with their RMSNorms: merged
             * q|k|v, o (+residual), merged gate|up (+SwiGLU), down (+residual) */
            rc = mdx_launch_norm_gemv(c->d_hidden, ly->in_norm, eps, &ly->qkv, 0, c->d_qkv, c->stream);
            if (!rc) rc = mdx_launch_gemv_add(c->d_attn16, &ly->o, c->d_tmp, c->stream);
            if (!rc) rc = mdx_launch_norm_gemv(c->d_tmp, ly->post_norm, eps, &ly->gu, 1, c->d_act16, c->stream);
            if (!rc) rc = mdx_launch_gemv_add(c->d_act16, &ly->down, c->d_tmp, c->stream);
            break;
        default:
            rc = mdx_launch_lmhead(c->d_hidden, c->d_final_norm, eps, w0, c->d_logits,
                                   c->d_partial, c->d_state, NULL, 0, c->stream);
    }
    return rc;
}

static int time_projection_bytes(const MatmulDecoderContext* c, int sel, double* bytes) {
    if (bytes && sel == 5) {
        /* weights and scales of the four launches, the two norm vectors, and
         * the activations each one reads and writes */
        const md_layer* ly = &c->layers[0];
        const mdx_wdesc* ws[4] = {&ly->qkv, &ly->o, &ly->gu, &ly->down};
        double b = 0.0;
        for (int i = 0; i < 4; i++)
            b += (double)md_row_bytes(ws[i]->kind, ws[i]->K) * ws[i]->N + (ws[i]->scale ? 4.0 * ws[i]->N : 0.0);
        b += 2.0 * 4.0 * c->d;                                   /* norm weights */
        b += 4.0 * c->d + 4.0 * ly->qkv.N;                       /* qkv: hidden in, y out */
        b += 2.0 * ly->o.K + 8.0 * c->d;                         /* o: fp16 in, read+write h */
        b += 4.0 * c->d + 2.0 * ly->gu.N / 2;                    /* gate/up: h in, act out */
        b += 2.0 * ly->down.K + 8.0 * c->d;                      /* down */
        *bytes = b;
    } else if (bytes) {
        const mdx_wdesc* w = sel == 4 ? &c->lm
                             : sel == 0 ? &c->layers[0].qkv
                             : sel == 1 ? &c->layers[0].o
                             : sel == 2 ? &c->layers[0].gu
                                        : &c->layers[0].down;
        double b = (double)md_row_bytes(w->kind, w->K) * w->N + (w->scale ? 4.0 * w->N : 0.0);
        const double xin = (sel == 0 || sel == 2 || sel == 4) ? 4.0 * w->K * 2 : 2.0 * w->K;
        const double yout = sel == 2 ? 2.0 * w->N / 2 : (sel == 1 || sel == 3 ? 8.0 * w->N : 4.0 * w->N);
        *bytes = b + xin + yout;
    }
    return 0;
}

int mdx_time_prefill(MatmulDecoderContext* c, const float* embeddings, int M, int iters,
                     float* avg_ms) {
    if (!c || !embeddings || M <= 0 || M > c->max_m || iters <= 0) return MATMUL_DECODER_ERR_INVALID_ARG;
    if (c->seq_len + M > c->max_seq) return MATMUL_DECODER_ERR_INVALID_ARG;
    void* g = prefill_graph(c, M);
    if (!g && c->use_graphs) return MATMUL_DECODER_ERR_RKNN;
    memcpy(c->h_io, embeddings, (size_t)M * c->d * 4);
    memset(c->h_state, 0, sizeof(mdx_state));
    c->h_state->pos = c->seq_len;
    int rc = mdxrt_event_record(c->ev0, c->stream);
    for (int i = 0; i < iters && !rc; i++) {
        rc = mdxrt_h2d_async(c->d_bhidden, c->h_io, (size_t)M * c->d * 4, c->stream);
        if (!rc) rc = mdxrt_h2d_async(c->d_state, c->h_state, sizeof(mdx_state), c->stream);
        if (!rc) rc = g ? mdxrt_graph_launch(g, c->stream) : run_prefill(c, M, c->stream);
    }
    if (!rc) rc = mdxrt_event_record(c->ev1, c->stream);
    if (!rc) rc = mdxrt_stream_sync(c->stream);
    if (rc) return MATMUL_DECODER_ERR_RKNN;
    float ms = 0.0f;
    mdxrt_event_elapsed_ms(c->ev0, c->ev1, &ms);
    if (avg_ms) *avg_ms = ms / iters;
    return 0;
}

const char* mdx_version(void) { return "1.0.0 gfx950"; }
int mdx_device_count(void) { return mdxrt_device_count(); }

int mdx_copy_probe(size_t bytes, int iters) {
    if (bytes == 0 || iters <= 0) return MATMUL_DECODER_ERR_INVALID_ARG;
    void *a = NULL, *b = NULL, *s = NULL;
    int rc = mdxrt_malloc(&a, bytes) || mdxrt_malloc(&b, bytes) || mdxrt_stream_create(&s);
    if (!rc) rc = mdxrt_fill_u32(a, 0x3f800000u, bytes / 4, s);
    for (int i = 0; i < iters && !rc; i++) rc = mdxrt_d2d_async(b, a, bytes, s);
    if (!rc) rc = mdxrt_stream_sync(s);
    if (s) mdxrt_stream_destroy(s);
    mdxrt_free(a);
    mdxrt_free(b);
    return rc ? MATMUL_DECODER_ERR_RKNN : 0;
}

int mdx_trace_step(MatmulDecoderContext* c, int token_id, unsigned long long* out, int cap) {
    if (!c || !out) return MATMUL_DECODER_ERR_INVALID_ARG;
    if (!c->persist_head) return MATMUL_DECODER_ERR_UNSUPPORTED;
    int rc = step_checks(c, token_id, NULL);
    if (rc) return rc;
    const int ev = mdx_persist_trace_events(c->L);
    if ((long long)cap < 256LL * ev) return MATMUL_DECODER_ERR_INVALID_ARG;
    unsigned long long* d = NULL;
    if (mdxrt_malloc((void**)&d, (size_t)256 * ev * 8)) return MATMUL_DECODER_ERR_MEMORY;
    pthread_mutex_lock(&g_persist_mu);
    rc = set_state(c, token_id, NULL);
    if (!rc) rc = mdxrt_fill_u32(d, 0u, (size_t)256 * ev * 2, c->stream);
    c->pargs.trace = d;
    c->pargs.trace_stride = ev;
    if (!rc) rc = launch_persist(c, 1, NULL, c->seq_len);
    c->pargs.trace = NULL;
    c->pargs.trace_stride = 0;
    if (!rc) rc = mdxrt_d2h_async(c->h_state, c->d_state, sizeof(mdx_state), c->stream);
    if (!rc) rc = mdxrt_stream_sync(c->stream);
    pthread_mutex_unlock(&g_persist_mu);
    if (!rc) rc = mdxrt_d2h(out, d, (size_t)256 * ev * 8);
    mdxrt_free(d);
    if (rc || c->h_state->pad[1]) return MATMUL_DECODER_ERR_RKNN;
    c->seq_len++;
    return ev;
}

int mdx_debug_persist_poison_retry(MatmulDecoderContext* c) {
    if (!c || !c->persist) return MATMUL_DECODER_ERR_INVALID_ARG;
    c->poison_retry = 1;
    return 0;
}

int mdx_debug_persist_spin_limit(MatmulDecoderContext* c, unsigned rounds) {
    if (!c) return MATMUL_DECODER_ERR_INVALID_ARG;
    if (!c->persist) return MATMUL_DECODER_ERR_UNSUPPORTED;
    c->spin_once = rounds;
    return 0;
}

int mdx_debug_persist_kv_stream(MatmulDecoderContext* c, int mode) {
    if (!c || mode < -1 || mode > 1) return MATMUL_DECODER_ERR_INVALID_ARG;
    if (!c->persist) return MATMUL_DECODER_ERR_UNSUPPORTED;
    c->kv_stream_force = mode;
    return 0;
}

int mdx_debug_persist_local_exchange(MatmulDecoderContext* c, int mode) {
    if (!c || mode < -1 || mode > 1) return MATMUL_DECODER_ERR_INVALID_ARG;
    if (!c->persist) return MATMUL_DECODER_ERR_UNSUPPORTED;
    if (!c->lx_buf) return MATMUL_DECODER_ERR_UNSUPPORTED;
    /* words left from steps that ran the other way could carry a current
     * epoch once the step counter wraps: start from zero words */
    if (mode != c->lx_force &&
        (mdxrt_fill_u32(c->lx_buf, 0u, mdx_persist_xbuf_bytes() / 4, c->stream) ||
         mdxrt_stream_sync(c->stream)))
        return MATMUL_DECODER_ERR_RKNN;
    c->lx_force = mode;
    return 0;
}

int mdx_decode_path(const MatmulDecoderContext* c) {
    if (!c) return MATMUL_DECODER_ERR_INVALID_ARG;
    return c->persist ? (c->persist_head ? 1 : 2) : 0;
}
const char* mdx_last_error(void) { return mdxrt_last_error(); }
