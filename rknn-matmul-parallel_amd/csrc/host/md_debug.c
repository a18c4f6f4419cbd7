/*
 * md_debug.c — single-kernel entry points of mdx_ext.h.  Each call copies
 * its operands to the device in the same layouts the decoder uses, runs the
 * same kernel the decoder runs, and copies the result back, so one kernel
 * can be compared with the oracle in isolation.  Not for the hot path: every
 * call allocates and frees its own device buffers.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "md_internal.h"

typedef struct {
    void* ptr[12];
    int n;
    void* stream;
} dbg_scope;

static void* dalloc(dbg_scope* s, size_t bytes) {
    void* p = NULL;
    if (s->n >= 12 || mdxrt_malloc(&p, bytes)) return NULL;
    s->ptr[s->n++] = p;
    return p;
}

static int scope_open(dbg_scope* s) {
    memset(s, 0, sizeof *s);
    if (mdxrt_device_count() <= 0) return MATMUL_DECODER_ERR_UNSUPPORTED;
    return mdxrt_stream_create(&s->stream) ? MATMUL_DECODER_ERR_RKNN : 0;
}

static int scope_close(dbg_scope* s, int rc) {
    if (s->stream) {
        int r2 = mdxrt_stream_sync(s->stream);
        if (!rc && r2) rc = MATMUL_DECODER_ERR_RKNN;
    }
    for (int i = 0; i < s->n; i++) mdxrt_free(s->ptr[i]);
    mdxrt_stream_destroy(s->stream);
    return rc;
}

/* Uploads a projection given in the on-disk layout (kinds 0-2) or as rows
 * (kinds 3 fp32, 4 fp16) and fills the descriptor. */
static int upload_weights(dbg_scope* s, int kind, int K, int N, const void* w, const float* scales,
                          mdx_wdesc* d) {
    memset(d, 0, sizeof *d);
    d->K = K;
    d->N = N;
    if (kind <= 2) {
        const int dk = kind == 0 ? MDX_W_F16 : (kind == 1 ? MDX_W_I8 : MDX_W_I4);
        md_host_proj p = {kind, K, N, (void*)w, (float*)scales};
        const size_t rb = md_row_bytes(dk, K);
        uint8_t* rows = (uint8_t*)malloc(rb * N);
        float* sc = scales ? (float*)malloc((size_t)N * 4) : NULL;
        int rc = rows && (!scales || sc) ? md_repack_rows(&p, dk, rows, sc, 0) : -1;
        void* dw = rc ? NULL : dalloc(s, rb * N);
        void* ds = (rc || !scales) ? NULL : dalloc(s, (size_t)N * 4);
        if (!rc && (!dw || (scales && !ds))) rc = -1;
        if (!rc) rc = mdxrt_h2d(dw, rows, rb * N);
        if (!rc && scales) rc = mdxrt_h2d(ds, sc, (size_t)N * 4);
        free(rows);
        free(sc);
        if (rc) return MATMUL_DECODER_ERR_INVALID_ARG;
        d->kind = dk;
        d->w = dw;
        d->scale = (const float*)ds;
        return 0;
    }
    const size_t bytes = (size_t)N * K * (kind == 3 ? 4 : 2);
    void* dw = dalloc(s, bytes);
    if (!dw || mdxrt_h2d(dw, w, bytes)) return MATMUL_DECODER_ERR_RKNN;
    if (scales) {
        void* ds = dalloc(s, (size_t)N * 4);
        if (!ds || mdxrt_h2d(ds, scales, (size_t)N * 4)) return MATMUL_DECODER_ERR_RKNN;
        d->scale = (const float*)ds;
    }
    d->kind = kind == 3 ? MDX_W_F32 : MDX_W_F16;
    d->w = dw;
    return 0;
}

int mdx_debug_gemv(int kind, int K, int N, const void* w, const float* scales, const float* x,
                   float* y) {
    if (kind < 0 || kind > 4 || K <= 0 || N <= 0 || !w || !x || !y) return MATMUL_DECODER_ERR_INVALID_ARG;
    dbg_scope s;
    int rc = scope_open(&s);
    if (rc) return rc;
    mdx_wdesc d;
    rc = upload_weights(&s, kind, K, N, w, scales, &d);
    float* dx = rc ? NULL : (float*)dalloc(&s, (size_t)K * 4);
    float* dy = rc ? NULL : (float*)dalloc(&s, (size_t)N * 4);
    if (!rc && (!dx || !dy)) rc = MATMUL_DECODER_ERR_MEMORY;
    if (!rc) rc = mdxrt_h2d(dx, x, (size_t)K * 4);
    if (!rc) rc = mdx_launch_gemv(dx, &d, kind >= 3, dy, s.stream);
    if (!rc) rc = mdxrt_stream_sync(s.stream);
    if (!rc) rc = mdxrt_d2h(y, dy, (size_t)N * 4);
    return scope_close(&s, rc);
}

int mdx_time_gemv(int kind, int K, int N, int copies, int iters, float* avg_us) {
    if ((kind != 0 && kind != 1) || K <= 0 || K % 32 || N <= 0 || copies <= 0 || iters <= 0 || !avg_us)
        return MATMUL_DECODER_ERR_INVALID_ARG;
    if (mdxrt_device_count() <= 0) return MATMUL_DECODER_ERR_UNSUPPORTED;
    const int dk = kind == 0 ? MDX_W_F16 : MDX_W_I8;
    const size_t wb = md_row_bytes(dk, K) * (size_t)N;
    const size_t per = (wb + (size_t)N * 4 + 255) / 256 * 256;     /* weights + scales */
    void *s = NULL, *e0 = NULL, *e1 = NULL;
    uint8_t* buf = NULL;
    float *dx = NULL, *dy = NULL;
    int rc = mdxrt_stream_create(&s) || mdxrt_event_create(&e0) || mdxrt_event_create(&e1);
    if (!rc) rc = mdxrt_malloc((void**)&buf, per * copies);
    if (!rc) rc = mdxrt_malloc((void**)&dx, (size_t)K * 4);
    if (!rc) rc = mdxrt_malloc((void**)&dy, (size_t)N * 4);
    /* weight bytes 0x01, 0x3c01 as fp16 (about 1.0), scales 1/256, x 1.0 */
    if (!rc) rc = mdxrt_fill_u32(buf, kind ? 0x01010101u : 0x3c013c01u, per * copies / 4, s);
    for (int i = 0; i < copies && !rc; i++)
        rc = mdxrt_fill_u32(buf + per * i + wb, 0x3b800000u, (size_t)N, s);
    if (!rc) rc = mdxrt_fill_u32(dx, 0x3f800000u, (size_t)K, s);
    mdx_wdesc w = {NULL, NULL, dk, K, N};
    /* The launches go back to back from a captured graph of one launch per
     * weight copy (replayed iters / copies times), so the host's launch
     * overhead is not what is timed; MDX_GRAPHS=0 issues them one by one. */
    const char* ge = getenv("MDX_GRAPHS");
    const int use_graph = !(ge && ge[0] == '0') && iters % copies == 0;
    void* g = NULL;
    if (!rc && use_graph) {
        rc = mdxrt_graph_begin(s);
        int rc2 = 0;
        for (int i = 0; i < copies && !rc2; i++) {
            w.w = buf + per * i;
            w.scale = (const float*)(buf + per * i + wb);
            rc2 = mdx_launch_gemv(dx, &w, 0, dy, s);
        }
        if (!rc) rc = mdxrt_graph_end(s, &g);
        if (rc2) rc = rc2;
        if (!rc) rc = mdxrt_graph_launch(g, s);   /* warm-up */
    }
    for (int i = 0; i < 8 && !rc && !use_graph; i++) {   /* warm-up */
        w.w = buf + per * (i % copies);
        w.scale = (const float*)(buf + per * (i % copies) + wb);
        rc = mdx_launch_gemv(dx, &w, 0, dy, s);
    }
    if (!rc) rc = mdxrt_event_record(e0, s);
    if (use_graph) {
        for (int i = 0; i < iters / copies && !rc; i++) rc = mdxrt_graph_launch(g, s);
    } else {
        for (int i = 0; i < iters && !rc; i++) {
            w.w = buf + per * (i % copies);
            w.scale = (const float*)(buf + per * (i % copies) + wb);
            rc = mdx_launch_gemv(dx, &w, 0, dy, s);
        }
    }
    if (!rc) rc = mdxrt_event_record(e1, s);
    if (!rc) rc = mdxrt_stream_sync(s);
    float ms = 0.0f;
    if (!rc) rc = mdxrt_event_elapsed_ms(e0, e1, &ms);
    if (!rc) *avg_us = ms * 1000.0f / iters;
    if (s) mdxrt_stream_sync(s);
    if (g) mdxrt_graph_destroy(g);
    mdxrt_free(buf);
    mdxrt_free(dx);
    mdxrt_free(dy);
    mdxrt_event_destroy(e0);
    mdxrt_event_destroy(e1);
    mdxrt_stream_destroy(s);
    return rc ? MATMUL_DECODER_ERR_RKNN : 0;
}

int mdx_debug_gemm(int kind, int M, int K, int N, const void* w, const float* scales,
                   const float* x, float* y) {
    if (kind < 0 || kind > 2 || M <= 0 || M > 64 || K <= 0 || N <= 0 || !w || !x || !y)
        return MATMUL_DECODER_ERR_INVALID_ARG;
    dbg_scope s;
    int rc = scope_open(&s);
    if (rc) return rc;
    mdx_wdesc d;
    rc = upload_weights(&s, kind, K, N, w, scales, &d);
    float* dx = rc ? NULL : (float*)dalloc(&s, (size_t)M * K * 4);
    uint16_t* dx16 = rc ? NULL : (uint16_t*)dalloc(&s, (size_t)M * K * 2);
    float* dy = rc ? NULL : (float*)dalloc(&s, (size_t)M * N * 4);
    float* scr = rc ? NULL : (float*)dalloc(&s, mdx_gemm_scratch_floats(M, N, K) * 4);
    if (!rc && (!dx || !dx16 || !dy || !scr)) rc = MATMUL_DECODER_ERR_MEMORY;
    if (!rc) rc = mdxrt_fill_u32(scr, 0u, mdx_gemm_scratch_floats(M, N, K), s.stream);
    if (!rc) rc = mdxrt_h2d(dx, x, (size_t)M * K * 4);
    if (!rc) rc = mdx_launch_to_f16(dx, M * K, dx16, s.stream);
    if (!rc) rc = mdx_launch_gemm(dx16, M, &d, 0, dy, scr, s.stream);
    if (!rc) rc = mdxrt_stream_sync(s.stream);
    if (!rc) rc = mdxrt_d2h(y, dy, (size_t)M * N * 4);
    return scope_close(&s, rc);
}

int mdx_debug_gemm_residual(int kind, int M, int K, int N, const void* w, const float* scales,
                            const float* x, float* hidden, const float* norm_w, float eps,
                            uint16_t* x16_out) {
    if (kind < 0 || kind > 2 || M <= 0 || M > 64 || K <= 0 || N <= 0 || !w || !x || !hidden ||
        (norm_w && !x16_out))
        return MATMUL_DECODER_ERR_INVALID_ARG;
    dbg_scope s;
    int rc = scope_open(&s);
    if (rc) return rc;
    mdx_wdesc d;
    rc = upload_weights(&s, kind, K, N, w, scales, &d);
    float* dx = rc ? NULL : (float*)dalloc(&s, (size_t)M * K * 4);
    uint16_t* dx16 = rc ? NULL : (uint16_t*)dalloc(&s, (size_t)M * K * 2);
    float* dh = rc ? NULL : (float*)dalloc(&s, (size_t)M * N * 4);
    float* dnw = (rc || !norm_w) ? NULL : (float*)dalloc(&s, (size_t)N * 4);
    uint16_t* dout = (rc || !norm_w) ? NULL : (uint16_t*)dalloc(&s, (size_t)M * N * 2);
    float* scr = rc ? NULL : (float*)dalloc(&s, mdx_gemm_scratch_floats(M, N, K) * 4);
    if (!rc && (!dx || !dx16 || !dh || !scr || (norm_w && (!dnw || !dout)))) rc = MATMUL_DECODER_ERR_MEMORY;
    if (!rc) rc = mdxrt_h2d(dx, x, (size_t)M * K * 4);
    if (!rc) rc = mdxrt_h2d(dh, hidden, (size_t)M * N * 4);
    if (!rc && norm_w) rc = mdxrt_h2d(dnw, norm_w, (size_t)N * 4);
    if (!rc) rc = mdx_launch_to_f16(dx, M * K, dx16, s.stream);
    if (!rc) rc = mdx_launch_gemm_residual_norm(dx16, M, &d, dh, dnw, eps, dout, scr, s.stream);
    if (!rc) rc = mdxrt_stream_sync(s.stream);
    if (!rc) rc = mdxrt_d2h(hidden, dh, (size_t)M * N * 4);
    if (!rc && norm_w) rc = mdxrt_d2h(x16_out, dout, (size_t)M * N * 2);
    return scope_close(&s, rc);
}

static int upload_state(dbg_scope* s, int pos, mdx_state** d_state) {
    mdx_state h;
    memset(&h, 0, sizeof h);
    h.pos = pos;
    *d_state = (mdx_state*)dalloc(s, sizeof h);
    if (!*d_state) return MATMUL_DECODER_ERR_MEMORY;
    return mdxrt_h2d(*d_state, &h, sizeof h);
}

static void widen(const uint16_t* h, float* f, size_t n) {
    for (size_t i = 0; i < n; i++) f[i] = mdx_f16_to_f32(h[i]);
}

/* RoPE tables for rows [0, rows) with the reference formula. */
static int rope_tables(int rows, int hd, float theta, float** ct, float** st) {
    const int half = hd / 2;
    *ct = (float*)malloc((size_t)rows * half * 4);
    *st = (float*)malloc((size_t)rows * half * 4);
    if (!*ct || !*st) return MATMUL_DECODER_ERR_MEMORY;
    for (int p = 0; p < rows; p++)
        for (int i = 0; i < half; i++) {
            const float freq = 1.0f / powf(theta, (2.0f * i) / hd);
            const float angle = p * freq;
            (*ct)[(size_t)p * half + i] = cosf(angle);
            (*st)[(size_t)p * half + i] = sinf(angle);
        }
    return 0;
}

int mdx_debug_attn_decode(int nq, int nkv, int hd, int pos, int rope_style, float theta, float eps,
                          const float* q_norm, const float* k_norm, const float* qkv,
                          const uint16_t* k16, const uint16_t* v16, float* out, uint16_t* k_new,
                          uint16_t* v_new) {
    if (nq <= 0 || nkv <= 0 || hd <= 0 || pos < 0 || !qkv || !out || !k_new || !v_new ||
        (pos > 0 && (!k16 || !v16)))
        return MATMUL_DECODER_ERR_INVALID_ARG;
    dbg_scope s;
    int rc = scope_open(&s);
    if (rc) return rc;
    const int kvd = nkv * hd, qd = nq * hd, rows = pos + 1, half = hd / 2;
    const int max_splits = mdx_attn_max_splits(rows);
    float *ct = NULL, *stt = NULL;
    rc = rope_tables(rows, hd, theta, &ct, &stt);
    mdx_state* st = NULL;
    if (!rc) rc = upload_state(&s, pos, &st);
    const size_t scr = mdx_attn_decode_scratch_bytes(nq, nkv, hd, max_splits);
    float* dcos = (float*)dalloc(&s, (size_t)rows * half * 4);
    float* dsin = (float*)dalloc(&s, (size_t)rows * half * 4);
    float* dqkv = (float*)dalloc(&s, (size_t)(qd + 2 * kvd) * 4);
    uint16_t* dk = (uint16_t*)dalloc(&s, (size_t)rows * kvd * 2);
    uint16_t* dv = (uint16_t*)dalloc(&s, (size_t)rows * kvd * 2);
    void* dscr = dalloc(&s, scr);
    uint16_t* o16 = (uint16_t*)dalloc(&s, (size_t)qd * 2);
    float* dqn = q_norm ? (float*)dalloc(&s, (size_t)hd * 4) : NULL;
    float* dkn = k_norm ? (float*)dalloc(&s, (size_t)hd * 4) : NULL;
    if (!rc && (!dcos || !dsin || !dqkv || !dk || !dv || !dscr || !o16 || (q_norm && !dqn) ||
                (k_norm && !dkn)))
        rc = MATMUL_DECODER_ERR_MEMORY;
    if (!rc) rc = mdxrt_fill_u32(dscr, 0u, scr / 4, s.stream);
    if (!rc) rc = mdxrt_h2d(dcos, ct, (size_t)rows * half * 4);
    if (!rc) rc = mdxrt_h2d(dsin, stt, (size_t)rows * half * 4);
    if (!rc) rc = mdxrt_h2d(dqkv, qkv, (size_t)(qd + 2 * kvd) * 4);
    if (!rc && pos > 0) rc = mdxrt_h2d(dk, k16, (size_t)pos * kvd * 2);
    if (!rc && pos > 0) rc = mdxrt_h2d(dv, v16, (size_t)pos * kvd * 2);
    if (!rc && dqn) rc = mdxrt_h2d(dqn, q_norm, (size_t)hd * 4);
    if (!rc && dkn) rc = mdxrt_h2d(dkn, k_norm, (size_t)hd * 4);
    if (!rc)
        rc = mdx_launch_attn_decode(st, dqkv, dqn, dkn, eps, dcos, dsin, rope_style, nq, nkv, hd, rows,
                                    max_splits, dk, dv, dscr, o16, s.stream);
    if (!rc) rc = mdxrt_stream_sync(s.stream);
    uint16_t* h = (uint16_t*)malloc((size_t)qd * 2);
    if (!rc) rc = h ? mdxrt_d2h(h, o16, (size_t)qd * 2) : MATMUL_DECODER_ERR_MEMORY;
    if (!rc) widen(h, out, (size_t)qd);
    if (!rc) rc = mdxrt_d2h(k_new, dk + (size_t)pos * kvd, (size_t)kvd * 2);
    if (!rc) rc = mdxrt_d2h(v_new, dv + (size_t)pos * kvd, (size_t)kvd * 2);
    free(h);
    free(ct);
    free(stt);
    return scope_close(&s, rc);
}

int mdx_debug_attn_prefill(int nq, int nkv, int hd, int S, int M, const float* q,
                           const uint16_t* k16, const uint16_t* v16, float* out) {
    if (nq <= 0 || nkv <= 0 || hd <= 0 || S < 0 || M <= 0 || !q || !k16 || !v16 || !out)
        return MATMUL_DECODER_ERR_INVALID_ARG;
    dbg_scope s;
    int rc = scope_open(&s);
    if (rc) return rc;
    const int kvd = nkv * hd, qd = nq * hd, L = S + M;
    mdx_state* st = NULL;
    rc = upload_state(&s, S, &st);
    float* dq = (float*)dalloc(&s, (size_t)M * qd * 4);
    uint16_t* dk = (uint16_t*)dalloc(&s, (size_t)L * kvd * 2);
    uint16_t* dv = (uint16_t*)dalloc(&s, (size_t)L * kvd * 2);
    uint16_t* o16 = (uint16_t*)dalloc(&s, (size_t)M * qd * 2);
    if (!rc && (!dq || !dk || !dv || !o16)) rc = MATMUL_DECODER_ERR_MEMORY;
    if (!rc) rc = mdxrt_h2d(dq, q, (size_t)M * qd * 4);
    if (!rc) rc = mdxrt_h2d(dk, k16, (size_t)L * kvd * 2);
    if (!rc) rc = mdxrt_h2d(dv, v16, (size_t)L * kvd * 2);
    if (!rc) rc = mdx_launch_attn_prefill(st, dq, M, dk, dv, nq, nkv, hd, o16, s.stream);
    if (!rc) rc = mdxrt_stream_sync(s.stream);
    uint16_t* h = (uint16_t*)malloc((size_t)M * qd * 2);
    if (!rc) rc = h ? mdxrt_d2h(h, o16, (size_t)M * qd * 2) : MATMUL_DECODER_ERR_MEMORY;
    if (!rc) widen(h, out, (size_t)M * qd);
    free(h);
    return scope_close(&s, rc);
}

int mdx_debug_qk_rope(int nq, int nkv, int hd, int pos, int rope_style, float theta, float eps,
                      const float* q_norm, const float* k_norm, const float* qkv, float* q_out,
                      uint16_t* k16, uint16_t* v16) {
    if (nq <= 0 || nkv <= 0 || hd <= 0 || hd % 2 || pos < 0 || !qkv || !q_out || !k16 || !v16)
        return MATMUL_DECODER_ERR_INVALID_ARG;
    dbg_scope s;
    int rc = scope_open(&s);
    if (rc) return rc;
    const int kvd = nkv * hd, qd = nq * hd, half = hd / 2, rows = pos + 1;
    float *ct = NULL, *stt = NULL;
    rc = rope_tables(rows, hd, theta, &ct, &stt);
    mdx_state* st = NULL;
    if (!rc) rc = upload_state(&s, pos, &st);
    float* dcos = (float*)dalloc(&s, (size_t)rows * half * 4);
    float* dsin = (float*)dalloc(&s, (size_t)rows * half * 4);
    float* dqkv = (float*)dalloc(&s, (size_t)(qd + 2 * kvd) * 4);
    float* dq = (float*)dalloc(&s, (size_t)qd * 4);
    uint16_t* dk = (uint16_t*)dalloc(&s, (size_t)rows * kvd * 2);
    uint16_t* dv = (uint16_t*)dalloc(&s, (size_t)rows * kvd * 2);
    float* dqn = q_norm ? (float*)dalloc(&s, (size_t)hd * 4) : NULL;
    float* dkn = k_norm ? (float*)dalloc(&s, (size_t)hd * 4) : NULL;
    if (!rc && (!dcos || !dsin || !dqkv || !dq || !dk || !dv || (q_norm && !dqn) || (k_norm && !dkn)))
        rc = MATMUL_DECODER_ERR_MEMORY;
    if (!rc) rc = mdxrt_h2d(dcos, ct, (size_t)rows * half * 4);
    if (!rc) rc = mdxrt_h2d(dsin, stt, (size_t)rows * half * 4);
    if (!rc) rc = mdxrt_h2d(dqkv, qkv, (size_t)(qd + 2 * kvd) * 4);
    if (!rc && dqn) rc = mdxrt_h2d(dqn, q_norm, (size_t)hd * 4);
    if (!rc && dkn) rc = mdxrt_h2d(dkn, k_norm, (size_t)hd * 4);
    if (!rc)
        rc = mdx_launch_qk_rope_append_rows(st, dqkv, 1, dqn, dkn, eps, dcos, dsin, nq, nkv, hd,
                                            rope_style, dq, dk, dv, s.stream);
    if (!rc) rc = mdxrt_stream_sync(s.stream);
    if (!rc) rc = mdxrt_d2h(q_out, dq, (size_t)qd * 4);
    if (!rc) rc = mdxrt_d2h(k16, dk + (size_t)pos * kvd, (size_t)kvd * 2);
    if (!rc) rc = mdxrt_d2h(v16, dv + (size_t)pos * kvd, (size_t)kvd * 2);
    free(ct);
    free(stt);
    return scope_close(&s, rc);
}

int mdx_debug_lmhead(int lm_kind, int K, int N, const void* w_rows, const float* scales,
                     const float* hidden, const float* norm_w, float eps, float* logits) {
    if (!(lm_kind == 1 || lm_kind == 3 || lm_kind == 4) || K <= 0 || N <= 0 || !w_rows || !hidden ||
        !norm_w || !logits)
        return MATMUL_DECODER_ERR_INVALID_ARG;
    dbg_scope s;
    int rc = scope_open(&s);
    if (rc) return rc;
    mdx_wdesc d;
    memset(&d, 0, sizeof d);
    d.K = K;
    d.N = N;
    const size_t bytes = (size_t)N * K * (lm_kind == 1 ? 1 : (lm_kind == 3 ? 4 : 2));
    void* dw = dalloc(&s, bytes);
    void* ds = scales ? dalloc(&s, (size_t)N * 4) : NULL;
    float* dh = (float*)dalloc(&s, (size_t)K * 4);
    float* dn = (float*)dalloc(&s, (size_t)K * 4);
    float* dl = (float*)dalloc(&s, (size_t)N * 4);
    void* dp = dalloc(&s, mdx_lmhead_scratch_bytes());
    mdx_state* st = NULL;
    rc = upload_state(&s, 0, &st);
    if (!rc && (!dw || (scales && !ds) || !dh || !dn || !dl || !dp)) rc = MATMUL_DECODER_ERR_MEMORY;
    if (!rc) rc = mdxrt_fill_u32(dp, 0u, mdx_lmhead_scratch_bytes() / 4, s.stream);
    if (!rc) rc = mdxrt_h2d(dw, w_rows, bytes);
    if (!rc && scales) rc = mdxrt_h2d(ds, scales, (size_t)N * 4);
    if (!rc) rc = mdxrt_h2d(dh, hidden, (size_t)K * 4);
    if (!rc) rc = mdxrt_h2d(dn, norm_w, (size_t)K * 4);
    d.w = dw;
    d.scale = (const float*)ds;
    d.kind = lm_kind == 1 ? MDX_W_I8 : (lm_kind == 3 ? MDX_W_F32 : MDX_W_F16);
    if (!rc) rc = mdx_launch_lmhead(dh, dn, eps, &d, dl, dp, st, NULL, 0, s.stream);
    if (!rc) rc = mdxrt_stream_sync(s.stream);
    if (!rc) rc = mdxrt_d2h(logits, dl, (size_t)N * 4);
    mdx_state h;
    if (!rc) rc = mdxrt_d2h(&h, st, sizeof h);
    rc = scope_close(&s, rc);
    return rc ? rc : h.argmax;
}

int mdx_debug_sample(const float* logits, int V, const SamplingParams* params, float uniform,
                     int* out, int* top_idx, float* top_val) {
    if (!logits || !out) return MATMUL_DECODER_ERR_INVALID_ARG;
    int k = 1, n = 0, *toks = NULL;
    int rc = md_sample_prepare(params, V, uniform, &k, &toks, &n);
    if (rc) return rc;
    dbg_scope s;
    rc = scope_open(&s);
    if (rc) {
        free(toks);
        return rc;
    }
    float* dl = (float*)dalloc(&s, (size_t)V * 4);
    int* dt = n ? (int*)dalloc(&s, (size_t)n * 4) : NULL;
    int* dout = (int*)dalloc(&s, 256);
    int* di = (int*)dalloc(&s, (size_t)k * 4);
    float* dv = (float*)dalloc(&s, (size_t)k * 4);
    void* dsc = dalloc(&s, mdx_sample_scratch_bytes());
    if (!dl || (n && !dt) || !dout || !di || !dv || !dsc) rc = MATMUL_DECODER_ERR_MEMORY;
    if (!rc) rc = mdxrt_h2d(dl, logits, (size_t)V * 4);
    if (!rc && n) rc = mdxrt_h2d(dt, toks, (size_t)n * 4);
    if (!rc && n) rc = mdx_launch_repeat_penalty(dl, dt, n, params->repeat_penalty, s.stream);
    if (!rc)
        rc = mdx_launch_topk_sample(dl, V, params->temperature, k, params->top_p, uniform, dsc, dout, di,
                                    dv, s.stream);
    if (!rc) rc = mdxrt_stream_sync(s.stream);
    if (!rc) rc = mdxrt_d2h(out, dout, 2 * sizeof(int));
    if (!rc && top_idx) rc = mdxrt_d2h(top_idx, di, (size_t)k * 4);
    if (!rc && top_val) rc = mdxrt_d2h(top_val, dv, (size_t)k * 4);
    free(toks);
    return scope_close(&s, rc);
}

int mdx_device_malloc(void** ptr, size_t bytes) {
    if (!ptr) return MATMUL_DECODER_ERR_INVALID_ARG;
    return mdxrt_malloc(ptr, bytes) ? MATMUL_DECODER_ERR_MEMORY : 0;
}

int mdx_device_free(void* ptr) { return mdxrt_free(ptr) ? MATMUL_DECODER_ERR_RKNN : 0; }

int mdx_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    if (!dst || !src) return MATMUL_DECODER_ERR_INVALID_ARG;
    return mdxrt_h2d(dst, src, bytes) ? MATMUL_DECODER_ERR_RKNN : 0;
}

int mdx_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (!dst || !src) return MATMUL_DECODER_ERR_INVALID_ARG;
    return mdxrt_d2h(dst, src, bytes) ? MATMUL_DECODER_ERR_RKNN : 0;
}

int mdx_device_synchronize(void) { return mdxrt_device_sync() ? MATMUL_DECODER_ERR_RKNN : 0; }
