/*
 * md_rmp.c — rknn_matmul_parallel.h on one GPU (reference:
 * src/rknn_matmul_parallel.c:200-425).
 *
 * The reference copies an fp16 [K,N] weight into two [K,N/2] halves, one per
 * NPU-core worker thread, and gathers their outputs.  Here the weight lives
 * in device memory once, in the W^T row layout, and one GEMV (M = 1) or MFMA
 * GEMM (M <= 64 per launch) produces all N columns.  Behaviour kept from the
 * reference: N must divide by n_workers, the weights are read as fp16 for
 * every RmpMatmulType, scales are ignored, rmp_get_single_core_time is the
 * last benchmark times 1.37.  Fixed on purpose: rmp_run writes a row-major
 * [M,N] fp32 output for every M (the reference's worker-major gather only
 * equals [M,N] when M == 1) and rmp_benchmark uses an fp32 output buffer.
 *
 * Any K is accepted, as in the reference: the kernels step K in blocks of
 * 32, so a ragged K is zero-padded to Kp (zero weight rows, and input rows
 * staged with zero tails in pinned memory); each padded term adds +0 to the
 * fp32 sums.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "md_internal.h"
#include "rknn_matmul_parallel.h"

struct RmpContext {
    RmpConfig config;
    int Kp;                 /* K rounded up to a multiple of 32 */
    void* stream;
    uint8_t* d_w;
    uint16_t* d_x;
    float* d_y;
    float* d_scratch;
    uint16_t* h_x;          /* pinned [M][Kp] staging when Kp != K (tails stay 0) */
    mdx_wdesc w;
    float last_benchmark_ms;
};

RmpContext* rmp_create(const RmpConfig* config, const void* weights, const float* scales) {
    (void)scales;
    if (!config || !weights) return NULL;
    const int n_workers = config->n_workers > 0 ? config->n_workers : RMP_MAX_WORKERS;
    if (config->M <= 0 || config->K <= 0 || config->N <= 0) return NULL;
    if (config->N % n_workers != 0) {
        fprintf(stderr, "rmp_create: N=%d must be divisible by n_workers=%d\n", config->N, n_workers);
        return NULL;
    }
    if (mdxrt_device_count() <= 0) {
        fprintf(stderr, "rmp_create: no GPU visible to the HIP runtime\n");
        return NULL;
    }
    RmpContext* c = (RmpContext*)calloc(1, sizeof *c);
    if (!c) return NULL;
    c->config = *config;
    c->config.n_workers = n_workers;
    const int M = config->M, K = config->K, N = config->N;
    const int Kp = (K + 31) / 32 * 32;
    c->Kp = Kp;
    const int mchunk = M < 64 ? M : 64;
    /* [Kp,N] with zero rows k >= K, then the device row layout */
    uint8_t* wpad = NULL;
    const void* wsrc = weights;
    if (Kp != K) {
        wpad = (uint8_t*)calloc((size_t)Kp * N, 2);
        if (wpad) memcpy(wpad, weights, (size_t)K * N * 2);
        wsrc = wpad;
    }
    md_host_proj p = {0, Kp, N, (void*)wsrc, NULL};
    uint8_t* rows = (uint8_t*)malloc((size_t)Kp * N * 2);
    int rc = rows && wsrc ? md_repack_rows(&p, MDX_W_F16, rows, NULL, 0) : -1;
    free(wpad);
    if (!rc) rc = mdxrt_stream_create(&c->stream);
    if (!rc) rc = mdxrt_malloc((void**)&c->d_w, (size_t)Kp * N * 2);
    if (!rc) rc = mdxrt_malloc((void**)&c->d_x, (size_t)M * Kp * 2);
    if (!rc) rc = mdxrt_malloc((void**)&c->d_y, (size_t)M * N * 4);
    if (!rc) rc = mdxrt_malloc((void**)&c->d_scratch, mdx_gemm_scratch_floats(mchunk, N, Kp) * 4);
    if (!rc) rc = mdxrt_fill_u32(c->d_scratch, 0u, mdx_gemm_scratch_floats(mchunk, N, Kp), c->stream);
    if (!rc && Kp != K) {
        rc = mdxrt_host_alloc((void**)&c->h_x, (size_t)M * Kp * 2);
        if (!rc) memset(c->h_x, 0, (size_t)M * Kp * 2);
    }
    if (!rc) rc = mdxrt_stream_sync(c->stream);
    if (!rc) rc = mdxrt_h2d(c->d_w, rows, (size_t)Kp * N * 2);
    free(rows);
    if (rc) {
        fprintf(stderr, "rmp_create: %s\n", mdxrt_last_error());
        rmp_destroy(c);
        return NULL;
    }
    c->w.w = c->d_w;
    c->w.scale = NULL;
    c->w.kind = MDX_W_F16;
    c->w.K = Kp;
    c->w.N = N;
    return c;
}

int rmp_run(RmpContext* c, const int16_t* input, float* output) {
    if (!c || !input || !output) return -1;
    const int M = c->config.M, K = c->config.K, N = c->config.N, Kp = c->Kp;
    int rc;
    if (Kp == K) {
        rc = mdxrt_h2d_async(c->d_x, input, (size_t)M * K * 2, c->stream);
    } else {
        for (int m = 0; m < M; m++)
            memcpy(c->h_x + (size_t)m * Kp, input + (size_t)m * K, (size_t)K * 2);
        rc = mdxrt_h2d_async(c->d_x, c->h_x, (size_t)M * Kp * 2, c->stream);
    }
    if (M == 1) {
        if (!rc) rc = mdx_launch_gemv_f16in(c->d_x, &c->w, c->d_y, c->stream);
    } else {
        for (int m0 = 0; m0 < M && !rc; m0 += 64) {
            const int mm = M - m0 < 64 ? M - m0 : 64;
            rc = mdx_launch_gemm(c->d_x + (size_t)m0 * Kp, mm, &c->w, 0, c->d_y + (size_t)m0 * N,
                                 c->d_scratch, c->stream);
        }
    }
    if (!rc) rc = mdxrt_d2h_async(output, c->d_y, (size_t)M * N * 4, c->stream);
    if (!rc) rc = mdxrt_stream_sync(c->stream);
    return rc ? -1 : 0;
}

void rmp_destroy(RmpContext* c) {
    if (!c) return;
    if (c->stream) mdxrt_stream_sync(c->stream);
    mdxrt_free(c->d_w);
    mdxrt_free(c->d_x);
    mdxrt_free(c->d_y);
    mdxrt_free(c->d_scratch);
    mdxrt_host_free(c->h_x);
    mdxrt_stream_destroy(c->stream);
    free(c);
}

float rmp_benchmark(RmpContext* c, int n_runs) {
    if (!c || n_runs <= 0) return -1.0f;
    const int M = c->config.M, K = c->config.K, N = c->config.N;
    int16_t* in = (int16_t*)malloc((size_t)M * K * 2);
    float* out = (float*)malloc((size_t)M * N * 4);
    if (!in || !out) {
        free(in);
        free(out);
        return -1.0f;
    }
    /* inputs uniform in [-1, 1), fp16 */
    uint64_t s = 42;
    for (int i = 0; i < M * K; i++) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        const float v = (float)((s >> 40) * 0x1.0p-24) * 2.0f - 1.0f;
        const uint16_t h = mdx_f32_to_f16(v);
        memcpy(&in[i], &h, 2);
    }
    for (int i = 0; i < 3; i++) rmp_run(c, in, out);
    const double t0 = md_now_ms();
    for (int i = 0; i < n_runs; i++) rmp_run(c, in, out);
    const float avg = (float)((md_now_ms() - t0) / n_runs);
    c->last_benchmark_ms = avg;
    free(in);
    free(out);
    return avg;
}

float rmp_get_single_core_time(RmpContext* c) {
    if (!c) return -1.0f;
    return c->last_benchmark_ms * 1.37f;
}
