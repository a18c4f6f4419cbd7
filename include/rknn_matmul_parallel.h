/*
 * rknn_matmul_parallel.h — the standalone parallel GEMM ABI, served on one
 * MI355X (gfx950).
 *
 * Drop-in replacement for the reference header of the same name
 * (reference: include/rknn_matmul_parallel.h:1-114).  The reference splits
 * the N columns of a [K,N] weight across two NPU-core worker threads; here
 * one device kernel covers all N columns, so `n_workers` is validated (N must
 * divide evenly, as in the reference) but does not split the work.
 */
#ifndef RKNN_MATMUL_PARALLEL_H
#define RKNN_MATMUL_PARALLEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RMP_MAX_WORKERS 2

/* Reference: include/rknn_matmul_parallel.h:31-35.  All types produce fp32
 * output.  The weight buffer is read as fp16 [K,N] for every type, as the
 * reference does (src/rknn_matmul_parallel.c:241-251). */
typedef enum {
    RMP_TYPE_FP16_FP16 = 0,
    RMP_TYPE_FP16_INT4 = 1,
    RMP_TYPE_FP16_INT8 = 2,
} RmpMatmulType;

/* Reference: include/rknn_matmul_parallel.h:38-41. */
typedef enum {
    RMP_LAYOUT_NORMAL = 0,
    RMP_LAYOUT_NATIVE = 1,
} RmpWeightLayout;

/* Reference: include/rknn_matmul_parallel.h:46-53. */
typedef struct {
    int M;
    int K;
    int N;
    RmpMatmulType type;
    RmpWeightLayout layout;
    int n_workers;              /* <= 0 means RMP_MAX_WORKERS */
} RmpConfig;

typedef struct RmpContext RmpContext;

/* Copies the fp16 [K,N] weights into device memory (reference:
 * src/rknn_matmul_parallel.c:200-300).  Any K >= 1 (a K that is not a
 * multiple of 32 is zero-padded on the device); N must divide by n_workers.
 * Returns NULL on failure. */
RmpContext* rmp_create(const RmpConfig* config, const void* weights, const float* scales);

/* output[M,N] fp32 = fp16 input[M,K] x W (reference:
 * src/rknn_matmul_parallel.c:303-338).  Row-major [M,N] output for every M. */
int rmp_run(RmpContext* ctx, const int16_t* input, float* output);

void rmp_destroy(RmpContext* ctx);

/* Mean milliseconds per rmp_run over n_runs after 3 warm-up runs
 * (reference: src/rknn_matmul_parallel.c:380-418). */
float rmp_benchmark(RmpContext* ctx, int n_runs);

/* last rmp_benchmark result x 1.37, the reference's fixed factor
 * (src/rknn_matmul_parallel.c:420-425). */
float rmp_get_single_core_time(RmpContext* ctx);

#ifdef __cplusplus
}
#endif

#endif /* RKNN_MATMUL_PARALLEL_H */
