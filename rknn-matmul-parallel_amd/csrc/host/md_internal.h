/*
 * md_internal.h — private declarations of the host C runtime.
 */
#ifndef MD_INTERNAL_H
#define MD_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#include "matmul_decoder.h"
#include "mdx_device.h"
#include "mdx_ext.h"

#define MD_ALIGN 256

/* Verbose logging (MATMUL_DECODER_VERBOSE=1); errors always go to stderr. */
int md_verbose(void);
double md_now_ms(void);

/* Whole-file reads; return NULL when the file is missing or short. */
void* md_read_file(const char* path, size_t bytes);
float* md_read_f32_first(const char* dir, const char* const* names, size_t n);
int md_write_file(const char* path, const void* data, size_t bytes);
/* One projection from fp32 [K,N] to <name>.bin (quant 0: fp16 [K,N]) or
 * <name>_weight.bin + <name>_scales.bin (1: int8, 2: int4), in the layouts
 * md_synth.c documents. */
int md_write_proj(const char* dir, const char* name, int K, int N, int quant, const float* w);

/* One projection after loading, in the on-disk semantic:
 * kind 0 fp16 [K,N], 1 int8 [K,N], 2 int4 [K,N/2]; scale may be NULL. */
typedef struct {
    int kind;
    int K, N;
    void* data;
    float* scale;
} md_host_proj;

/* Host repack of one projection into the device layout (W^T rows, see
 * mdx_device.h), writing rows [row0, row0+N) of a merged buffer of kind
 * dst_kind (MDX_W_F16/I8/I4) and its scales (1.0 where the source has none).
 * Returns 0, or -1 if the source cannot be represented in dst_kind. */
int md_repack_rows(const md_host_proj* p, int dst_kind, void* dst_rows, float* dst_scale,
                   int row0);
size_t md_row_bytes(int dev_kind, int K);

/* Validates SamplingParams for the device sampler: *k_out = clamp(top_k, 1,
 * V); *toks (malloc'd, caller frees) = the distinct repeat tokens when the
 * penalty applies, *n_toks their count. */
int md_sample_prepare(const SamplingParams* p, int V, float uniform, int* k_out, int** toks,
                      int* n_toks);

#endif
