/*
 * md_kvcache.c — the standalone host KV cache object of matmul_decoder.h
 * (reference: src/matmul_decoder.c:449-502): fp32
 * [layer][max_seq][kv_head][head_dim], zero-initialised, clear() resets only
 * the length.  The decoder itself keeps its cache in device memory.
 */
#include <stdlib.h>
#include <string.h>

#include "md_internal.h"

struct MatmulKVCache {
    float* k_cache;
    float* v_cache;
    int num_layers, num_kv_heads, head_dim, max_seq_len;
    int seq_len;
};

MatmulKVCache* matmul_kv_cache_create(int num_layers, int num_kv_heads, int head_dim,
                                      int max_seq_len) {
    if (num_layers <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_seq_len <= 0) return NULL;
    MatmulKVCache* c = (MatmulKVCache*)calloc(1, sizeof *c);
    if (!c) return NULL;
    c->num_layers = num_layers;
    c->num_kv_heads = num_kv_heads;
    c->head_dim = head_dim;
    c->max_seq_len = max_seq_len;
    const size_t n = (size_t)num_layers * max_seq_len * num_kv_heads * head_dim;
    c->k_cache = (float*)calloc(n, sizeof(float));
    c->v_cache = (float*)calloc(n, sizeof(float));
    if (!c->k_cache || !c->v_cache) {
        matmul_kv_cache_destroy(c);
        return NULL;
    }
    return c;
}

void matmul_kv_cache_clear(MatmulKVCache* cache) {
    if (cache) cache->seq_len = 0;
}

int matmul_kv_cache_get_seq_len(const MatmulKVCache* cache) { return cache ? cache->seq_len : 0; }

void matmul_kv_cache_destroy(MatmulKVCache* cache) {
    if (!cache) return;
    free(cache->k_cache);
    free(cache->v_cache);
    free(cache);
}
