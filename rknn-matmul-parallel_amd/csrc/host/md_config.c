/*
 * md_config.c — config.json reader (reference: src/matmul_decoder.c:2182-2312).
 *
 * Same contract as the reference: start from the Qwen3-0.6B defaults, then
 * overwrite the keys found at any nesting level.  Keys read by the reference:
 * hidden_dim, num_q_heads, num_kv_heads, head_dim, ffn_dim, num_layers,
 * vocab_size, max_seq_len, rms_eps, rope_theta, has_qk_norm (number or
 * bool), tie_word_embeddings (bool).  Differences, chosen on purpose:
 *   - numbers go through strtod, so "1e-06" is 1e-6 (the reference stops at
 *     the 'e' and reads 1.0);
 *   - keys match exactly (the reference compares only the key's own length,
 *     so a key that is a prefix of a known name also matched);
 *   - "rope_style", "max_batch_prefill", "num_lm_heads",
 *     "lm_head_vocab_size" and "tie_word_embeddings" as 0/1 are read too.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "md_internal.h"

static const char* skip_ws(const char* p) {
    while (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t') p++;
    return p;
}

static void apply_number(MatmulDecoderConfig* c, const char* key, size_t klen, double v) {
#define KEY(name) (klen == sizeof(name) - 1 && memcmp(key, name, klen) == 0)
    if (KEY("hidden_dim")) c->hidden_dim = (int)v;
    else if (KEY("num_q_heads")) c->num_q_heads = (int)v;
    else if (KEY("num_kv_heads")) c->num_kv_heads = (int)v;
    else if (KEY("head_dim")) c->head_dim = (int)v;
    else if (KEY("ffn_dim")) c->ffn_dim = (int)v;
    else if (KEY("num_layers")) c->num_layers = (int)v;
    else if (KEY("vocab_size")) c->vocab_size = (int)v;
    else if (KEY("max_seq_len")) c->max_seq_len = (int)v;
    else if (KEY("rms_eps")) c->rms_eps = (float)v;
    else if (KEY("rope_theta")) c->rope_theta = (float)v;
    else if (KEY("has_qk_norm")) c->has_qk_norm = (int)v;
    else if (KEY("tie_word_embeddings")) c->tie_word_embeddings = (int)v;
    else if (KEY("rope_style")) c->rope_style = (int)v;
    else if (KEY("max_batch_prefill")) c->max_batch_prefill = (int)v;
    else if (KEY("num_lm_heads")) c->num_lm_heads = (int)v;
    else if (KEY("lm_head_vocab_size")) c->lm_head_vocab_size = (int)v;
#undef KEY
}

int matmul_decoder_load_config(const char* json_path, MatmulDecoderConfig* config) {
    if (!json_path || !config) return MATMUL_DECODER_ERR_INVALID_ARG;
    FILE* f = fopen(json_path, "rb");
    if (!f) {
        fprintf(stderr, "[MatmulDecoder] cannot open config %s\n", json_path);
        return MATMUL_DECODER_ERR_FILE_IO;
    }
    fseek(f, 0, SEEK_END);
    long size = ftell(f);
    fseek(f, 0, SEEK_SET);
    if (size < 0) {
        fclose(f);
        return MATMUL_DECODER_ERR_FILE_IO;
    }
    char* text = (char*)malloc((size_t)size + 1);
    if (!text) {
        fclose(f);
        return MATMUL_DECODER_ERR_MEMORY;
    }
    size_t got = fread(text, 1, (size_t)size, f);
    text[got] = '\0';
    fclose(f);

    *config = matmul_decoder_config_qwen3_0_6b();

    const char* p = text;
    while (*p) {
        if (*p != '"') {
            p++;
            continue;
        }
        const char* key = ++p;
        while (*p && *p != '"') p++;
        if (!*p) break;
        const size_t klen = (size_t)(p - key);
        p = skip_ws(p + 1);
        if (*p != ':') continue;     /* a string value, not a key */
        p = skip_ws(p + 1);
        if (*p == '-' || (*p >= '0' && *p <= '9')) {
            char* end = NULL;
            const double v = strtod(p, &end);
            if (end && end != p) {
                apply_number(config, key, klen, v);
                p = end;
            } else {
                p++;
            }
        } else if (strncmp(p, "true", 4) == 0 || strncmp(p, "false", 5) == 0) {
            const int b = (*p == 't');
            if ((klen == 19 && memcmp(key, "tie_word_embeddings", 19) == 0) ||
                (klen == 11 && memcmp(key, "has_qk_norm", 11) == 0))
                apply_number(config, key, klen, b);
            p += b ? 4 : 5;
        }
        /* strings, objects and arrays: keep scanning for the next key */
    }
    free(text);
    if (md_verbose())
        printf("[MatmulDecoder] config: hidden=%d layers=%d heads=%d/%d vocab=%d\n",
               config->hidden_dim, config->num_layers, config->num_q_heads,
               config->num_kv_heads, config->vocab_size);
    return MATMUL_DECODER_OK;
}

