/*
 * md_synth.c — synthetic model writer in the reference on-disk format.
 *
 * Files follow the loader of the reference (src/matmul_decoder.c:698-826,
 * :869-926, :1155-1168): config.json, embeddings.bin fp32 [V,d],
 * layers/layer_LL/{input_norm,post_attn_norm,q_norm,k_norm}.bin fp32,
 * <proj>.bin fp16 [K,N] or <proj>_weight.bin + <proj>_scales.bin, and
 * final_norm.bin.  Random-init semantics of a fresh HF model: projections
 * and embeddings ~N(0, 0.02), norm weights 1.0, lm_head tied.
 *
 * Quantised layouts (defined here; the reference only reads them):
 *   int8: [K,N] row-major, per-column scale = max|col|/127,
 *         q = clamp((int)roundf(w * (127/max)), -128, 127);
 *   int4: [K,N/2], byte (k,j) holds column 2j in its low nibble and 2j+1 in
 *         its high nibble (two's complement), per-column scale =
 *         fp16(max|col|/7) kept as fp32, q = clamp((int)roundf(w / scale), -8, 7).
 */
#include <errno.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include "md_internal.h"

static int ensure_dir(const char* path) {
    if (mkdir(path, 0755) == 0 || errno == EEXIST) return 0;
    fprintf(stderr, "[synth] mkdir %s: %s\n", path, strerror(errno));
    return -1;
}

static int write_ones(const char* path, int n) {
    float* v = (float*)malloc((size_t)n * 4);
    if (!v) return -1;
    for (int i = 0; i < n; i++) v[i] = 1.0f;
    int rc = md_write_file(path, v, (size_t)n * 4);
    free(v);
    return rc;
}

/* Writes one projection given as fp32 [K,N] in the format above (quant 0
 * fp16, 1 int8, 2 int4); shared with the checkpoint exporter. */
int md_write_proj(const char* dir, const char* name, int K, int N, int quant, const float* w) {
    const size_t kn = (size_t)K * N;
    char path[1024];
    int rc = 0;
    if (quant == 0) {
        uint16_t* h = (uint16_t*)malloc(kn * 2);
        if (!h) return -1;
        for (size_t i = 0; i < kn; i++) h[i] = mdx_f32_to_f16(w[i]);
        snprintf(path, sizeof path, "%s/%s.bin", dir, name);
        rc = md_write_file(path, h, kn * 2);
        free(h);
        return rc;
    }
    if (quant == 2 && N % 2) return -1;
    float* sc = (float*)malloc((size_t)N * 4);
    float* amax = (float*)calloc((size_t)N, 4);
    const size_t qbytes = quant == 1 ? kn : kn / 2;
    uint8_t* q = (uint8_t*)calloc(qbytes, 1);
    if (!sc || !amax || !q) rc = -1;
    for (int k = 0; !rc && k < K; k++)
        for (int n = 0; n < N; n++) {
            const float a = fabsf(w[(size_t)k * N + n]);
            if (a > amax[n]) amax[n] = a;
        }
    for (int n = 0; !rc && n < N; n++) {
        if (quant == 1) sc[n] = amax[n] / 127.0f;
        else sc[n] = mdx_f16_to_f32(mdx_f32_to_f16(amax[n] / 7.0f));
    }
    for (int k = 0; !rc && k < K; k++) {
        for (int n = 0; n < N; n++) {
            const float v = w[(size_t)k * N + n];
            if (quant == 1) {
                const float inv = amax[n] > 0 ? 127.0f / amax[n] : 0.0f;
                int qi = (int)roundf(v * inv);
                qi = qi < -128 ? -128 : (qi > 127 ? 127 : qi);
                q[(size_t)k * N + n] = (uint8_t)(int8_t)qi;
            } else {
                int qi = sc[n] > 0 ? (int)roundf(v / sc[n]) : 0;
                qi = qi < -8 ? -8 : (qi > 7 ? 7 : qi);
                uint8_t* b = &q[(size_t)k * (N / 2) + (n >> 1)];
                *b |= (uint8_t)(((unsigned)qi & 0xfu) << ((n & 1) ? 4 : 0));
            }
        }
    }
    snprintf(path, sizeof path, "%s/%s_weight.bin", dir, name);
    if (!rc) rc = md_write_file(path, q, qbytes);
    snprintf(path, sizeof path, "%s/%s_scales.bin", dir, name);
    if (!rc) rc = md_write_file(path, sc, (size_t)N * 4);
    free(sc);
    free(amax);
    free(q);
    return rc;
}

static int write_proj(const char* dir, const char* name, int K, int N, int quant, uint64_t seed,
                      const char* stream_name) {
    const size_t kn = (size_t)K * N;
    float* w = (float*)malloc(kn * 4);
    if (!w) return -1;
    mdx_synth_fill_normal(w, kn, mdx_synth_seed(seed, stream_name), 0.0, 0.02);
    const int rc = md_write_proj(dir, name, K, N, quant, w);
    free(w);
    return rc;
}

int mdx_synth_write_model(const char* dir, const MatmulDecoderConfig* cfg, int quant,
                          uint64_t seed) {
    if (!dir || !cfg || quant < 0 || quant > 2) return MATMUL_DECODER_ERR_INVALID_ARG;
    if (quant == 2 && ((cfg->num_q_heads * cfg->head_dim) % 2 || cfg->ffn_dim % 2 ||
                       cfg->hidden_dim % 2 || (cfg->num_kv_heads * cfg->head_dim) % 2))
        return MATMUL_DECODER_ERR_INVALID_ARG;
    const int d = cfg->hidden_dim, hd = cfg->head_dim;
    const int qd = cfg->num_q_heads * hd, kvd = cfg->num_kv_heads * hd, F = cfg->ffn_dim;
    char path[1024], ldir[1024];
    if (ensure_dir(dir)) return MATMUL_DECODER_ERR_FILE_IO;

    snprintf(path, sizeof path, "%s/config.json", dir);
    FILE* f = fopen(path, "w");
    if (!f) return MATMUL_DECODER_ERR_FILE_IO;
    fprintf(f,
            "{\n  \"name\": \"synthetic\",\n  \"hidden_dim\": %d,\n  \"num_q_heads\": %d,\n"
            "  \"num_kv_heads\": %d,\n  \"head_dim\": %d,\n  \"ffn_dim\": %d,\n"
            "  \"num_layers\": %d,\n  \"vocab_size\": %d,\n  \"max_seq_len\": %d,\n"
            "  \"rms_eps\": %.9f,\n  \"rope_theta\": %.1f,\n  \"has_qk_norm\": %s,\n"
            "  \"tie_word_embeddings\": true,\n  \"rope_style\": %d,\n"
            "  \"max_batch_prefill\": %d,\n  \"num_lm_heads\": %d,\n"
            "  \"lm_head_vocab_size\": %d,\n  \"quant_type\": \"%s\"\n}\n",
            d, cfg->num_q_heads, cfg->num_kv_heads, hd, F, cfg->num_layers, cfg->vocab_size,
            cfg->max_seq_len, (double)cfg->rms_eps, (double)cfg->rope_theta,
            cfg->has_qk_norm ? "true" : "false", cfg->rope_style,
            cfg->max_batch_prefill > 0 ? cfg->max_batch_prefill : 64, cfg->num_lm_heads,
            cfg->lm_head_vocab_size, quant == 0 ? "fp16" : (quant == 1 ? "int8" : "int4"));
    if (fclose(f) != 0) return MATMUL_DECODER_ERR_FILE_IO;

    {
        const size_t n = (size_t)cfg->vocab_size * d;
        float* e = (float*)malloc(n * 4);
        if (!e) return MATMUL_DECODER_ERR_MEMORY;
        mdx_synth_fill_normal(e, n, mdx_synth_seed(seed, "embeddings"), 0.0, 0.02);
        snprintf(path, sizeof path, "%s/embeddings.bin", dir);
        int rc = md_write_file(path, e, n * 4);
        free(e);
        if (rc) return MATMUL_DECODER_ERR_FILE_IO;
    }
    if (cfg->num_lm_heads > 1) {
        const int lv = cfg->lm_head_vocab_size > 0 ? cfg->lm_head_vocab_size : cfg->vocab_size;
        const size_t n = (size_t)lv * d;
        float* e = (float*)malloc(n * 4);
        if (!e) return MATMUL_DECODER_ERR_MEMORY;
        for (int i = 0; i < cfg->num_lm_heads; i++) {
            char sname[64];
            snprintf(sname, sizeof sname, "lm_head_%02d", i);
            mdx_synth_fill_normal(e, n, mdx_synth_seed(seed, sname), 0.0, 0.02);
            snprintf(path, sizeof path, "%s/%s.bin", dir, sname);
            if (md_write_file(path, e, n * 4)) {
                free(e);
                return MATMUL_DECODER_ERR_FILE_IO;
            }
        }
        free(e);
    }

    snprintf(path, sizeof path, "%s/layers", dir);
    if (ensure_dir(path)) return MATMUL_DECODER_ERR_FILE_IO;
    static const char* const names[7] = {"q_proj", "k_proj", "v_proj", "o_proj",
                                         "gate_proj", "up_proj", "down_proj"};
    const int Ks[7] = {d, d, d, qd, d, d, F};
    const int Ns[7] = {qd, kvd, kvd, d, F, F, d};
    for (int l = 0; l < cfg->num_layers; l++) {
        snprintf(ldir, sizeof ldir, "%s/layers/layer_%02d", dir, l);
        if (ensure_dir(ldir)) return MATMUL_DECODER_ERR_FILE_IO;
        snprintf(path, sizeof path, "%s/input_norm.bin", ldir);
        if (write_ones(path, d)) return MATMUL_DECODER_ERR_FILE_IO;
        snprintf(path, sizeof path, "%s/post_attn_norm.bin", ldir);
        if (write_ones(path, d)) return MATMUL_DECODER_ERR_FILE_IO;
        if (cfg->has_qk_norm) {
            snprintf(path, sizeof path, "%s/q_norm.bin", ldir);
            if (write_ones(path, hd)) return MATMUL_DECODER_ERR_FILE_IO;
            snprintf(path, sizeof path, "%s/k_norm.bin", ldir);
            if (write_ones(path, hd)) return MATMUL_DECODER_ERR_FILE_IO;
        }
        for (int p = 0; p < 7; p++) {
            char sname[96];
            snprintf(sname, sizeof sname, "layer_%02d/%s", l, names[p]);
            if (write_proj(ldir, names[p], Ks[p], Ns[p], quant, seed, sname))
                return MATMUL_DECODER_ERR_FILE_IO;
        }
    }
    snprintf(path, sizeof path, "%s/final_norm.bin", dir);
    if (write_ones(path, d)) return MATMUL_DECODER_ERR_FILE_IO;
    return MATMUL_DECODER_OK;
}
