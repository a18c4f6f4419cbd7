/*
 * md_export.c — HuggingFace checkpoint (safetensors) to the reference on-disk
 * format: matmul_decoder_export_hf_model, which the reference declares
 * (include/matmul_decoder.h:467) but never defines.  The output follows the
 * reference exporter examples/qwen3_asr/export_weights.py:128-216 (config.json,
 * embeddings.bin fp32 [V,d], lm_head.bin fp32 when untied, layer_LL/ with the
 * fp32 norms and each projection transposed to [K,N]) and what the loader
 * reads besides (src/matmul_decoder.c:698-926): final_norm.bin, the QK norms,
 * and for INT8/INT4 the <proj>_weight.bin + <proj>_scales.bin pair written by
 * md_write_proj.
 *
 * Input: <hf_model_path>/config.json and every *.safetensors file in the
 * directory (one file or the shards of an index).  Tensors may be F32, F16 or
 * BF16.  The text model's prefix is taken from its embed_tokens tensor
 * ("model." in a plain checkpoint, e.g. "thinker.model." in a multimodal one,
 * whose other towers have layers of their own); every other tensor is looked
 * up under that prefix (the lm_head and final norm by the usual names beside
 * it).  Qwen3's rotary embedding rotates the halves of a head (rope_style 1).
 */
#include <dirent.h>
#include <errno.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include "md_internal.h"

enum { ST_F32 = 0, ST_F16 = 1, ST_BF16 = 2 };

typedef struct {
    char name[192];
    int dtype;
    int ndim;
    long long shape[4];
    unsigned long long begin, end;   /* byte range inside the file's data section */
    int file;
} st_tensor;

typedef struct {
    char (*paths)[1024];
    unsigned long long* data_off;
    int nfiles;
    st_tensor* t;
    int n, cap;
} st_set;

/* ---- a small JSON scanner for safetensors headers and config.json ---------- */

static const char* js_ws(const char* p) {
    while (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t') p++;
    return p;
}

/* String at p (which points at '"'): copies at most cap-1 bytes; returns the
 * position after the closing quote, NULL on malformed input. */
static const char* js_string(const char* p, char* out, size_t cap) {
    if (*p != '"') return NULL;
    p++;
    size_t n = 0;
    while (*p && *p != '"') {
        if (*p == '\\' && p[1]) p++;
        if (n + 1 < cap) out[n++] = *p;
        p++;
    }
    if (*p != '"') return NULL;
    if (cap) out[n] = '\0';
    return p + 1;
}

/* Skips any JSON value. */
static const char* js_skip(const char* p) {
    p = js_ws(p);
    if (*p == '"') {
        char tmp[8];
        return js_string(p, tmp, sizeof tmp);
    }
    if (*p == '{' || *p == '[') {
        const char open = *p, close = open == '{' ? '}' : ']';
        p++;
        for (;;) {
            p = js_ws(p);
            if (*p == close) return p + 1;
            if (open == '{') {
                char tmp[8];
                p = js_string(p, tmp, sizeof tmp);
                if (!p) return NULL;
                p = js_ws(p);
                if (*p != ':') return NULL;
                p++;
            }
            p = js_skip(p);
            if (!p) return NULL;
            p = js_ws(p);
            if (*p == ',') p++;
            else if (*p != close) return NULL;
        }
    }
    /* number or literal */
    while (*p && *p != ',' && *p != '}' && *p != ']' && *p != ' ' && *p != '\n' && *p != '\r' &&
           *p != '\t')
        p++;
    return p;
}

/* Array of up to `cap` integers. */
static const char* js_int_array(const char* p, long long* out, int cap, int* n) {
    p = js_ws(p);
    if (*p != '[') return NULL;
    p++;
    *n = 0;
    for (;;) {
        p = js_ws(p);
        if (*p == ']') return p + 1;
        char* end = NULL;
        const long long v = strtoll(p, &end, 10);
        if (end == p) return NULL;
        if (*n < cap) out[*n] = v;
        (*n)++;
        p = js_ws(end);
        if (*p == ',') p++;
        else if (*p != ']') return NULL;
    }
}

/* ---- safetensors ------------------------------------------------------------ */

static int st_add_file(st_set* s, const char* path) {
    FILE* f = fopen(path, "rb");
    if (!f) return MATMUL_DECODER_ERR_FILE_IO;
    unsigned char len8[8];
    if (fread(len8, 1, 8, f) != 8) {
        fclose(f);
        return MATMUL_DECODER_ERR_FILE_IO;
    }
    unsigned long long hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | len8[i];
    if (hlen == 0 || hlen > (1ull << 30)) {
        fclose(f);
        return MATMUL_DECODER_ERR_FILE_IO;
    }
    char* h = (char*)malloc((size_t)hlen + 1);
    if (!h || fread(h, 1, (size_t)hlen, f) != (size_t)hlen) {
        free(h);
        fclose(f);
        return MATMUL_DECODER_ERR_FILE_IO;
    }
    fclose(f);
    h[hlen] = '\0';

    const int fi = s->nfiles;
    char(*np)[1024] = (char(*)[1024])realloc(s->paths, (size_t)(fi + 1) * sizeof *np);
    unsigned long long* no = (unsigned long long*)realloc(s->data_off, (size_t)(fi + 1) * sizeof *no);
    if (np) s->paths = np;
    if (no) s->data_off = no;
    if (!np || !no) {
        free(h);
        return MATMUL_DECODER_ERR_MEMORY;
    }
    snprintf(s->paths[fi], sizeof s->paths[fi], "%s", path);
    s->data_off[fi] = 8 + hlen;
    s->nfiles = fi + 1;

    int rc = MATMUL_DECODER_OK;
    const char* p = js_ws(h);
    if (*p != '{') rc = MATMUL_DECODER_ERR_FILE_IO;
    else p++;
    while (rc == MATMUL_DECODER_OK) {
        p = js_ws(p);
        if (*p == '}') break;
        st_tensor t;
        memset(&t, 0, sizeof t);
        t.dtype = -1;
        p = js_string(p, t.name, sizeof t.name);
        if (!p) { rc = MATMUL_DECODER_ERR_FILE_IO; break; }
        p = js_ws(p);
        if (*p != ':') { rc = MATMUL_DECODER_ERR_FILE_IO; break; }
        p = js_ws(p + 1);
        if (strcmp(t.name, "__metadata__") == 0 || *p != '{') {
            p = js_skip(p);
        } else {
            p++;
            long long offs[2] = {0, 0};
            int have_offs = 0;
            for (;;) {
                p = js_ws(p);
                if (*p == '}') { p++; break; }
                char key[32];
                p = js_string(p, key, sizeof key);
                if (!p) break;
                p = js_ws(p);
                if (*p != ':') { p = NULL; break; }
                p = js_ws(p + 1);
                if (strcmp(key, "dtype") == 0) {
                    char dt[16];
                    p = js_string(p, dt, sizeof dt);
                    if (p) t.dtype = strcmp(dt, "F32") == 0 ? ST_F32 : strcmp(dt, "F16") == 0 ? ST_F16
                                     : strcmp(dt, "BF16") == 0 ? ST_BF16 : -1;
                } else if (strcmp(key, "shape") == 0) {
                    p = js_int_array(p, t.shape, 4, &t.ndim);
                } else if (strcmp(key, "data_offsets") == 0) {
                    int n = 0;
                    p = js_int_array(p, offs, 2, &n);
                    have_offs = n == 2;
                } else {
                    p = js_skip(p);
                }
                if (!p) break;
                p = js_ws(p);
                if (*p == ',') p++;
            }
            if (!p || !have_offs || offs[0] < 0 || offs[1] < offs[0]) { rc = MATMUL_DECODER_ERR_FILE_IO; break; }
            t.begin = (unsigned long long)offs[0];
            t.end = (unsigned long long)offs[1];
            t.file = fi;
            if (s->n == s->cap) {
                const int cap = s->cap ? 2 * s->cap : 256;
                st_tensor* nt = (st_tensor*)realloc(s->t, (size_t)cap * sizeof *nt);
                if (!nt) { rc = MATMUL_DECODER_ERR_MEMORY; break; }
                s->t = nt;
                s->cap = cap;
            }
            s->t[s->n++] = t;
        }
        if (!p) { rc = MATMUL_DECODER_ERR_FILE_IO; break; }
        p = js_ws(p);
        if (*p == ',') p++;
    }
    free(h);
    if (rc) fprintf(stderr, "[MatmulDecoder] export: malformed safetensors header in %s\n", path);
    return rc;
}

static int name_cmp(const void* a, const void* b) {
    return strcmp((const char*)a, (const char*)b);
}

static int st_open_dir(st_set* s, const char* dir) {
    memset(s, 0, sizeof *s);
    DIR* d = opendir(dir);
    if (!d) {
        fprintf(stderr, "[MatmulDecoder] export: cannot open %s: %s\n", dir, strerror(errno));
        return MATMUL_DECODER_ERR_FILE_IO;
    }
    char(*names)[256] = NULL;
    int n = 0, cap = 0;
    struct dirent* e;
    while ((e = readdir(d)) != NULL) {
        const size_t len = strlen(e->d_name);
        if (len < 12 || strcmp(e->d_name + len - 12, ".safetensors") != 0 || len >= 256) continue;
        if (n == cap) {
            cap = cap ? 2 * cap : 8;
            char(*nn)[256] = (char(*)[256])realloc(names, (size_t)cap * sizeof *nn);
            if (!nn) break;
            names = nn;
        }
        snprintf(names[n++], 256, "%s", e->d_name);
    }
    closedir(d);
    if (n == 0) {
        free(names);
        fprintf(stderr, "[MatmulDecoder] export: no .safetensors file in %s\n", dir);
        return MATMUL_DECODER_ERR_FILE_IO;
    }
    qsort(names, (size_t)n, sizeof *names, name_cmp);
    int rc = MATMUL_DECODER_OK;
    for (int i = 0; i < n && !rc; i++) {
        char path[1300];
        snprintf(path, sizeof path, "%s/%s", dir, names[i]);
        rc = st_add_file(s, path);
    }
    free(names);
    return rc;
}

static void st_close(st_set* s) {
    free(s->paths);
    free(s->data_off);
    free(s->t);
    memset(s, 0, sizeof *s);
}

/* The tensor whose name ends with `suffix` (the shortest such name). */
static const st_tensor* st_find(const st_set* s, const char* suffix) {
    const size_t sl = strlen(suffix);
    const st_tensor* best = NULL;
    for (int i = 0; i < s->n; i++) {
        const size_t nl = strlen(s->t[i].name);
        if (nl < sl || strcmp(s->t[i].name + nl - sl, suffix) != 0) continue;
        if (nl > sl && s->t[i].name[nl - sl - 1] != '.') continue;
        if (!best || nl < strlen(best->name)) best = &s->t[i];
    }
    return best;
}

static float bf16_to_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static const st_tensor* st_exact(const st_set* s, const char* name) {
    for (int i = 0; i < s->n; i++)
        if (strcmp(s->t[i].name, name) == 0) return &s->t[i];
    return NULL;
}

/* Reads the tensor `name` of exactly `count` elements as fp32 (NULL if absent
 * or of another size). */
static float* st_read_f32(const st_set* s, const char* name, size_t count) {
    const st_tensor* t = st_exact(s, name);
    if (!t) return NULL;
    if (t->ndim > 4) return NULL;
    size_t elems = 1;
    for (int i = 0; i < t->ndim; i++) {
        if (t->shape[i] < 0 || t->shape[i] > (1ll << 32)) return NULL;
        elems *= (size_t)t->shape[i];
    }
    const size_t esz = t->dtype == ST_F32 ? 4 : 2;
    if (t->dtype < 0 || elems != count || t->end - t->begin != elems * esz) {
        fprintf(stderr, "[MatmulDecoder] export: %s has an unexpected dtype or shape\n", t->name);
        return NULL;
    }
    FILE* f = fopen(s->paths[t->file], "rb");
    if (!f) return NULL;
    void* raw = malloc(elems * esz);
    float* out = (float*)malloc(elems * 4);
    int ok = raw && out && fseeko(f, (off_t)(s->data_off[t->file] + t->begin), SEEK_SET) == 0 &&
             fread(raw, 1, elems * esz, f) == elems * esz;
    fclose(f);
    if (ok) {
        if (t->dtype == ST_F32) {
            memcpy(out, raw, elems * 4);
        } else {
            const uint16_t* h = (const uint16_t*)raw;
            for (size_t i = 0; i < elems; i++)
                out[i] = t->dtype == ST_F16 ? mdx_f16_to_f32(h[i]) : bf16_to_f32(h[i]);
        }
    }
    free(raw);
    if (!ok) {
        free(out);
        return NULL;
    }
    return out;
}

/* ---- HF config.json --------------------------------------------------------- */

typedef struct {
    long long hidden, heads, kv_heads, head_dim, ffn, layers, vocab;
    double eps, theta;
    int tied;
} hf_config;

/* Keys of the top-level object, overridden by those of a "text_config"
 * object when there is one (multimodal checkpoints nest the text model). */
static void hf_scan(const char* p, hf_config* c, int depth) {
    p = js_ws(p);
    if (*p != '{') return;
    p++;
    for (;;) {
        p = js_ws(p);
        if (*p == '}' || !*p) return;
        char key[64];
        p = js_string(p, key, sizeof key);
        if (!p) return;
        p = js_ws(p);
        if (*p != ':') return;
        p = js_ws(p + 1);
        if (*p == '{' && depth == 0 && strcmp(key, "text_config") == 0) {
            hf_scan(p, c, 1);
            p = js_skip(p);
        } else if (*p == '-' || (*p >= '0' && *p <= '9')) {
            char* end = NULL;
            const double v = strtod(p, &end);
#define HK(k) (strcmp(key, k) == 0)
            if (HK("hidden_size")) c->hidden = (long long)v;
            else if (HK("num_attention_heads")) c->heads = (long long)v;
            else if (HK("num_key_value_heads")) c->kv_heads = (long long)v;
            else if (HK("head_dim")) c->head_dim = (long long)v;
            else if (HK("intermediate_size")) c->ffn = (long long)v;
            else if (HK("num_hidden_layers")) c->layers = (long long)v;
            else if (HK("vocab_size")) c->vocab = (long long)v;
            else if (HK("rms_norm_eps")) c->eps = v;
            else if (HK("rope_theta")) c->theta = v;
#undef HK
            p = end && end != p ? end : js_skip(p);
        } else if (strncmp(p, "true", 4) == 0 || strncmp(p, "false", 5) == 0) {
            if (strcmp(key, "tie_word_embeddings") == 0) c->tied = *p == 't';
            p = js_skip(p);
        } else {
            p = js_skip(p);
        }
        if (!p) return;
        p = js_ws(p);
        if (*p == ',') p++;
    }
}

static int hf_read_config(const char* dir, hf_config* c) {
    char path[1100];
    snprintf(path, sizeof path, "%s/config.json", dir);
    FILE* f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "[MatmulDecoder] export: cannot open %s\n", path);
        return MATMUL_DECODER_ERR_FILE_IO;
    }
    fseek(f, 0, SEEK_END);
    const long size = ftell(f);
    fseek(f, 0, SEEK_SET);
    char* text = size > 0 ? (char*)malloc((size_t)size + 1) : NULL;
    const size_t got = text ? fread(text, 1, (size_t)size, f) : 0;
    fclose(f);
    if (!text) return MATMUL_DECODER_ERR_FILE_IO;
    text[got] = '\0';
    memset(c, 0, sizeof *c);
    c->eps = 1e-6;
    c->theta = 1e6;
    c->tied = 1;
    hf_scan(text, c, 0);
    free(text);
    if (c->head_dim <= 0 && c->heads > 0) c->head_dim = c->hidden / c->heads;
    const long long lim = 1ll << 22;   /* keeps every product below in int range */
    if (c->hidden <= 0 || c->heads <= 0 || c->kv_heads <= 0 || c->head_dim <= 0 || c->ffn <= 0 ||
        c->layers <= 0 || c->vocab <= 0 || c->hidden > 65536 || c->ffn > 262144 ||
        c->heads * c->head_dim > 65536 || c->kv_heads * c->head_dim > 65536 || c->layers > 4096 ||
        c->vocab > lim) {
        fprintf(stderr, "[MatmulDecoder] export: %s lacks a model dimension or has one out of range\n", path);
        return MATMUL_DECODER_ERR_INVALID_ARG;
    }
    return MATMUL_DECODER_OK;
}

/* ---- export ----------------------------------------------------------------- */

static int make_dir(const char* path) {
    if (mkdir(path, 0755) == 0 || errno == EEXIST) return 0;
    fprintf(stderr, "[MatmulDecoder] export: mkdir %s: %s\n", path, strerror(errno));
    return MATMUL_DECODER_ERR_FILE_IO;
}

static int copy_f32(const st_set* s, const char* name, size_t n, const char* out_path, int required) {
    float* v = st_read_f32(s, name, n);
    if (!v) {
        if (required) fprintf(stderr, "[MatmulDecoder] export: tensor %s missing\n", name);
        return required ? MATMUL_DECODER_ERR_FILE_IO : 1;
    }
    const int rc = md_write_file(out_path, v, n * 4) ? MATMUL_DECODER_ERR_FILE_IO : 0;
    free(v);
    return rc;
}

int matmul_decoder_export_hf_model(const char* hf_model_path, const char* output_dir,
                                   QuantizationType quant_type) {
    if (!hf_model_path || !output_dir) return MATMUL_DECODER_ERR_INVALID_ARG;
    const int quant = quant_type == QUANT_INT8 ? 1
                      : (quant_type == QUANT_INT4 || quant_type == QUANT_INT4_G128) ? 2 : 0;
    hf_config hc;
    int rc = hf_read_config(hf_model_path, &hc);
    if (rc) return rc;
    const int d = (int)hc.hidden, hd = (int)hc.head_dim, F = (int)hc.ffn;
    const int qd = (int)(hc.heads * hd), kvd = (int)(hc.kv_heads * hd), V = (int)hc.vocab;
    if (quant == 2 && (qd % 2 || kvd % 2 || d % 2 || F % 2)) return MATMUL_DECODER_ERR_INVALID_ARG;

    st_set s;
    rc = st_open_dir(&s, hf_model_path);
    if (rc) {
        st_close(&s);
        return rc;
    }
    char path[1400], ldir[1200], name[256], pre[192] = "";
    const st_tensor* emb = st_find(&s, "embed_tokens.weight");
    if (!emb) {
        fprintf(stderr, "[MatmulDecoder] export: no embed_tokens tensor in %s\n", hf_model_path);
        st_close(&s);
        return MATMUL_DECODER_ERR_FILE_IO;
    }
    snprintf(pre, sizeof pre, "%.*s", (int)(strlen(emb->name) - strlen("embed_tokens.weight")), emb->name);
    /* the lm_head sits beside the text model: "<outer>lm_head.weight" */
    char lm_name[256];
    {
        const size_t pl = strlen(pre);
        const size_t outer = pl >= 6 && strcmp(pre + pl - 6, "model.") == 0 ? pl - 6 : pl;
        snprintf(lm_name, sizeof lm_name, "%.*slm_head.weight", (int)outer, pre);
    }
    rc = make_dir(output_dir);

    /* QK norms present in the checkpoint (Qwen3) or not (Qwen2) */
    snprintf(name, sizeof name, "%slayers.0.self_attn.q_norm.weight", pre);
    const int has_qk = st_exact(&s, name) != NULL;
    const int tied = hc.tied || st_exact(&s, lm_name) == NULL;
    if (!rc) {
        snprintf(path, sizeof path, "%s/config.json", output_dir);
        FILE* f = fopen(path, "w");
        if (!f) rc = MATMUL_DECODER_ERR_FILE_IO;
        if (!rc) {
            fprintf(f,
                    "{\n  \"name\": \"hf-export\",\n  \"hidden_dim\": %d,\n  \"num_q_heads\": %lld,\n"
                    "  \"num_kv_heads\": %lld,\n  \"head_dim\": %d,\n  \"ffn_dim\": %d,\n"
                    "  \"num_layers\": %lld,\n  \"vocab_size\": %d,\n  \"max_seq_len\": 4096,\n"
                    "  \"rms_eps\": %.9g,\n  \"rope_theta\": %.1f,\n  \"has_qk_norm\": %s,\n"
                    "  \"tie_word_embeddings\": %s,\n  \"rope_style\": 1,\n  \"quant_type\": \"%s\"\n}\n",
                    d, hc.heads, hc.kv_heads, hd, F, hc.layers, V, hc.eps, hc.theta,
                    has_qk ? "true" : "false", tied ? "true" : "false",
                    quant == 0 ? "fp16" : (quant == 1 ? "int8" : "int4"));
            if (fclose(f) != 0) rc = MATMUL_DECODER_ERR_FILE_IO;
        }
    }
    if (!rc) {
        snprintf(path, sizeof path, "%s/embeddings.bin", output_dir);
        rc = copy_f32(&s, emb->name, (size_t)V * d, path, 1);
    }
    if (!rc && !tied) {
        snprintf(path, sizeof path, "%s/lm_head.bin", output_dir);
        rc = copy_f32(&s, lm_name, (size_t)V * d, path, 1);
    }
    if (!rc) {
        snprintf(path, sizeof path, "%s/final_norm.bin", output_dir);
        snprintf(name, sizeof name, "%snorm.weight", pre);
        rc = copy_f32(&s, name, (size_t)d, path, 1);
    }
    static const char* const proj[7] = {"q_proj", "k_proj", "v_proj", "o_proj",
                                        "gate_proj", "up_proj", "down_proj"};
    const int pK[7] = {d, d, d, qd, d, d, F};
    const int pN[7] = {qd, kvd, kvd, d, F, F, d};
    for (long long l = 0; l < hc.layers && !rc; l++) {
        snprintf(ldir, sizeof ldir, "%s/layer_%02lld", output_dir, l);
        rc = make_dir(ldir);
        static const char* const norms[4][2] = {{"input_layernorm", "input_norm"},
                                                {"post_attention_layernorm", "post_attn_norm"},
                                                {"self_attn.q_norm", "q_norm"},
                                                {"self_attn.k_norm", "k_norm"}};
        for (int i = 0; i < 4 && !rc; i++) {
            if (i >= 2 && !has_qk) break;
            snprintf(name, sizeof name, "%slayers.%lld.%s.weight", pre, l, norms[i][0]);
            snprintf(path, sizeof path, "%s/%s.bin", ldir, norms[i][1]);
            rc = copy_f32(&s, name, (size_t)(i >= 2 ? hd : d), path, 1);
        }
        for (int p = 0; p < 7 && !rc; p++) {
            snprintf(name, sizeof name, "%slayers.%lld.%s.%s.weight", pre, l, p < 4 ? "self_attn" : "mlp",
                     proj[p]);
            const int K = pK[p], N = pN[p];
            float* w = st_read_f32(&s, name, (size_t)K * N);   /* HF [N, K] */
            float* wt = w ? (float*)malloc((size_t)K * N * 4) : NULL;
            if (!w || !wt) {
                fprintf(stderr, "[MatmulDecoder] export: tensor %s missing\n", name);
                rc = MATMUL_DECODER_ERR_FILE_IO;
            } else {
                for (int n = 0; n < N; n++)
                    for (int k = 0; k < K; k++) wt[(size_t)k * N + n] = w[(size_t)n * K + k];
                if (md_write_proj(ldir, proj[p], K, N, quant, wt)) rc = MATMUL_DECODER_ERR_FILE_IO;
            }
            free(w);
            free(wt);
        }
    }
    st_close(&s);
    if (!rc && md_verbose())
        printf("[MatmulDecoder] exported %lld layers (%s) to %s\n", hc.layers,
               quant == 0 ? "fp16" : (quant == 1 ? "int8" : "int4"), output_dir);
    return rc;
}
