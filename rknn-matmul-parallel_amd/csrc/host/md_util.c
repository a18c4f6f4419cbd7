/*
 * md_util.c — host helpers: fp16 conversion, the synthetic-data generator,
 * file IO, the INT8 lm_head quantiser and the device-layout repack.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <pthread.h>
#include <time.h>

#include "md_internal.h"

int md_verbose(void) {
    static int v = -1;
    if (v < 0) {
        const char* e = getenv("MATMUL_DECODER_VERBOSE");
        v = (e && e[0] && e[0] != '0') ? 1 : 0;
    }
    return v;
}

double md_now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1000.0 + ts.tv_nsec / 1e6;
}

/* ---- fp16 ---- */

static inline uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float float_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t mdx_f32_to_f16(float f) {
    const uint32_t x = bits_of(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t mag = x & 0x7fffffffu;
    if (mag > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((mag >> 13) & 0x3ffu)); /* NaN */
    if (mag >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);                        /* overflow */
    if (mag < 0x38800000u) {
        /* subnormal result: scale so the half ulp (2^-24) becomes 1, then
         * round the integer part to nearest even */
        if (mag < 0x33000000u) return (uint16_t)sign;
        const uint32_t exp = mag >> 23;
        const uint32_t man = (mag & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - exp;
        uint32_t q = man >> shift;
        const uint32_t rest = man - (q << shift);
        const uint32_t tie = 1u << (shift - 1u);
        q += (rest > tie) || (rest == tie && (q & 1u));
        return (uint16_t)(sign | q);
    }
    /* normal: drop 13 mantissa bits with round-half-even; a carry out of the
     * mantissa increments the exponent (and reaches inf above 65504) */
    uint32_t h = ((mag - 0x38000000u) >> 13);
    const uint32_t rest = mag & 0x1fffu;
    h += (rest > 0x1000u) || (rest == 0x1000u && (h & 1u));
    return (uint16_t)(sign | h);
}

float mdx_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t man = h & 0x3ffu;
    if (exp == 0x1fu) return float_of(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        float v = (float)man * 0x1p-24f;
        return sign ? -v : v;
    }
    return float_of(sign | ((exp + 112u) << 23) | (man << 13));
}

/* ---- generator ---- */

#define MD_STREAM_CHUNK ((size_t)1 << 20)

static inline uint64_t sm64(uint64_t* state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t mdx_synth_seed(uint64_t base, const char* name) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (const unsigned char* p = (const unsigned char*)name; *p; ++p) {
        h ^= (uint64_t)*p;
        h *= 0x100000001b3ull;
    }
    uint64_t st = h ^ base;
    return sm64(&st);
}

typedef struct {
    float* out;
    size_t n, c0, c1;
    uint64_t seed;
    double mean, std;
} fill_job;

static void fill_chunks(const fill_job* j) {
    const double tau = 6.283185307179586476925286766559;
    for (size_t c = j->c0; c < j->c1; c++) {
        uint64_t st = j->seed + (uint64_t)c * 0xD1B54A32D192ED03ull;
        const size_t lo = c * MD_STREAM_CHUNK;
        const size_t hi = lo + MD_STREAM_CHUNK < j->n ? lo + MD_STREAM_CHUNK : j->n;
        for (size_t i = lo; i < hi; i += 2) {
            const double u1 = 1.0 - (double)(sm64(&st) >> 11) * 0x1.0p-53;
            const double u2 = (double)(sm64(&st) >> 11) * 0x1.0p-53;
            const double rad = sqrt(-2.0 * log(u1));
            const double ang = tau * u2;
            j->out[i] = (float)(j->mean + j->std * (rad * cos(ang)));
            if (i + 1 < hi) j->out[i + 1] = (float)(j->mean + j->std * (rad * sin(ang)));
        }
    }
}

static void* fill_thread(void* arg) {
    fill_chunks((const fill_job*)arg);
    return NULL;
}

/* Chunks are independent streams, so the result does not depend on how many
 * threads fill them. */
void mdx_synth_fill_normal(float* out, size_t n, uint64_t seed, double mean, double std) {
    const size_t nchunks = (n + MD_STREAM_CHUNK - 1) / MD_STREAM_CHUNK;
    size_t nt = nchunks < 16 ? nchunks : 16;
    if (nt <= 1) {
        fill_job j = {out, n, 0, nchunks, seed, mean, std};
        fill_chunks(&j);
        return;
    }
    fill_job jobs[16];
    pthread_t th[16];
    int started[16] = {0};
    for (size_t t = 0; t < nt; t++) {
        jobs[t] = (fill_job){out, n, nchunks * t / nt, nchunks * (t + 1) / nt, seed, mean, std};
        started[t] = pthread_create(&th[t], NULL, fill_thread, &jobs[t]) == 0;
        if (!started[t]) fill_chunks(&jobs[t]);
    }
    for (size_t t = 0; t < nt; t++)
        if (started[t]) pthread_join(th[t], NULL);
}

/* ---- files ---- */

void* md_read_file(const char* path, size_t bytes) {
    FILE* f = fopen(path, "rb");
    if (!f) return NULL;
    void* buf = malloc(bytes ? bytes : 1);
    size_t got = buf ? fread(buf, 1, bytes, f) : 0;
    fclose(f);
    if (!buf || got != bytes) {
        free(buf);
        return NULL;
    }
    return buf;
}

float* md_read_f32_first(const char* dir, const char* const* names, size_t n) {
    char path[1024];
    for (int i = 0; names[i]; i++) {
        snprintf(path, sizeof path, "%s/%s", dir, names[i]);
        float* p = (float*)md_read_file(path, n * sizeof(float));
        if (p) return p;
    }
    return NULL;
}

int md_write_file(const char* path, const void* data, size_t bytes) {
    FILE* f = fopen(path, "wb");
    if (!f) return -1;
    size_t put = fwrite(data, 1, bytes, f);
    int rc = fclose(f);
    return (put == bytes && rc == 0) ? 0 : -1;
}

/* ---- INT8 lm_head quantiser (reference: src/matmul_decoder.c:1216-1244) ---- */

void mdx_quantize_lm_head(int8_t* q, float* scales, const uint16_t* lm_f16, int V, int K) {
    for (int v = 0; v < V; v++) {
        const uint16_t* row = lm_f16 + (size_t)v * K;
        float amax = 0.0f;
        for (int k = 0; k < K; k++) {
            const float a = fabsf(mdx_f16_to_f32(row[k]));
            if (a > amax) amax = a;
        }
        scales[v] = amax / 127.0f;
        const float inv = amax > 0 ? 127.0f / amax : 0.0f;
        int8_t* dst = q + (size_t)v * K;
        for (int k = 0; k < K; k++) {
            int qi = (int)roundf(mdx_f16_to_f32(row[k]) * inv);
            dst[k] = (int8_t)(qi < -128 ? -128 : (qi > 127 ? 127 : qi));
        }
    }
}

/* ---- device-layout repack ---- */

size_t md_row_bytes(int dev_kind, int K) {
    switch (dev_kind) {
        case MDX_W_F16: return (size_t)K * 2;
        case MDX_W_I8: return (size_t)K;
        case MDX_W_I4: return (size_t)K / 2;
        default: return (size_t)K * 4;
    }
}

/* Signed value of element (k, n) of an on-disk projection. */
static inline int disk_int(const md_host_proj* p, int k, int n) {
    if (p->kind == 1) return ((const int8_t*)p->data)[(size_t)k * p->N + n];
    const uint8_t b = ((const uint8_t*)p->data)[(size_t)k * (p->N / 2) + (n >> 1)];
    const int nib = (n & 1) ? (b >> 4) : (b & 0xf);
    return nib >= 8 ? nib - 16 : nib;
}

int md_repack_rows(const md_host_proj* p, int dst_kind, void* dst_rows, float* dst_scale,
                   int row0) {
    const int K = p->K, N = p->N;
    const size_t rb = md_row_bytes(dst_kind, K);
    if (dst_kind == MDX_W_F16) {
        for (int n = 0; n < N; n++) {
            uint16_t* dst = (uint16_t*)((uint8_t*)dst_rows + (size_t)(row0 + n) * rb);
            if (p->kind == 0) {
                const uint16_t* src = (const uint16_t*)p->data;
                for (int k = 0; k < K; k++) dst[k] = src[(size_t)k * N + n];
            } else {
                for (int k = 0; k < K; k++) dst[k] = mdx_f32_to_f16((float)disk_int(p, k, n));
            }
        }
    } else if (dst_kind == MDX_W_I8) {
        if (p->kind == 0) return -1;
        for (int n = 0; n < N; n++) {
            int8_t* dst = (int8_t*)((uint8_t*)dst_rows + (size_t)(row0 + n) * rb);
            for (int k = 0; k < K; k++) dst[k] = (int8_t)disk_int(p, k, n);
        }
    } else if (dst_kind == MDX_W_I4) {
        if (p->kind != 2 || K % 8) return -1;
        for (int n = 0; n < N; n++) {
            uint32_t* dst = (uint32_t*)((uint8_t*)dst_rows + (size_t)(row0 + n) * rb);
            for (int w = 0; w < K / 8; w++) {
                uint32_t word = 0;
                for (int i = 0; i < 4; i++) {
                    const uint32_t lo = (uint32_t)disk_int(p, 8 * w + 2 * i, n) & 0xfu;
                    const uint32_t hi = (uint32_t)disk_int(p, 8 * w + 2 * i + 1, n) & 0xfu;
                    word |= lo << (4 * i);
                    word |= hi << (4 * i + 16);
                }
                dst[w] = word;
            }
        }
    } else {
        return -1;
    }
    if (dst_scale)
        for (int n = 0; n < N; n++) dst_scale[row0 + n] = p->scale ? p->scale[n] : 1.0f;
    return 0;
}
