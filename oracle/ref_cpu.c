/*
 * ref_cpu.c — the oracle (scalar C restatement of the reference CPU path).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, never by the product.  Conventions are in
 * ref_cpu.h.  Build: oracle/Makefile (gcc -O3 -ffp-contract=off, no
 * intrinsics, no -ffast-math, single thread).
 */
#include "ref_cpu.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

/* ------------------------------------------------------------------------ */
/* fp16 conversions                                                          */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Round to nearest even; overflow to inf; NaN stays NaN
 * (reference: src/cpu_ops.c:383-394, vcvt_f16_f32). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);      /* >= 65536 */
    if (ax >= 0x38800000u) {                                        /* fp16 normal */
        uint32_t h = ((((ax >> 23) - 112u)) << 10) | ((ax >> 13) & 0x3ffu);
        uint32_t rem = ax & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;    /* may carry to inf */
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return (uint16_t)sign;                    /* < 2^-25 */
    {
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t s = 126u - e;                                      /* 14..24 */
        uint32_t h = m >> s;
        uint32_t rem = m & ((1u << s) - 1u);
        uint32_t half = 1u << (s - 1u);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
}

/* Exact widening (reference: src/cpu_ops.c:396-406).  Normal halves rebias
 * the exponent, subnormal halves are mantissa * 2^-24 (exact, and never a
 * denormal fp32 operand), inf/NaN keep their payload; integer masks select
 * the case so that loops over it vectorise. */
static inline float f16_widen(uint16_t h) {
    const uint32_t e = h & 0x7c00u;
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t normal = ((uint32_t)(h & 0x7fffu) << 13) + (112u << 23);
    const uint32_t sub = f2u((float)(int32_t)(h & 0x3ffu) * 0x1p-24f);
    const uint32_t special = ((uint32_t)(h & 0x3ffu) << 13) | 0x7f800000u;
    const uint32_t is_sub = 0u - (uint32_t)(e == 0);
    const uint32_t is_spec = 0u - (uint32_t)(e == 0x7c00u);
    uint32_t r = (normal & ~is_sub) | (sub & is_sub);
    r = (r & ~is_spec) | (special & is_spec);
    return u2f(r | sign);
}

float orc_f16_to_f32(uint16_t h) { return f16_widen(h); }

void orc_vec_f32_to_f16(uint16_t* dst, const float* src, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f32_to_f16(src[i]);
}

void orc_vec_f16_to_f32(float* dst, const uint16_t* src, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = f16_widen(src[i]);
}

/* ------------------------------------------------------------------------ */
/* Generator: SplitMix64 + Box-Muller in double, streams of 2^20 values      */
/* ------------------------------------------------------------------------ */

#define ORC_CHUNK ((size_t)1 << 20)

static inline uint64_t splitmix_next(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline double unit_double(uint64_t* s) {
    return (double)(splitmix_next(s) >> 11) * 0x1.0p-53;
}

uint64_t orc_seed_for(uint64_t base, const char* name) {
    uint64_t h = 0xcbf29ce484222325ull;                 /* FNV-1a 64 */
    for (const unsigned char* p = (const unsigned char*)name; *p; p++) {
        h ^= *p;
        h *= 0x100000001b3ull;
    }
    uint64_t s = h ^ base;
    return splitmix_next(&s);
}

void orc_fill_normal_f32(float* out, size_t n, uint64_t seed, double mean, double std) {
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t c0 = 0; c0 < n; c0 += ORC_CHUNK) {
        uint64_t s = seed + (uint64_t)(c0 / ORC_CHUNK) * 0xD1B54A32D192ED03ull;
        size_t c1 = c0 + ORC_CHUNK < n ? c0 + ORC_CHUNK : n;
        for (size_t i = c0; i < c1; i += 2) {
            double u1 = 1.0 - unit_double(&s);
            double u2 = unit_double(&s);
            double r = sqrt(-2.0 * log(u1));
            double t = two_pi * u2;
            out[i] = (float)(mean + std * (r * cos(t)));
            if (i + 1 < c1) out[i + 1] = (float)(mean + std * (r * sin(t)));
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Element-wise ops                                                          */
/* ------------------------------------------------------------------------ */

/* Reference: src/cpu_ops.c:18-55.  Four lane sums over steps of eight,
 * reduced (l0+l1)+(l2+l3), scalar tail, rms = 1/sqrtf(sum/dim+eps),
 * out = (x*rms)*w.  out may alias x. */
void orc_rms_norm(float* out, const float* x, const float* w, int dim, float eps) {
    float l[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int i;
    for (i = 0; i <= dim - 8; i += 8) {
        for (int j = 0; j < 4; j++) l[j] = l[j] + x[i + j] * x[i + j];
        for (int j = 0; j < 4; j++) l[j] = l[j] + x[i + 4 + j] * x[i + 4 + j];
    }
    float sum = (l[0] + l[1]) + (l[2] + l[3]);
    for (; i < dim; i++) sum += x[i] * x[i];
    float rms = 1.0f / sqrtf(sum / dim + eps);
    for (i = 0; i < dim; i++) out[i] = (x[i] * rms) * w[i];
}

/* Reference: src/matmul_decoder.c:620-631. */
void orc_rope_tables(float* cos_t, float* sin_t, int max_seq, int head_dim, float theta) {
    int half = head_dim / 2;
    for (int pos = 0; pos < max_seq; pos++) {
        for (int i = 0; i < half; i++) {
            float freq = 1.0f / powf(theta, (2.0f * i) / head_dim);
            float angle = pos * freq;
            cos_t[(size_t)pos * half + i] = cosf(angle);
            sin_t[(size_t)pos * half + i] = sinf(angle);
        }
    }
}

/* Reference: src/cpu_ops.c:109-155.  Style 0 rotates (x[2i],x[2i+1]),
 * style 1 rotates (x[i],x[i+half]); each output is two rounded products
 * then one rounded add/sub. */
void orc_apply_rope(float* x, const float* c, const float* s, int num_heads, int head_dim,
                    int rope_style) {
    int half = head_dim / 2;
    for (int h = 0; h < num_heads; h++) {
        float* hx = x + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            int i0 = rope_style == 0 ? 2 * i : i;
            int i1 = rope_style == 0 ? 2 * i + 1 : i + half;
            float x0 = hx[i0], x1 = hx[i1];
            float a = x0 * c[i], b = x1 * s[i];
            float d = x1 * c[i], e = x0 * s[i];
            hx[i0] = a - b;
            hx[i1] = d + e;
        }
    }
}

/* Reference: src/cpu_ops.c:417-445 (recomputes the table formula). */
void orc_apply_rope_batch(float* x, int M, int start_pos, int num_heads, int head_dim,
                          float theta, int rope_style) {
    int half = head_dim / 2;
    float* c = (float*)malloc(sizeof(float) * half);
    float* s = (float*)malloc(sizeof(float) * half);
    for (int t = 0; t < M; t++) {
        int pos = start_pos + t;
        for (int i = 0; i < half; i++) {
            float freq = 1.0f / powf(theta, (2.0f * i) / head_dim);
            float angle = pos * freq;
            c[i] = cosf(angle);
            s[i] = sinf(angle);
        }
        orc_apply_rope(x + (size_t)t * num_heads * head_dim, c, s, num_heads, head_dim,
                       rope_style);
    }
    free(c);
    free(s);
}

/* q.k over head_dim in chunks of four, each chunk reduced (p0+p1)+(p2+p3)
 * and added to the running dot, scalar tail (reference: src/cpu_ops.c:226-232,
 * :500-509). */
static inline float dot_chunks4(const float* a, const float* b, int n) {
    float dot = 0.0f;
    int d;
    for (d = 0; d <= n - 4; d += 4) {
        float p0 = a[d] * b[d], p1 = a[d + 1] * b[d + 1];
        float p2 = a[d + 2] * b[d + 2], p3 = a[d + 3] * b[d + 3];
        dot += (p0 + p1) + (p2 + p3);
    }
    for (; d < n; d++) dot += a[d] * b[d];
    return dot;
}

/* Softmax over scores[0,n) in place: max from -1e30, expf, sequential sum,
 * multiply by 1/sum (reference: src/cpu_ops.c:235-247). */
static void softmax_ref(float* sc, int n, float max_score) {
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        sc[i] = expf(sc[i] - max_score);
        sum += sc[i];
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) sc[i] *= inv;
}

/* Reference: src/cpu_ops.c:202-264.  Cache rows are [pos][kv_head][head_dim]. */
void orc_attention(float* out, const float* q, const float* kc, const float* vc,
                   int nq, int nkv, int hd, int L) {
    float scale = 1.0f / sqrtf((float)hd);
    int groups = nq / nkv;
    int stride = nkv * hd;
    float* sc = (float*)malloc(sizeof(float) * (L > 0 ? L : 1));
    for (int h = 0; h < nq; h++) {
        int kvh = h / groups;
        const float* qh = q + (size_t)h * hd;
        float mx = -1e30f;
        for (int s = 0; s < L; s++) {
            sc[s] = dot_chunks4(qh, kc + (size_t)s * stride + (size_t)kvh * hd, hd) * scale;
            if (sc[s] > mx) mx = sc[s];
        }
        softmax_ref(sc, L, mx);
        float* oh = out + (size_t)h * hd;
        for (int d = 0; d < hd; d++) oh[d] = 0.0f;
        for (int s = 0; s < L; s++) {
            const float* vs = vc + (size_t)s * stride + (size_t)kvh * hd;
            float p = sc[s];
            for (int d = 0; d < hd; d++) oh[d] = oh[d] + vs[d] * p;
        }
    }
    free(sc);
}

/* Reference: src/cpu_ops.c:459-571.  Scores over cache[0,S) then batch[0,t]. */
void orc_attention_batch_causal(float* out, const float* qb, const float* kb, const float* vb,
                                const float* kc, const float* vc, int M, int nq, int nkv,
                                int hd, int S) {
    float scale = 1.0f / sqrtf((float)hd);
    int groups = nq / nkv;
    int kvs = nkv * hd;
    int qs = nq * hd;
    float* sc = (float*)malloc(sizeof(float) * (size_t)(S + M));
    for (int t = 0; t < M; t++) {
        int L = S + t + 1;
        for (int h = 0; h < nq; h++) {
            int kvh = h / groups;
            const float* qh = qb + (size_t)t * qs + (size_t)h * hd;
            float mx = -1e30f;
            for (int s = 0; s < S; s++) {
                sc[s] = dot_chunks4(qh, kc + (size_t)s * kvs + (size_t)kvh * hd, hd) * scale;
                if (sc[s] > mx) mx = sc[s];
            }
            for (int b = 0; b <= t; b++) {
                sc[S + b] = dot_chunks4(qh, kb + (size_t)b * kvs + (size_t)kvh * hd, hd) * scale;
                if (sc[S + b] > mx) mx = sc[S + b];
            }
            softmax_ref(sc, L, mx);
            float* oh = out + (size_t)t * qs + (size_t)h * hd;
            for (int d = 0; d < hd; d++) oh[d] = 0.0f;
            for (int s = 0; s < S; s++) {
                const float* vs = vc + (size_t)s * kvs + (size_t)kvh * hd;
                for (int d = 0; d < hd; d++) oh[d] = oh[d] + vs[d] * sc[s];
            }
            for (int b = 0; b <= t; b++) {
                const float* vs = vb + (size_t)b * kvs + (size_t)kvh * hd;
                for (int d = 0; d < hd; d++) oh[d] = oh[d] + vs[d] * sc[S + b];
            }
        }
    }
    free(sc);
}

/* Reference: src/cpu_ops.c:296-319.  Blocks of four use g*(1/(1+expf(-g)))*u,
 * the tail uses (g/(1+expf(-g)))*u.  out may alias gate. */
void orc_silu_mul(float* out, const float* g, const float* u, int dim) {
    int blk = dim - dim % 4;
    for (int i = 0; i < blk; i++) {
        float sig = 1.0f / (1.0f + expf(-g[i]));
        out[i] = (g[i] * sig) * u[i];
    }
    for (int i = blk; i < dim; i++) out[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

/* Reference: src/cpu_ops.c:350-359. */
void orc_vec_add(float* dst, const float* src, int n) {
    for (int i = 0; i < n; i++) dst[i] = dst[i] + src[i];
}

/* Reference: src/cpu_ops.c:575-586.  First index of the maximum. */
int orc_argmax(const float* x, int n) {
    float mv = x[0];
    int mi = 0;
    for (int i = 1; i < n; i++) {
        if (x[i] > mv) { mv = x[i]; mi = i; }
    }
    return mi;
}

/* Sampling.  Reference: src/cpu_ops.c:593-648 (top_k_sample_f32), with the
 * caller's uniform u in [0,1] in place of rand() / RAND_MAX so that a draw is
 * reproducible.  Steps the reference does not define (it declares
 * repeat_penalty in include/matmul_decoder.h:395-397 and applies it nowhere;
 * its top_p_sample_f32, src/cpu_ops.c:650-665, returns the argmax) follow the
 * device sampler's definitions:
 *   - penalty p != 1: each distinct listed token's logit l -> l > 0 ? l / p : l * p;
 *   - top_p < 1: keep the shortest prefix of the sorted candidates whose
 *     running sum of e_j reaches top_p * sum, and draw from it.
 * x is modified (penalty, temperature).  top_idx/top_val (k each, may be
 * NULL) receive the candidates; *kept the prefix length.  Returns the token. */
int orc_sample_topk(float* x, int vocab_size, const int* rep, int n_rep, float penalty, int k,
                    float temperature, float top_p, float u, int* top_idx, float* top_val, int* kept) {
    if (penalty != 1.0f) {
        for (int i = 0; i < n_rep; i++) {
            int seen = 0;
            for (int j = 0; j < i && !seen; j++) seen = rep[j] == rep[i];
            if (seen) continue;
            const float l = x[rep[i]];
            x[rep[i]] = l > 0.0f ? l / penalty : l * penalty;
        }
    }
    /* src/cpu_ops.c:597-601 */
    if (temperature != 1.0f)
        for (int i = 0; i < vocab_size; i++) x[i] /= temperature;
    /* src/cpu_ops.c:604-624: insertion into a descending list of k */
    int* idx = (int*)malloc((size_t)k * sizeof(int));
    float* val = (float*)malloc((size_t)k * sizeof(float));
    for (int i = 0; i < k; i++) {
        val[i] = -1e30f;
        idx[i] = 0;
    }
    for (int i = 0; i < vocab_size; i++) {
        if (x[i] > val[k - 1]) {
            int j = k - 1;
            while (j > 0 && x[i] > val[j - 1]) {
                val[j] = val[j - 1];
                idx[j] = idx[j - 1];
                j--;
            }
            val[j] = x[i];
            idx[j] = i;
        }
    }
    if (top_idx)
        for (int i = 0; i < k; i++) top_idx[i] = idx[i];
    if (top_val)
        for (int i = 0; i < k; i++) top_val[i] = val[i];
    /* src/cpu_ops.c:626-632: softmax over the k, summed in order */
    const float max_val = val[0];
    float sum = 0.0f;
    for (int i = 0; i < k; i++) {
        val[i] = expf(val[i] - max_val);
        sum += val[i];
    }
    int m = k;
    if (top_p < 1.0f) {
        const float lim = top_p * sum;
        float run = 0.0f;
        for (int i = 0; i < k; i++) {
            run += val[i];
            if (run >= lim) {
                m = i + 1;
                break;
            }
        }
        sum = run;
    }
    if (kept) *kept = m;
    /* src/cpu_ops.c:634-646 */
    const float r = u * sum;
    float cumsum = 0.0f;
    int result = idx[m - 1];
    for (int i = 0; i < m; i++) {
        cumsum += val[i];
        if (r < cumsum) {
            result = idx[i];
            break;
        }
    }
    free(idx);
    free(val);
    return result;
}

/* ------------------------------------------------------------------------ */
/* Projections                                                               */
/* ------------------------------------------------------------------------ */

/* Accumulation order of the projections.  The reference runs them on the
 * NPU, whose fp32 accumulation order is not specified (src/matmul_decoder.c
 * only sees the results), so the oracle defines order 0: increasing k.
 * Orders 1 and 2 are equally valid ones, used only to measure how much valid
 * orders disagree after many layers: k mod 4 (order 1) or k mod 16 (order 2)
 * in separate sums, each in increasing k, combined as a pairwise tree
 * ((s0+s1)+(s2+s3) for four; the same levels for sixteen, the shape of a
 * lane-parallel dot product reduced across lanes). */
static int g_accum_order = 0;
void orc_set_accum_order(int order) { g_accum_order = order >= 0 && order <= 2 ? order : 0; }

static int accum_sets(void) { return g_accum_order == 1 ? 4 : (g_accum_order == 2 ? 16 : 1); }

/* y[m][n] += xk * wrow[n] into the accumulator set of k (k mod the set count). */
static void accum_row(float* acc, const float* wrow, float xk, int k, size_t MN_stride, int N) {
    float* a = acc + (size_t)(k & (accum_sets() - 1)) * MN_stride;
    for (int n = 0; n < N; n++) a[n] = a[n] + xk * wrow[n];
}

static float* accum_alloc(size_t MN) { return (float*)calloc((size_t)accum_sets() * MN, sizeof(float)); }

/* The sets combined pairwise: (s0+s1), (s2+s3), ... then the pairs of those. */
static void accum_finish(float* y, float* acc, size_t MN) {
    for (int w = accum_sets(); w > 1; w /= 2)
        for (int j = 0; j < w / 2; j++)
            for (size_t i = 0; i < MN; i++) acc[(size_t)j * MN + i] = acc[(size_t)(2 * j) * MN + i] + acc[(size_t)(2 * j + 1) * MN + i];
    memcpy(y, acc, MN * sizeof(float));
}

/* Reference: src/matmul_decoder.c:382-445 (type 1) and :1841-1899 (batch).
 * fp32 input rounded to fp16, products exact in fp32, fp32 accumulation in
 * increasing k. */
void orc_matmul_f16(float* y, const float* x, const uint16_t* w, int M, int K, int N) {
    if (g_accum_order != 0) {
        const size_t MN = (size_t)M * N;
        float* acc = accum_alloc(MN);
        float* wrow = (float*)malloc(sizeof(float) * (size_t)N);
        for (int k = 0; k < K; k++) {
            for (int n = 0; n < N; n++) wrow[n] = f16_widen(w[(size_t)k * N + n]);
            for (int m = 0; m < M; m++)
                accum_row(acc + (size_t)m * N, wrow,
                          orc_f16_to_f32(orc_f32_to_f16(x[(size_t)m * K + k])), k, MN, N);
        }
        accum_finish(y, acc, MN);
        free(acc);
        free(wrow);
        return;
    }
    float* wrow = (float*)malloc(sizeof(float) * (size_t)N);
    for (int m = 0; m < M; m++) {
        float* ym = y + (size_t)m * N;
        for (int n = 0; n < N; n++) ym[n] = 0.0f;
    }
    for (int k = 0; k < K; k++) {
        const uint16_t* wk = w + (size_t)k * N;
        for (int n = 0; n < N; n++) wrow[n] = f16_widen(wk[n]);
        for (int m = 0; m < M; m++) {
            float xk = orc_f16_to_f32(orc_f32_to_f16(x[(size_t)m * K + k]));
            float* ym = y + (size_t)m * N;
            for (int n = 0; n < N; n++) ym[n] = ym[n] + xk * wrow[n];
        }
    }
    free(wrow);
}

/* Reference: src/matmul_decoder.c:406-420 (type 5 plus the scale epilogue). */
void orc_matmul_i8(float* y, const float* x, const int8_t* q, const float* scale,
                   int M, int K, int N) {
    float* wrow = (float*)malloc(sizeof(float) * (size_t)N);
    const size_t MN = (size_t)M * N;
    float* acc = accum_alloc(MN);
    for (int k = 0; k < K; k++) {
        const int8_t* qk = q + (size_t)k * N;
        for (int n = 0; n < N; n++) wrow[n] = (float)qk[n];
        for (int m = 0; m < M; m++)
            accum_row(acc + (size_t)m * N, wrow, orc_f16_to_f32(orc_f32_to_f16(x[(size_t)m * K + k])),
                      k, MN, N);
    }
    accum_finish(y, acc, MN);
    free(acc);
    if (scale)
        for (int m = 0; m < M; m++)
            for (int n = 0; n < N; n++) y[(size_t)m * N + n] = y[(size_t)m * N + n] * scale[n];
    free(wrow);
}

void orc_matmul_i4(float* y, const float* x, const uint8_t* q, const float* scale,
                   int M, int K, int N) {
    float* wrow = (float*)malloc(sizeof(float) * (size_t)N);
    const size_t MN = (size_t)M * N;
    float* acc = accum_alloc(MN);
    for (int k = 0; k < K; k++) {
        const uint8_t* qk = q + (size_t)k * (N / 2);
        for (int j = 0; j < N / 2; j++) {
            /* sign-extend each nibble: column 2j low, 2j+1 high */
            wrow[2 * j] = (float)((int8_t)(uint8_t)(qk[j] << 4) >> 4);
            wrow[2 * j + 1] = (float)((int8_t)qk[j] >> 4);
        }
        for (int m = 0; m < M; m++)
            accum_row(acc + (size_t)m * N, wrow, orc_f16_to_f32(orc_f32_to_f16(x[(size_t)m * K + k])),
                      k, MN, N);
    }
    accum_finish(y, acc, MN);
    free(acc);
    if (scale)
        for (int m = 0; m < M; m++)
            for (int n = 0; n < N; n++) y[(size_t)m * N + n] = y[(size_t)m * N + n] * scale[n];
    free(wrow);
}

/* Reference: src/matmul_decoder.c:572-616.  Four fused lane accumulators
 * per row over steps of four, reduced (l0+l1)+(l2+l3), scalar tail. */
void orc_gemv_rows_f16(float* out, const float* x, const uint16_t* w, int N, int K) {
    for (int v = 0; v < N; v++) {
        const uint16_t* wr = w + (size_t)v * K;
        float l[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        int h;
        for (h = 0; h <= K - 4; h += 4)
            for (int j = 0; j < 4; j++) l[j] = fmaf(x[h + j], orc_f16_to_f32(wr[h + j]), l[j]);
        float s = (l[0] + l[1]) + (l[2] + l[3]);
        for (; h < K; h++) s += x[h] * orc_f16_to_f32(wr[h]);
        out[v] = s;
    }
}

/* Reference: src/matmul_decoder.c:511-566. */
void orc_gemv_rows_f32(float* out, const float* x, const float* w, int N, int K) {
    for (int v = 0; v < N; v++) {
        const float* wr = w + (size_t)v * K;
        float l[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        int h;
        for (h = 0; h <= K - 4; h += 4)
            for (int j = 0; j < 4; j++) l[j] = fmaf(x[h + j], wr[h + j], l[j]);
        float s = (l[0] + l[1]) + (l[2] + l[3]);
        for (; h < K; h++) s += x[h] * wr[h];
        out[v] = s;
    }
}

/* Reference: src/matmul_decoder.c:1216-1244, per vocab entry (the tiling
 * only pads).  scale = max|v|/127, q = clamp((int)roundf(v * (127/max))). */
void orc_quantize_lm_head(int8_t* q, float* scales, const uint16_t* lm16, int V, int K) {
    for (int v = 0; v < V; v++) {
        const uint16_t* row = lm16 + (size_t)v * K;
        float col_max = 0.0f;
        for (int k = 0; k < K; k++) {
            float a = fabsf(orc_f16_to_f32(row[k]));
            if (a > col_max) col_max = a;
        }
        scales[v] = col_max / 127.0f;
        float inv = (col_max > 0) ? 127.0f / col_max : 0;
        for (int k = 0; k < K; k++) {
            int qi = (int)roundf(orc_f16_to_f32(row[k]) * inv);
            if (qi < -128) qi = -128;
            if (qi > 127) qi = 127;
            q[(size_t)v * K + k] = (int8_t)qi;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* The decoder                                                               */
/* ------------------------------------------------------------------------ */

typedef struct {
    int kind;                /* 0 fp16, 1 int8, 2 int4 */
    int K, N;
    void* w;
    float* scale;            /* NULL = unscaled */
} orc_proj;

typedef struct {
    orc_proj p[7];           /* q k v o gate up down */
    float *in_norm, *post_norm, *q_norm, *k_norm;
} orc_layer;

struct orc_model {
    orc_config c;
    int max_seq, kv_fp16, seq_len;
    float* emb;
    float* lm_f32;           /* single head, fp32 (may alias emb) */
    uint16_t* lm_f16;
    int8_t* lm_q;            /* [V][K] as quantised */
    int8_t* lm_qt;           /* [K][V]: the NPU B-matrix orientation */
    float* lm_s;
    float** lm_heads;        /* multi-head */
    orc_layer* layers;
    float* final_norm;
    int final_norm_owned;
    float *kc, *vc;          /* [layer][max_seq][kv_dim] */
    float *cos_t, *sin_t;
    /* scratch */
    float *hidden, *residual, *normed, *q, *k, *v, *attn, *gate, *up, *down, *logits;
};

static void* read_file(const char* path, size_t bytes) {
    FILE* f = fopen(path, "rb");
    if (!f) return NULL;
    void* p = malloc(bytes ? bytes : 1);
    size_t got = p ? fread(p, 1, bytes, f) : 0;
    fclose(f);
    if (!p || got != bytes) { free(p); return NULL; }
    return p;
}

static float* read_f32_alt(const char* dir, const char* const* names, size_t n) {
    char path[1024];
    for (int i = 0; names[i]; i++) {
        snprintf(path, sizeof path, "%s/%s", dir, names[i]);
        float* p = (float*)read_file(path, n * sizeof(float));
        if (p) return p;
    }
    return NULL;
}

/* Reference: src/matmul_decoder.c:698-826 (file names and fallbacks). */
static int load_layer(orc_layer* L, const char* dir, const orc_config* c, int quant) {
    static const char* in_n[] = {"input_norm.bin", "input_norm_weight.bin", NULL};
    static const char* post_n[] = {"post_attn_norm.bin", "post_norm.bin",
                                   "post_attn_norm_weight.bin", NULL};
    static const char* qn_n[] = {"q_norm.bin", "q_norm_weight.bin", NULL};
    static const char* kn_n[] = {"k_norm.bin", "k_norm_weight.bin", NULL};
    static const char* names[7] = {"q_proj", "k_proj", "v_proj", "o_proj",
                                   "gate_proj", "up_proj", "down_proj"};
    int d = c->hidden_dim, qd = c->num_q_heads * c->head_dim, kvd = c->num_kv_heads * c->head_dim;
    int Ks[7] = {d, d, d, qd, d, d, c->ffn_dim};
    int Ns[7] = {qd, kvd, kvd, d, c->ffn_dim, c->ffn_dim, d};
    L->in_norm = read_f32_alt(dir, in_n, (size_t)d);
    L->post_norm = read_f32_alt(dir, post_n, (size_t)d);
    if (!L->in_norm || !L->post_norm) return -1;
    if (c->has_qk_norm) {
        L->q_norm = read_f32_alt(dir, qn_n, (size_t)c->head_dim);
        L->k_norm = read_f32_alt(dir, kn_n, (size_t)c->head_dim);
        if (!L->q_norm || !L->k_norm) return -1;
    }
    char path[1024];
    for (int i = 0; i < 7; i++) {
        orc_proj* p = &L->p[i];
        p->K = Ks[i];
        p->N = Ns[i];
        size_t kn = (size_t)p->K * p->N;
        if (quant != 0) {
            snprintf(path, sizeof path, "%s/%s_weight.bin", dir, names[i]);
            p->w = read_file(path, quant == 2 ? kn / 2 : kn);
            if (p->w) {
                p->kind = quant;
                snprintf(path, sizeof path, "%s/%s_scales.bin", dir, names[i]);
                p->scale = (float*)read_file(path, (size_t)p->N * sizeof(float));
                continue;
            }
        }
        snprintf(path, sizeof path, "%s/%s.bin", dir, names[i]);
        p->w = read_file(path, kn * 2);
        p->kind = 0;
        if (!p->w) p->w = calloc(kn, 2);          /* missing projection: zeros */
    }
    return 0;
}

static void proj_run(const orc_proj* p, const float* x, float* y, int M) {
    if (p->kind == 0) orc_matmul_f16(y, x, (const uint16_t*)p->w, M, p->K, p->N);
    else if (p->kind == 1) orc_matmul_i8(y, x, (const int8_t*)p->w, p->scale, M, p->K, p->N);
    else orc_matmul_i4(y, x, (const uint8_t*)p->w, p->scale, M, p->K, p->N);
}

orc_model* orc_model_open(const char* dir, const orc_config* c, int quant, int max_seq,
                          int kv_fp16) {
    orc_model* m = (orc_model*)calloc(1, sizeof *m);
    if (!m) return NULL;
    m->c = *c;
    m->max_seq = max_seq;
    m->kv_fp16 = kv_fp16;
    int d = c->hidden_dim, V = c->vocab_size, hd = c->head_dim;
    int qd = c->num_q_heads * hd, kvd = c->num_kv_heads * hd;
    char path[1024];
    snprintf(path, sizeof path, "%s/embeddings.bin", dir);
    m->emb = (float*)read_file(path, (size_t)V * d * 4);
    if (!m->emb) goto fail;
    if (c->num_lm_heads > 1) {
        int lv = c->lm_head_vocab_size > 0 ? c->lm_head_vocab_size : V;
        m->lm_heads = (float**)calloc((size_t)c->num_lm_heads, sizeof(float*));
        for (int i = 0; i < c->num_lm_heads; i++) {
            snprintf(path, sizeof path, "%s/lm_head_%02d.bin", dir, i);
            m->lm_heads[i] = (float*)read_file(path, (size_t)lv * d * 4);
            if (!m->lm_heads[i]) goto fail;
        }
    } else {
        snprintf(path, sizeof path, "%s/lm_head.bin", dir);
        m->lm_f32 = (float*)read_file(path, (size_t)V * d * 4);
        if (!m->lm_f32 && !c->tie_word_embeddings) goto fail;
        if (!m->lm_f32) m->lm_f32 = m->emb;
        m->lm_f16 = (uint16_t*)malloc((size_t)V * d * 2);
        orc_vec_f32_to_f16(m->lm_f16, m->lm_f32, (size_t)V * d);
        if (!c->disable_npu_lm_head) {
            m->lm_q = (int8_t*)malloc((size_t)V * d);
            m->lm_s = (float*)malloc((size_t)V * 4);
            orc_quantize_lm_head(m->lm_q, m->lm_s, m->lm_f16, V, d);
            m->lm_qt = (int8_t*)malloc((size_t)V * d);
            if (!m->lm_qt) goto fail;
            for (int v = 0; v < V; v++)
                for (int k = 0; k < d; k++) m->lm_qt[(size_t)k * V + v] = m->lm_q[(size_t)v * d + k];
        }
    }
    m->layers = (orc_layer*)calloc((size_t)c->num_layers, sizeof(orc_layer));
    for (int l = 0; l < c->num_layers; l++) {
        struct stat st;
        snprintf(path, sizeof path, "%s/layers/layer_%02d", dir, l);
        if (!(stat(path, &st) == 0 && S_ISDIR(st.st_mode)))
            snprintf(path, sizeof path, "%s/layer_%02d", dir, l);
        if (load_layer(&m->layers[l], path, c, quant) != 0) goto fail;
    }
    {
        static const char* fn[] = {"final_norm.bin", "model_norm.bin", NULL};
        m->final_norm = read_f32_alt(dir, fn, (size_t)d);
        m->final_norm_owned = m->final_norm != NULL;
        if (!m->final_norm) m->final_norm = m->layers[c->num_layers - 1].post_norm;
    }
    m->kc = (float*)calloc((size_t)c->num_layers * max_seq * kvd, 4);
    m->vc = (float*)calloc((size_t)c->num_layers * max_seq * kvd, 4);
    m->cos_t = (float*)malloc((size_t)max_seq * (hd / 2) * 4);
    m->sin_t = (float*)malloc((size_t)max_seq * (hd / 2) * 4);
    if (!m->kc || !m->vc || !m->cos_t || !m->sin_t) goto fail;
    orc_rope_tables(m->cos_t, m->sin_t, max_seq, hd, c->rope_theta);
    int lv = V;
    if (c->num_lm_heads > 1 && c->lm_head_vocab_size > lv) lv = c->lm_head_vocab_size;
    int mm = c->max_batch_prefill > 0 ? c->max_batch_prefill : 64;
    m->hidden = (float*)malloc((size_t)mm * d * 4);
    m->residual = (float*)malloc((size_t)mm * d * 4);
    m->normed = (float*)malloc((size_t)mm * d * 4);
    m->q = (float*)malloc((size_t)mm * qd * 4);
    m->k = (float*)malloc((size_t)mm * kvd * 4);
    m->v = (float*)malloc((size_t)mm * kvd * 4);
    m->attn = (float*)malloc((size_t)mm * qd * 4);
    m->gate = (float*)malloc((size_t)mm * c->ffn_dim * 4);
    m->up = (float*)malloc((size_t)mm * c->ffn_dim * 4);
    m->down = (float*)malloc((size_t)mm * d * 4);
    m->logits = (float*)malloc((size_t)lv * 4);
    return m;
fail:
    orc_model_close(m);
    return NULL;
}

void orc_model_close(orc_model* m) {
    if (!m) return;
    if (m->layers) {
        for (int l = 0; l < m->c.num_layers; l++) {
            orc_layer* L = &m->layers[l];
            for (int i = 0; i < 7; i++) { free(L->p[i].w); free(L->p[i].scale); }
            free(L->in_norm); free(L->post_norm); free(L->q_norm); free(L->k_norm);
        }
    }
    if (m->final_norm_owned) free(m->final_norm);
    free(m->layers);
    if (m->lm_heads) {
        for (int i = 0; i < m->c.num_lm_heads; i++) free(m->lm_heads[i]);
        free(m->lm_heads);
    }
    if (m->lm_f32 != m->emb) free(m->lm_f32);
    free(m->emb); free(m->lm_f16); free(m->lm_q); free(m->lm_qt); free(m->lm_s);
    free(m->kc); free(m->vc); free(m->cos_t); free(m->sin_t);
    free(m->hidden); free(m->residual); free(m->normed); free(m->q); free(m->k); free(m->v);
    free(m->attn); free(m->gate); free(m->up); free(m->down); free(m->logits);
    free(m);
}

static void round_to_f16(float* x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = orc_f16_to_f32(orc_f32_to_f16(x[i]));
}

/* The layer stack for one token (reference: src/matmul_decoder.c:1464-1546). */
static void layers_one(orc_model* m) {
    const orc_config* c = &m->c;
    int d = c->hidden_dim, hd = c->head_dim, nq = c->num_q_heads, nkv = c->num_kv_heads;
    int kvd = nkv * hd, pos = m->seq_len;
    for (int l = 0; l < c->num_layers; l++) {
        orc_layer* L = &m->layers[l];
        float* kc = m->kc + (size_t)l * m->max_seq * kvd;
        float* vc = m->vc + (size_t)l * m->max_seq * kvd;
        memcpy(m->residual, m->hidden, (size_t)d * 4);
        orc_rms_norm(m->normed, m->hidden, L->in_norm, d, c->rms_eps);
        proj_run(&L->p[0], m->normed, m->q, 1);
        proj_run(&L->p[1], m->normed, m->k, 1);
        proj_run(&L->p[2], m->normed, m->v, 1);
        if (c->has_qk_norm && L->q_norm && L->k_norm) {
            for (int h = 0; h < nq; h++)
                orc_rms_norm(m->q + (size_t)h * hd, m->q + (size_t)h * hd, L->q_norm, hd, c->rms_eps);
            for (int h = 0; h < nkv; h++)
                orc_rms_norm(m->k + (size_t)h * hd, m->k + (size_t)h * hd, L->k_norm, hd, c->rms_eps);
        }
        const float* cr = m->cos_t + (size_t)pos * (hd / 2);
        const float* sr = m->sin_t + (size_t)pos * (hd / 2);
        orc_apply_rope(m->q, cr, sr, nq, hd, c->rope_style);
        orc_apply_rope(m->k, cr, sr, nkv, hd, c->rope_style);
        if (m->kv_fp16) { round_to_f16(m->k, kvd); round_to_f16(m->v, kvd); }
        memcpy(kc + (size_t)pos * kvd, m->k, (size_t)kvd * 4);
        memcpy(vc + (size_t)pos * kvd, m->v, (size_t)kvd * 4);
        orc_attention(m->attn, m->q, kc, vc, nq, nkv, hd, pos + 1);
        proj_run(&L->p[3], m->attn, m->hidden, 1);
        orc_vec_add(m->hidden, m->residual, d);
        orc_rms_norm(m->normed, m->hidden, L->post_norm, d, c->rms_eps);
        proj_run(&L->p[4], m->normed, m->gate, 1);
        proj_run(&L->p[5], m->normed, m->up, 1);
        orc_silu_mul(m->gate, m->gate, m->up, c->ffn_dim);
        proj_run(&L->p[6], m->gate, m->down, 1);
        orc_vec_add(m->hidden, m->down, d);
    }
}

static int load_input(orc_model* m, int token_id, const float* embedding) {
    int d = m->c.hidden_dim;
    if (embedding) {
        memcpy(m->hidden, embedding, (size_t)d * 4);
    } else {
        if (token_id < 0 || token_id >= m->c.vocab_size) return -1;
        memcpy(m->hidden, m->emb + (size_t)token_id * d, (size_t)d * 4);
    }
    if (m->seq_len >= m->max_seq) return -1;
    return 0;
}

/* Reference: src/matmul_decoder.c:1430-1634. */
int orc_model_step(orc_model* m, int token_id, const float* embedding, float* logits) {
    const orc_config* c = &m->c;
    if (load_input(m, token_id, embedding) != 0) return -1;
    layers_one(m);
    if (!logits) { m->seq_len++; return 0; }
    int d = c->hidden_dim, V = c->vocab_size;
    orc_rms_norm(m->normed, m->hidden, m->final_norm, d, c->rms_eps);
    if (m->lm_q) {
        /* NPU lm_head tiles (reference: src/matmul_decoder.c:1569-1605):
         * logits[v] = scale[v] * sum_k fp16(normed_k) * q[k][v] */
        orc_matmul_i8(m->logits, m->normed, m->lm_qt, m->lm_s, 1, d, V);
    } else {
        orc_gemv_rows_f16(m->logits, m->normed, m->lm_f16, V, d);
    }
    m->seq_len++;
    memcpy(logits, m->logits, (size_t)V * 4);
    return orc_argmax(m->logits, V);
}

/* Reference: src/matmul_decoder.c:1636-1742. */
int orc_model_step_head(orc_model* m, int token_id, const float* embedding, int head,
                        float* logits) {
    const orc_config* c = &m->c;
    if (c->num_lm_heads <= 1) return orc_model_step(m, token_id, embedding, logits);
    if (head < 0 || head >= c->num_lm_heads || !m->lm_heads) return -1;
    int lv = c->lm_head_vocab_size > 0 ? c->lm_head_vocab_size : c->vocab_size;
    if (load_input(m, token_id, embedding) != 0) return -1;
    layers_one(m);
    orc_rms_norm(m->normed, m->hidden, m->final_norm, c->hidden_dim, c->rms_eps);
    orc_gemv_rows_f32(m->logits, m->normed, m->lm_heads[head], lv, c->hidden_dim);
    m->seq_len++;
    if (logits) memcpy(logits, m->logits, (size_t)lv * 4);
    return orc_argmax(m->logits, lv);
}

/* Reference: src/matmul_decoder.c:1901-2065. */
int orc_model_prefill_batch(orc_model* m, const float* emb, int M) {
    const orc_config* c = &m->c;
    if (!emb || M <= 0) return -1;
    int d = c->hidden_dim, hd = c->head_dim, nq = c->num_q_heads, nkv = c->num_kv_heads;
    int qd = nq * hd, kvd = nkv * hd, S = m->seq_len;
    if (S + M > m->max_seq) return -1;
    int mm = c->max_batch_prefill > 0 ? c->max_batch_prefill : 64;
    if (M > mm) {
        for (int off = 0; off < M; off += mm) {
            int ch = M - off < mm ? M - off : mm;
            int r = orc_model_prefill_batch(m, emb + (size_t)off * d, ch);
            if (r != 0) return r;
        }
        return 0;
    }
    memcpy(m->hidden, emb, (size_t)M * d * 4);
    for (int l = 0; l < c->num_layers; l++) {
        orc_layer* L = &m->layers[l];
        float* kc = m->kc + (size_t)l * m->max_seq * kvd;
        float* vc = m->vc + (size_t)l * m->max_seq * kvd;
        memcpy(m->residual, m->hidden, (size_t)M * d * 4);
        for (int t = 0; t < M; t++)
            orc_rms_norm(m->normed + (size_t)t * d, m->hidden + (size_t)t * d, L->in_norm, d, c->rms_eps);
        proj_run(&L->p[0], m->normed, m->q, M);
        proj_run(&L->p[1], m->normed, m->k, M);
        proj_run(&L->p[2], m->normed, m->v, M);
        if (c->has_qk_norm && L->q_norm && L->k_norm) {
            for (int t = 0; t < M; t++) {
                for (int h = 0; h < nq; h++) {
                    float* p = m->q + (size_t)t * qd + (size_t)h * hd;
                    orc_rms_norm(p, p, L->q_norm, hd, c->rms_eps);
                }
                for (int h = 0; h < nkv; h++) {
                    float* p = m->k + (size_t)t * kvd + (size_t)h * hd;
                    orc_rms_norm(p, p, L->k_norm, hd, c->rms_eps);
                }
            }
        }
        orc_apply_rope_batch(m->q, M, S, nq, hd, c->rope_theta, c->rope_style);
        orc_apply_rope_batch(m->k, M, S, nkv, hd, c->rope_theta, c->rope_style);
        if (m->kv_fp16) { round_to_f16(m->k, (size_t)M * kvd); round_to_f16(m->v, (size_t)M * kvd); }
        orc_attention_batch_causal(m->attn, m->q, m->k, m->v, kc, vc, M, nq, nkv, hd, S);
        for (int t = 0; t < M; t++) {
            memcpy(kc + (size_t)(S + t) * kvd, m->k + (size_t)t * kvd, (size_t)kvd * 4);
            memcpy(vc + (size_t)(S + t) * kvd, m->v + (size_t)t * kvd, (size_t)kvd * 4);
        }
        proj_run(&L->p[3], m->attn, m->hidden, M);
        for (int t = 0; t < M; t++) orc_vec_add(m->hidden + (size_t)t * d, m->residual + (size_t)t * d, d);
        for (int t = 0; t < M; t++)
            orc_rms_norm(m->normed + (size_t)t * d, m->hidden + (size_t)t * d, L->post_norm, d, c->rms_eps);
        proj_run(&L->p[4], m->normed, m->gate, M);
        proj_run(&L->p[5], m->normed, m->up, M);
        for (int t = 0; t < M; t++)
            orc_silu_mul(m->gate + (size_t)t * c->ffn_dim, m->gate + (size_t)t * c->ffn_dim,
                         m->up + (size_t)t * c->ffn_dim, c->ffn_dim);
        proj_run(&L->p[6], m->gate, m->down, M);
        for (int t = 0; t < M; t++) orc_vec_add(m->hidden + (size_t)t * d, m->down + (size_t)t * d, d);
    }
    /* keep the last row's normed final state for lm_head checks */
    memmove(m->hidden, m->hidden + (size_t)(M - 1) * d, (size_t)d * 4);
    orc_rms_norm(m->normed, m->hidden, m->final_norm, d, c->rms_eps);
    m->seq_len += M;
    return 0;
}

int orc_model_seq_len(const orc_model* m) { return m->seq_len; }
void orc_model_set_seq_len(orc_model* m, int n) { m->seq_len = n; }

int orc_model_kv_fill_normal(orc_model* m, int n_pos, uint64_t seed) {
    if (n_pos < 0 || n_pos > m->max_seq) return -1;
    int kvd = m->c.num_kv_heads * m->c.head_dim;
    size_t n = (size_t)n_pos * kvd;
    char name[64];
    for (int l = 0; l < m->c.num_layers; l++) {
        for (int which = 0; which < 2; which++) {
            float* dst = (which ? m->vc : m->kc) + (size_t)l * m->max_seq * kvd;
            snprintf(name, sizeof name, which ? "kv/v/%02d" : "kv/k/%02d", l);
            orc_fill_normal_f32(dst, n, orc_seed_for(seed, name), 0.0, 1.0);
            if (m->kv_fp16) round_to_f16(dst, n);
        }
    }
    m->seq_len = n_pos;
    return 0;
}

int orc_model_kv_read(const orc_model* m, int layer, int pos0, int n, float* k, float* v) {
    if (layer < 0 || layer >= m->c.num_layers || pos0 < 0 || n < 0 || pos0 + n > m->max_seq)
        return -1;
    int kvd = m->c.num_kv_heads * m->c.head_dim;
    size_t off = (size_t)layer * m->max_seq * kvd + (size_t)pos0 * kvd;
    memcpy(k, m->kc + off, (size_t)n * kvd * 4);
    memcpy(v, m->vc + off, (size_t)n * kvd * 4);
    return 0;
}

void orc_model_last_normed(const orc_model* m, float* out) {
    memcpy(out, m->normed, (size_t)m->c.hidden_dim * 4);
}

const int8_t* orc_model_lm_q(const orc_model* m) { return m->lm_q; }
const float* orc_model_lm_scales(const orc_model* m) { return m->lm_s; }
