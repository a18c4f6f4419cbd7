// mdx_decode.hip — M = 1 decode kernels for gfx950.
//
// Projections (reference: src/matmul_decoder.c:382-445, the NPU call sites
// K1/K2; CPU GEMVs :511-616) run as bandwidth-bound GEMVs over the W^T
// device layout: each wave owns RW weight rows, every lane streams 16-byte
// chunks of each row (so one wave load instruction reads 1 KiB contiguous),
// dequantises in registers, accumulates with v_dot2_f32_f16 and the wave
// reduces with lane shuffles.  The activation vector is built once per
// workgroup in LDS, fused with the RMSNorm that precedes it in the layer
// (reference: src/cpu_ops.c:18-55).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>

#include "mdx_common.h"
#include "mdx_device.h"

using namespace mdx;

namespace {

enum XMode { XM_NORM = 0, XM_F16 = 1, XM_F32 = 2 };
enum Epi { EP_STORE = 0, EP_ADD = 1, EP_SWIGLU = 2, EP_LOGITS = 3 };
// KF16/KI8/KI4: fp16 activations (the NPU input).  KF32X: fp32 rows with fp32
// activations, KF16X: fp16 rows with fp32 activations (the CPU GEMVs).
enum Kind { KF16 = 0, KI8 = 1, KI4 = 2, KF32X = 3, KF16X = 4 };

struct ArgPair {
    float v;
    int i;
};

struct GemvArgs {
    const uint8_t* w;
    const float* scale;
    int K, N;             // N weight rows
    int n_units;          // output units; unit u uses rows u (and u + n_units when unit_rows == 2)
    int unit_rows;
    int xmode;
    const float* xf32;
    const uint16_t* x16;
    const float* norm_w;
    float eps;
    int epi;
    float* out_f32;
    uint16_t* out_f16;
    ArgPair* partial;
};

template <int KIND> struct KindTraits;
template <> struct KindTraits<KF16> { static constexpr int E = 8; static constexpr bool XF32 = false; static constexpr int EB2 = 4; };
template <> struct KindTraits<KI8> { static constexpr int E = 16; static constexpr bool XF32 = false; static constexpr int EB2 = 2; };
template <> struct KindTraits<KI4> { static constexpr int E = 32; static constexpr bool XF32 = false; static constexpr int EB2 = 1; };
template <> struct KindTraits<KF32X> { static constexpr int E = 4; static constexpr bool XF32 = true; static constexpr int EB2 = 8; };
template <> struct KindTraits<KF16X> { static constexpr int E = 8; static constexpr bool XF32 = true; static constexpr int EB2 = 4; };
// EB2 = row bytes per element, times 2 (int4 rows hold half a byte per element).

template <int KIND>
__device__ __forceinline__ float chunk_dot(uint4 w, const uint4* xs, int j, float acc) {
    if constexpr (KIND == KF16) {
        return dot8_f16(w, xs[j], acc);
    } else if constexpr (KIND == KI8) {
        return dot16_i8(w, xs[2 * j], xs[2 * j + 1], acc);
    } else if constexpr (KIND == KI4) {
        acc = dot8_i4(w.x, xs[4 * j + 0], acc);
        acc = dot8_i4(w.y, xs[4 * j + 1], acc);
        acc = dot8_i4(w.z, xs[4 * j + 2], acc);
        acc = dot8_i4(w.w, xs[4 * j + 3], acc);
        return acc;
    } else if constexpr (KIND == KF32X) {
        const float4 x = reinterpret_cast<const float4*>(xs)[j];
        acc = fmaf(__uint_as_float(w.x), x.x, acc);
        acc = fmaf(__uint_as_float(w.y), x.y, acc);
        acc = fmaf(__uint_as_float(w.z), x.z, acc);
        acc = fmaf(__uint_as_float(w.w), x.w, acc);
        return acc;
    } else {  // KF16X
        const float4 x0 = reinterpret_cast<const float4*>(xs)[2 * j];
        const float4 x1 = reinterpret_cast<const float4*>(xs)[2 * j + 1];
        half2_t h;
        h = as_h2(w.x);
        acc = fmaf((float)h.x, x0.x, acc);
        acc = fmaf((float)h.y, x0.y, acc);
        h = as_h2(w.y);
        acc = fmaf((float)h.x, x0.z, acc);
        acc = fmaf((float)h.y, x0.w, acc);
        h = as_h2(w.z);
        acc = fmaf((float)h.x, x1.x, acc);
        acc = fmaf((float)h.y, x1.y, acc);
        h = as_h2(w.w);
        acc = fmaf((float)h.x, x1.z, acc);
        acc = fmaf((float)h.y, x1.w, acc);
        return acc;
    }
}

// Builds the activation vector in LDS: fp16 for the NPU-style kinds, fp32 for
// the CPU-GEMV kinds.  XM_NORM applies the reference RMSNorm first.
template <bool XF32>
__device__ __forceinline__ void build_x(const GemvArgs& a, void* xs_raw, float* red) {
    const int tid = threadIdx.x;
    const int K = a.K;
    float rms = 1.0f;
    if (a.xmode == XM_NORM) {
        float ss = 0.0f;
        for (int k = tid; k < K; k += blockDim.x) {
            float v = a.xf32[k];
            ss += v * v;
        }
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int wv = 0; wv < (int)(blockDim.x >> 6); wv++) tot += red[wv];
        rms = 1.0f / sqrtf(tot / (float)K + a.eps);
    }
    if constexpr (XF32) {
        float* xs = reinterpret_cast<float*>(xs_raw);
        for (int k = tid; k < K; k += blockDim.x) {
            float v;
            if (a.xmode == XM_NORM) v = (a.xf32[k] * rms) * a.norm_w[k];
            else if (a.xmode == XM_F16) v = f16_bits_to_f32(a.x16[k]);
            else v = a.xf32[k];
            xs[k] = v;
        }
    } else {
        uint16_t* xs = reinterpret_cast<uint16_t*>(xs_raw);
        for (int k = tid; k < K; k += blockDim.x) {
            uint16_t v;
            if (a.xmode == XM_NORM) v = f32_to_f16_bits((a.xf32[k] * rms) * a.norm_w[k]);
            else if (a.xmode == XM_F16) v = a.x16[k];
            else v = f32_to_f16_bits(a.xf32[k]);
            xs[k] = v;
        }
    }
    __syncthreads();
}

// The GEMV.  grid.x = ceil(n_units * unit_rows / (4 * RW)), block = 256.
template <int KIND, int RW, int U>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
    using T = KindTraits<KIND>;
    extern __shared__ uint4 xs[];
    __shared__ float red[4];
    __shared__ ArgPair amax[4];

    build_x<T::XF32>(a, xs, red);

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int nchunks = a.K / T::E;
    const size_t row_bytes = (size_t)a.K * T::EB2 / 2;
    const int ru = a.unit_rows;
    const int slot0 = (blockIdx.x * 4 + wave) * RW;   // first row slot of this wave

    int rows[RW];
    bool valid[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int slot = slot0 + r;
        const int unit = slot / ru, which = slot % ru;
        valid[r] = unit < a.n_units;
        rows[r] = unit + which * a.n_units;
    }

    float acc[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) acc[r] = 0.0f;

    for (int base = 0; base < nchunks; base += 64 * U) {
        uint4 wv[RW][U];
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const uint8_t* rp = a.w + (size_t)rows[r] * row_bytes;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int j = base + u * 64 + lane;
                if (valid[r] && j < nchunks)
                    wv[r][u] = reinterpret_cast<const uint4*>(rp)[j];
                else
                    wv[r][u] = make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int r = 0; r < RW; r++) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int j = base + u * 64 + lane;
                if (j < nchunks) acc[r] = chunk_dot<KIND>(wv[r][u], xs, j, acc[r]);
            }
        }
    }

    float y[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        y[r] = wave_sum(acc[r]);
        if (a.scale && valid[r]) y[r] = y[r] * a.scale[rows[r]];
    }

    if (a.epi == EP_STORE || a.epi == EP_ADD || a.epi == EP_LOGITS) {
#pragma unroll
        for (int r = 0; r < RW; r++) {
            if (valid[r] && lane == (r & 63)) {
                if (a.epi == EP_ADD) a.out_f32[rows[r]] = a.out_f32[rows[r]] + y[r];
                else a.out_f32[rows[r]] = y[r];
            }
        }
    } else if (a.epi == EP_SWIGLU) {
        // slots come in (gate, up) pairs: slot 2c is row unit, slot 2c+1 is row unit + F
#pragma unroll
        for (int r = 0; r + 1 < RW; r += 2) {
            if (valid[r] && lane == (r & 63)) {
                const int unit = rows[r];
                const float g = y[r], u = y[r + 1];
                float v;
                if (unit < (a.n_units & ~3)) v = silu_mul(g, u);
                else v = (g / (1.0f + expf(-g))) * u;     // reference tail formula
                a.out_f16[unit] = f32_to_f16_bits(v);
            }
        }
    }

    if (a.epi == EP_LOGITS) {
        ArgPair best = {-INFINITY, -1};
#pragma unroll
        for (int r = 0; r < RW; r++) {
            if (valid[r] && (y[r] > best.v || best.i < 0)) {
                if (!(y[r] != y[r])) { best.v = y[r]; best.i = rows[r]; }
            }
        }
        if (lane == 0) amax[wave] = best;
        __syncthreads();
        if (tid == 0) {
            ArgPair b = amax[0];
            for (int wv = 1; wv < 4; wv++) {
                const ArgPair c = amax[wv];
                if (c.i >= 0 && (b.i < 0 || c.v > b.v)) b = c;
            }
            a.partial[blockIdx.x] = b;
        }
    }
}

typedef void (*GemvKernel)(GemvArgs);

template <int KIND>
GemvKernel pick_kernel(int rw, int u) {
#define MDX_U_CASES(RW_)                                        \
    switch (u) {                                                \
        case 1: return k_gemv<KIND, RW_, 1>;                    \
        case 2: return k_gemv<KIND, RW_, 2>;                    \
        case 4: return k_gemv<KIND, RW_, 4>;                    \
        default: return k_gemv<KIND, RW_, 8>;                   \
    }
    switch (rw) {
        case 1: MDX_U_CASES(1)
        case 2: MDX_U_CASES(2)
        case 4: MDX_U_CASES(4)
        default: MDX_U_CASES(8)
    }
#undef MDX_U_CASES
}

GemvKernel pick(int kind, int rw, int u) {
    switch (kind) {
        case KF16: return pick_kernel<KF16>(rw, u);
        case KI8: return pick_kernel<KI8>(rw, u);
        case KI4: return pick_kernel<KI4>(rw, u);
        case KF32X: return pick_kernel<KF32X>(rw, u);
        default: return pick_kernel<KF16X>(rw, u);
    }
}

int elems_per_chunk(int kind) {
    switch (kind) {
        case KF16: return 8;
        case KI8: return 16;
        case KI4: return 32;
        case KF32X: return 4;
        default: return 8;
    }
}

int pow2_at_least(int v, int cap) {
    int p = 1;
    while (p < v && p < cap) p <<= 1;
    return p;
}

// rows_per_wave: how many weight rows one wave streams at once.
int launch_gemv(int kind, GemvArgs a, int rows_per_wave, void* stream) {
    const int E = elems_per_chunk(kind);
    if (a.K <= 0 || a.K % E != 0 || a.n_units <= 0) return -1;
    const int nchunks = a.K / E;
    const int rw = rows_per_wave;
    // at most 16 outstanding 16-byte loads per lane (64 VGPRs of weights)
    const int u = pow2_at_least((nchunks + 63) / 64, 16 / rw < 8 ? 16 / rw : 8);
    const long slots = (long)a.n_units * a.unit_rows;
    const long grid = (slots + 4L * rw - 1) / (4L * rw);
    const bool xf32 = kind == KF32X || kind == KF16X;
    const size_t lds = (size_t)a.K * (xf32 ? 4 : 2);
    if (lds > 64 * 1024) return -5;
    GemvKernel k = pick(kind, rw, u);
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(256), lds, (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int kind_from(const mdx_wdesc* w, int x_fp32_exact) {
    switch (w->kind) {
        case MDX_W_F16: return x_fp32_exact ? KF16X : KF16;
        case MDX_W_I8: return KI8;
        case MDX_W_I4: return KI4;
        default: return KF32X;
    }
}

// Rows per wave chosen so that a launch has enough waves in flight for HBM.
int rows_per_wave_for(int kind, int units_rows, int K) {
    (void)K;
    if (units_rows >= 65536) return 8;
    if (units_rows >= 4096) return 2;
    return 1;
}

__global__ void k_embed(const mdx_state* st, const float* table, const float* emb_in,
                        float* hidden, int d, int vocab) {
    const int mode = st->mode;
    int tok = st->token;
    if (tok < 0) tok = 0;
    if (tok >= vocab) tok = vocab - 1;
    const float* src = mode == 1 ? emb_in : table + (size_t)tok * d;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < d; i += gridDim.x * blockDim.x)
        hidden[i] = src[i];
}

// QK-norm + RoPE + KV append for one token (reference:
// src/matmul_decoder.c:1493-1516).  grid = nq + 2*nkv waves: q heads, k heads,
// then v heads.
__global__ __launch_bounds__(64) void k_qk_rope_append(
    const mdx_state* st, const float* qkv, const float* q_norm, const float* k_norm, float eps,
    const float* cos_t, const float* sin_t, int nq, int nkv, int hd, int style, float* q_out,
    uint16_t* k_cache, uint16_t* v_cache) {
    const int b = blockIdx.x, lane = threadIdx.x;
    const int pos = st->pos;
    const int half = hd / 2;
    const int qd = nq * hd, kvd = nkv * hd;
    if (b >= nq + nkv) {
        const int h = b - nq - nkv;
        const float* src = qkv + qd + kvd + h * hd;
        uint16_t* dst = v_cache + (size_t)pos * kvd + h * hd;
        for (int e = lane; e < hd; e += 64) dst[e] = f32_to_f16_bits(src[e]);
        return;
    }
    const bool is_q = b < nq;
    const float* src = is_q ? qkv + b * hd : qkv + qd + (b - nq) * hd;
    const float* nw = is_q ? q_norm : k_norm;
    float rms = 1.0f;
    if (nw) {
        float ss = 0.0f;
        for (int e = lane; e < hd; e += 64) ss += src[e] * src[e];
        ss = wave_sum(ss);
        rms = 1.0f / sqrtf(ss / (float)hd + eps);
    }
    const float* cr = cos_t + (size_t)pos * half;
    const float* sr = sin_t + (size_t)pos * half;
    for (int i = lane; i < half; i += 64) {
        const int i0 = style == 0 ? 2 * i : i;
        const int i1 = style == 0 ? 2 * i + 1 : i + half;
        float x0 = src[i0], x1 = src[i1];
        if (nw) {
            x0 = (x0 * rms) * nw[i0];
            x1 = (x1 * rms) * nw[i1];
        }
        const float c = cr[i], s = sr[i];
        const float o0 = x0 * c - x1 * s;
        const float o1 = x1 * c + x0 * s;
        if (is_q) {
            q_out[b * hd + i0] = o0;
            q_out[b * hd + i1] = o1;
        } else {
            uint16_t* dst = k_cache + (size_t)pos * kvd + (b - nq) * hd;
            dst[i0] = f32_to_f16_bits(o0);
            dst[i1] = f32_to_f16_bits(o1);
        }
    }
}

__device__ __forceinline__ void split_plan(int L, int max_splits, int& splits, int& chunk) {
    splits = (L + 15) / 16;
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    chunk = (L + splits - 1) / splits;
}

// Split-K decode attention (reference: src/cpu_ops.c:202-264).  grid =
// (nkv, max_splits), 256 threads.  Each block covers one KV head (all G query
// heads of its group share the K/V reads) and one range of positions, and
// writes (max, sum of exp, unnormalised P.V) for each query head.
template <int HD, int G>
__global__ __launch_bounds__(256) void k_attn_split(const mdx_state* st, const float* q,
                                                    const uint16_t* kc, const uint16_t* vc,
                                                    int nkv, int max_splits, float* part) {
    constexpr int LP = HD / 8;          // lanes per position row (16-byte chunks)
    constexpr int PPW = 64 / LP;        // positions per wave step
    constexpr int PG = 256 / LP;        // position groups for P.V
    extern __shared__ float smem[];
    float* qs = smem;                   // [G][HD]
    float* sc = qs + G * HD;            // [G][chunk]
    __shared__ float ml[2 * G];

    const int L = st->pos + 1;
    int splits, chunk;
    split_plan(L, max_splits, splits, chunk);
    const int s = blockIdx.y;
    if (s >= splits) return;
    const int kvh = blockIdx.x;
    const int p0 = s * chunk;
    const int p1 = min(L, p0 + chunk);
    const int n = p1 - p0;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kvd = nkv * HD;
    const float scale = 1.0f / sqrtf((float)HD);

    for (int i = tid; i < G * HD; i += 256) qs[i] = q[(size_t)kvh * G * HD + i];
    __syncthreads();

    {
        const int sub = lane % LP, slot = lane / LP;
        for (int pi = wave * PPW + slot; pi - slot < n; pi += 4 * PPW) {
            const bool act = pi < n;
            uint4 kv = make_uint4(0, 0, 0, 0);
            if (act) kv = *reinterpret_cast<const uint4*>(kc + (size_t)(p0 + pi) * kvd + kvh * HD + sub * 8);
            const half2_t k01 = as_h2(kv.x), k23 = as_h2(kv.y), k45 = as_h2(kv.z), k67 = as_h2(kv.w);
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float* qq = qs + g * HD + sub * 8;
                float pd = qq[0] * (float)k01.x;
                pd = pd + qq[1] * (float)k01.y;
                pd = pd + qq[2] * (float)k23.x;
                pd = pd + qq[3] * (float)k23.y;
                pd = pd + qq[4] * (float)k45.x;
                pd = pd + qq[5] * (float)k45.y;
                pd = pd + qq[6] * (float)k67.x;
                pd = pd + qq[7] * (float)k67.y;
                pd = group_sum(pd, LP);
                if (act && sub == 0) sc[g * chunk + pi] = pd * scale;
            }
        }
    }
    __syncthreads();

    for (int g = wave; g < G; g += 4) {
        float m = -1e30f;
        for (int i = lane; i < n; i += 64) m = fmaxf(m, sc[g * chunk + i]);
        m = wave_max(m);
        float l = 0.0f;
        for (int i = lane; i < n; i += 64) {
            const float e = expf(sc[g * chunk + i] - m);
            sc[g * chunk + i] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) { ml[2 * g] = m; ml[2 * g + 1] = l; }
    }
    __syncthreads();

    // P.V: thread = (position group, 8-wide slice of the head dimension)
    const int dsub = tid % LP, pg = tid / LP;
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.0f;
    for (int pi = pg; pi < n; pi += PG) {
        const uint4 vv = *reinterpret_cast<const uint4*>(vc + (size_t)(p0 + pi) * kvd + kvh * HD + dsub * 8);
        const half2_t v01 = as_h2(vv.x), v23 = as_h2(vv.y), v45 = as_h2(vv.z), v67 = as_h2(vv.w);
        const float vf[8] = {(float)v01.x, (float)v01.y, (float)v23.x, (float)v23.y,
                             (float)v45.x, (float)v45.y, (float)v67.x, (float)v67.y};
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float p = sc[g * chunk + pi];
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] = acc[g][e] + vf[e] * p;
        }
    }
    __syncthreads();   // scores no longer needed: reuse smem for the cross-group sum
    float* red = smem; // [PG][G][HD]
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) red[(pg * G + g) * HD + dsub * 8 + e] = acc[g][e];
    __syncthreads();
    float* out = part + ((size_t)kvh * max_splits + s) * G * (HD + 2);
    for (int i = tid; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        float sum = 0.0f;
        for (int k = 0; k < PG; k++) sum += red[(k * G + g) * HD + d];
        out[g * (HD + 2) + d] = sum;
    }
    if (tid < G) {
        out[tid * (HD + 2) + HD] = ml[2 * tid];
        out[tid * (HD + 2) + HD + 1] = ml[2 * tid + 1];
    }
}

// Merges the split partials of one query head: grid = nq, block = HD.
template <int HD, int G>
__global__ __launch_bounds__(256) void k_attn_combine(const mdx_state* st, const float* part,
                                                      int max_splits, uint16_t* out16) {
    const int L = st->pos + 1;
    int splits, chunk;
    split_plan(L, max_splits, splits, chunk);
    const int h = blockIdx.x, kvh = h / G, g = h % G;
    const int d = threadIdx.x;
    const float* base = part + (size_t)kvh * max_splits * G * (HD + 2) + g * (HD + 2);
    const size_t stride = (size_t)G * (HD + 2);
    float m = -1e30f;
    for (int s = 0; s < splits; s++) m = fmaxf(m, base[s * stride + HD]);
    float l = 0.0f, o = 0.0f;
    for (int s = 0; s < splits; s++) {
        const float f = expf(base[s * stride + HD] - m);
        l = l + base[s * stride + HD + 1] * f;
        o = o + base[s * stride + d] * f;
    }
    out16[h * HD + d] = f32_to_f16_bits(o / l);
}

__global__ __launch_bounds__(256) void k_argmax_finish(mdx_state* st, const ArgPair* partial,
                                                       int n, int* out_tokens, int advance) {
    __shared__ ArgPair sh[256];
    const int tid = threadIdx.x;
    ArgPair b = {-INFINITY, -1};
    for (int i = tid; i < n; i += 256) {
        const ArgPair c = partial[i];
        if (c.i >= 0 && (b.i < 0 || c.v > b.v)) b = c;   // i ascending: earlier wins ties
    }
    sh[tid] = b;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) {
            const ArgPair x = sh[tid], y = sh[tid + w];
            ArgPair r = x;
            if (y.i >= 0 && (x.i < 0 || y.v > x.v || (y.v == x.v && y.i < x.i))) r = y;
            sh[tid] = r;
        }
        __syncthreads();
    }
    if (tid == 0) {
        const int tok = sh[0].i < 0 ? 0 : sh[0].i;
        st->argmax = tok;
        st->token = tok;
        st->mode = 0;
        if (out_tokens) out_tokens[st->n_out] = tok;
        if (out_tokens) st->n_out = st->n_out + 1;
        st->pos = st->pos + advance;
    }
}

__global__ void k_advance(mdx_state* st, int advance) {
    if (threadIdx.x == 0) st->pos = st->pos + advance;
}

}  // namespace

extern "C" {

int mdx_launch_embed(const mdx_state* state, const float* emb_table, const float* emb_in,
                     float* hidden, int d, int vocab, void* stream) {
    const int blocks = (d + 255) / 256;
    hipLaunchKernelGGL(k_embed, dim3(blocks), dim3(256), 0, (hipStream_t)stream, state, emb_table,
                       emb_in, hidden, d, vocab);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int mdx_launch_norm_gemv(const float* hidden, const float* norm_w, float eps, const mdx_wdesc* w,
                         int epilogue, void* out, void* stream) {
    GemvArgs a = {};
    a.w = (const uint8_t*)w->w;
    a.scale = w->scale;
    a.K = w->K;
    a.N = w->N;
    a.xmode = XM_NORM;
    a.xf32 = hidden;
    a.norm_w = norm_w;
    a.eps = eps;
    if (epilogue == 1) {
        if (w->N % 2) return -1;
        a.n_units = w->N / 2;
        a.unit_rows = 2;
        a.epi = EP_SWIGLU;
        a.out_f16 = (uint16_t*)out;
    } else {
        a.n_units = w->N;
        a.unit_rows = 1;
        a.epi = EP_STORE;
        a.out_f32 = (float*)out;
    }
    const int kind = kind_from(w, 0);
    int rw = rows_per_wave_for(kind, a.n_units * a.unit_rows, a.K);
    if (a.unit_rows == 2 && rw < 2) rw = 2;
    return launch_gemv(kind, a, rw, stream);
}

int mdx_launch_gemv_add(const uint16_t* x16, const mdx_wdesc* w, float* out, void* stream) {
    GemvArgs a = {};
    a.w = (const uint8_t*)w->w;
    a.scale = w->scale;
    a.K = w->K;
    a.N = w->N;
    a.n_units = w->N;
    a.unit_rows = 1;
    a.xmode = XM_F16;
    a.x16 = x16;
    a.epi = EP_ADD;
    a.out_f32 = out;
    const int kind = kind_from(w, 0);
    return launch_gemv(kind, a, rows_per_wave_for(kind, a.N, a.K), stream);
}

int mdx_launch_gemv_f16in(const uint16_t* x16, const mdx_wdesc* w, float* y, void* stream) {
    GemvArgs a = {};
    a.w = (const uint8_t*)w->w;
    a.scale = w->scale;
    a.K = w->K;
    a.N = w->N;
    a.n_units = w->N;
    a.unit_rows = 1;
    a.xmode = XM_F16;
    a.x16 = x16;
    a.epi = EP_STORE;
    a.out_f32 = y;
    const int kind = kind_from(w, 0);
    return launch_gemv(kind, a, rows_per_wave_for(kind, a.N, a.K), stream);
}

int mdx_launch_gemv(const float* x, const mdx_wdesc* w, int x_fp32_exact, float* y, void* stream) {
    GemvArgs a = {};
    a.w = (const uint8_t*)w->w;
    a.scale = w->scale;
    a.K = w->K;
    a.N = w->N;
    a.n_units = w->N;
    a.unit_rows = 1;
    a.xmode = XM_F32;
    a.xf32 = x;
    a.epi = EP_STORE;
    a.out_f32 = y;
    const int kind = kind_from(w, x_fp32_exact);
    return launch_gemv(kind, a, rows_per_wave_for(kind, a.N, a.K), stream);
}

int mdx_lmhead_partials(int N) {
    const int rw = rows_per_wave_for(KI8, N, 0);
    return (N + 4 * rw - 1) / (4 * rw);
}

int mdx_launch_lmhead(const float* hidden, const float* norm_w, float eps, const mdx_wdesc* w,
                      float* logits, void* partial, void* stream) {
    GemvArgs a = {};
    a.w = (const uint8_t*)w->w;
    a.scale = w->scale;
    a.K = w->K;
    a.N = w->N;
    a.n_units = w->N;
    a.unit_rows = 1;
    a.xmode = XM_NORM;
    a.xf32 = hidden;
    a.norm_w = norm_w;
    a.eps = eps;
    a.epi = EP_LOGITS;
    a.out_f32 = logits;
    a.partial = (ArgPair*)partial;
    // fp16 rows take fp32 activations here (the reference's CPU lm_head)
    const int kind = kind_from(w, 1);
    return launch_gemv(kind, a, rows_per_wave_for(KI8, w->N, 0), stream);
}

int mdx_launch_argmax_finish(mdx_state* state, const void* partial, int n_partials,
                             int* out_tokens, int advance, void* stream) {
    hipLaunchKernelGGL(k_argmax_finish, dim3(1), dim3(256), 0, (hipStream_t)stream, state,
                       (const ArgPair*)partial, n_partials, out_tokens, advance);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int mdx_launch_advance(mdx_state* state, int advance, void* stream) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, (hipStream_t)stream, state, advance);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int mdx_launch_qk_rope_append(const mdx_state* state, const float* qkv, const float* q_norm,
                              const float* k_norm, float eps, const float* cos_t,
                              const float* sin_t, int nq, int nkv, int hd, int rope_style,
                              float* q_out, uint16_t* k_cache, uint16_t* v_cache, void* stream) {
    if (hd % 2) return -1;
    hipLaunchKernelGGL(k_qk_rope_append, dim3(nq + 2 * nkv), dim3(64), 0, (hipStream_t)stream,
                       state, qkv, q_norm, k_norm, eps, cos_t, sin_t, nq, nkv, hd, rope_style,
                       q_out, k_cache, v_cache);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

size_t mdx_attn_decode_scratch_floats(int nq, int hd, int max_splits) {
    return (size_t)nq * max_splits * (hd + 2);
}

int mdx_launch_attn_decode(const mdx_state* state, const float* q, const uint16_t* k_cache,
                           const uint16_t* v_cache, int nq, int nkv, int hd, int max_seq,
                           int max_splits, float* part, uint16_t* attn_out16, void* stream) {
    if (nkv <= 0 || nq % nkv) return -1;
    const int G = nq / nkv;
    // The split plan keeps chunk <= 16 positions as long as L <= 16*max_splits;
    // L <= max_seq, so that bound is required here (it sizes the LDS score row).
    if ((long)max_splits * 16 < (long)max_seq) return -1;
    const int chunk_max = 16;
    const int LP = hd / 8;
    const int PG = 256 / (LP > 0 ? LP : 1);
    size_t lds_a = (size_t)(G * hd + G * chunk_max) * 4;
    size_t lds_b = (size_t)PG * G * hd * 4;
    const size_t lds = lds_a > lds_b ? lds_a : lds_b;
    if (lds > 64 * 1024) return -5;
    dim3 grid(nkv, max_splits);
#define MDX_ATTN(HD_, G_)                                                                        \
    if (hd == HD_ && G == G_) {                                                                  \
        hipLaunchKernelGGL((k_attn_split<HD_, G_>), grid, dim3(256), lds, (hipStream_t)stream,   \
                           state, q, k_cache, v_cache, nkv, max_splits, part);                   \
        hipLaunchKernelGGL((k_attn_combine<HD_, G_>), dim3(nq), dim3(HD_), 0,                   \
                           (hipStream_t)stream, state, part, max_splits, attn_out16);            \
        return hipGetLastError() == hipSuccess ? 0 : -4;                                         \
    }
    MDX_ATTN(64, 1) MDX_ATTN(64, 2) MDX_ATTN(64, 4) MDX_ATTN(64, 8)
    MDX_ATTN(128, 1) MDX_ATTN(128, 2) MDX_ATTN(128, 4) MDX_ATTN(128, 8)
    MDX_ATTN(256, 1) MDX_ATTN(256, 2) MDX_ATTN(256, 4)
#undef MDX_ATTN
    return -5;
}

}  // extern "C"
