// mdx_prefill.hip — batch prefill (M <= 64 rows) kernels for gfx950.
//
// Projections (reference: src/matmul_decoder.c:1841-1899, run_batch_matmul)
// run on MFMA v_mfma_f32_16x16x32_f16: a block owns a 64 x 32 output tile
// (all M rows, 32 weight rows of W^T) over a K range; int8/int4 weights are
// widened to fp16 exactly while being staged into LDS, and the next K chunk
// is fetched into registers while the current one is multiplied.  Split-K
// partials are summed in a second pass that applies the per-column scale and
// the epilogue (residual add or SwiGLU), so the result does not depend on
// scheduling.
#include <hip/hip_runtime.h>

#include <cmath>

#include "mdx_common.h"
#include "mdx_device.h"

using namespace mdx;

namespace {

constexpr int kMaxM = 64;
constexpr int kNT = 32;        // weight rows (output columns) per block
constexpr int kKC = 128;       // K per staged chunk
constexpr int kLdsStride = kKC + 8;   // halfs per LDS row (pad against bank conflicts)

__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float* x, const float* w, float eps,
                                                       int d, uint16_t* x16) {
    __shared__ float red[4];
    const int m = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (size_t)m * d;
    float ss = 0.0f;
    for (int k = tid; k < d; k += 256) ss += xr[k] * xr[k];
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float tot = red[0] + red[1] + red[2] + red[3];
    const float rms = 1.0f / sqrtf(tot / (float)d + eps);
    for (int k = tid; k < d; k += 256) x16[(size_t)m * d + k] = f32_to_f16_bits((xr[k] * rms) * w[k]);
}

__global__ void k_to_f16(const float* x, int n, uint16_t* x16) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        x16[i] = f32_to_f16_bits(x[i]);
}

// Bytes of one staged chunk row (kKC elements) for each weight kind.
template <int KIND> struct Stage;
template <> struct Stage<MDX_W_F16> { static constexpr int RB = kKC * 2; };
template <> struct Stage<MDX_W_I8> { static constexpr int RB = kKC; };
template <> struct Stage<MDX_W_I4> { static constexpr int RB = kKC / 2; };
// 16-byte pieces per chunk = kNT * RB / 16; pieces per thread = that / 256.

template <int KIND>
__device__ __forceinline__ void widen_store(uint4 v, uint16_t* dst /* LDS, 8/16/32 halfs */) {
    if constexpr (KIND == MDX_W_F16) {
        *reinterpret_cast<uint4*>(dst) = v;
    } else if constexpr (KIND == MDX_W_I8) {
        const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
        uint32_t o[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            half2_t a, b;
            i8x4_to_h2x2(wd[i], a, b);
            o[2 * i] = h2_bits(a);
            o[2 * i + 1] = h2_bits(b);
        }
        *reinterpret_cast<uint4*>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<uint4*>(dst + 8) = make_uint4(o[4], o[5], o[6], o[7]);
    } else {
        const uint32_t wd[4] = {v.x ^ 0x88888888u, v.y ^ 0x88888888u, v.z ^ 0x88888888u,
                                v.w ^ 0x88888888u};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t o[4];
#pragma unroll
            for (int p = 0; p < 4; p++) o[p] = h2_bits(i4_pair(wd[i], p));
            *reinterpret_cast<uint4*>(dst + 8 * i) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}

// grid = (ceil(N / 32), nsplit); block 256 = 4 waves, wave w owns rows
// [16w, 16w+16) of the M dimension and both 16-column MFMA tiles.
template <int KIND>
__global__ __launch_bounds__(256) void k_gemm(const uint16_t* x16, int M, const uint8_t* w, int K,
                                              int N, int kchunks_per_split, float* part) {
    constexpr int RB = Stage<KIND>::RB;
    constexpr int EPP = 16 * kKC / RB;                       // elements per 16-byte piece
    constexpr int PIECES = kNT * RB / 16;
    constexpr int PPT = PIECES / 256 > 0 ? PIECES / 256 : 1; // pieces per thread
    __shared__ __attribute__((aligned(16))) uint16_t bs[kNT * kLdsStride];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n0 = blockIdx.x * kNT;
    const int nkc = (K + kKC - 1) / kKC;
    const int c_begin = blockIdx.y * kchunks_per_split;
    const int c_end = min(nkc, c_begin + kchunks_per_split);
    const size_t row_bytes = (size_t)K * (KIND == MDX_W_F16 ? 2 : 1) / (KIND == MDX_W_I4 ? 2 : 1);

    float4_t acc[2];
    acc[0] = float4_t{0.f, 0.f, 0.f, 0.f};
    acc[1] = float4_t{0.f, 0.f, 0.f, 0.f};

    const int arow = 16 * wave + (lane & 15);
    const int kq = 8 * (lane >> 4);            // this lane's k offset inside a 32-wide step

    auto load_chunk = [&](int c, uint4* regs) {
#pragma unroll
        for (int p = 0; p < PPT; p++) {
            const int piece = tid + p * 256;
            regs[p] = make_uint4(0, 0, 0, 0);
            if (piece < PIECES) {
                const int r = piece / (RB / 16), q = piece % (RB / 16);
                const int n = n0 + r;
                const size_t off = (size_t)c * RB + (size_t)q * 16;
                if (n < N && off + 16 <= row_bytes)
                    regs[p] = *reinterpret_cast<const uint4*>(w + (size_t)n * row_bytes + off);
            }
        }
    };
    auto store_chunk = [&](const uint4* regs) {
#pragma unroll
        for (int p = 0; p < PPT; p++) {
            const int piece = tid + p * 256;
            if (piece < PIECES) {
                const int r = piece / (RB / 16), q = piece % (RB / 16);
                widen_store<KIND>(regs[p], bs + r * kLdsStride + q * EPP);
            }
        }
    };

    uint4 regs[PPT];
    if (c_begin < c_end) load_chunk(c_begin, regs);
    for (int c = c_begin; c < c_end; c++) {
        __syncthreads();
        store_chunk(regs);
        __syncthreads();
        if (c + 1 < c_end) load_chunk(c + 1, regs);
        const int kbase = c * kKC;
#pragma unroll
        for (int ks = 0; ks < kKC; ks += 32) {
            const int k = kbase + ks + kq;
            half8_t a = {};
            if (arow < M && k + 8 <= K)
                a = *reinterpret_cast<const half8_t*>(x16 + (size_t)arow * K + k);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const half8_t b =
                    *reinterpret_cast<const half8_t*>(bs + (16 * t + (lane & 15)) * kLdsStride + ks + kq);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[t], 0, 0, 0);
            }
        }
    }

    float* out = part + (size_t)blockIdx.y * kMaxM * N;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int col = n0 + 16 * t + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = 16 * wave + 4 * (lane >> 4) + i;
            if (row < M && col < N) out[(size_t)row * N + col] = acc[t][i];
        }
    }
}

// Sums split partials, applies scale and the epilogue.  grid over outputs.
__global__ void k_gemm_reduce(const float* part, int nsplit, int M, int N, const float* scale,
                              int epi, float* out_f32, uint16_t* out_f16) {
    const int cols = epi == 2 ? N / 2 : N;
    const int total = M * cols;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int m = i / cols, n = i % cols;
        if (epi == 2) {
            float g = 0.0f, u = 0.0f;
            for (int s = 0; s < nsplit; s++) {
                g += part[((size_t)s * kMaxM + m) * N + n];
                u += part[((size_t)s * kMaxM + m) * N + n + cols];
            }
            if (scale) {
                g = g * scale[n];
                u = u * scale[n + cols];
            }
            float v;
            if (n < (cols & ~3)) v = silu_mul(g, u);
            else v = (g / (1.0f + expf(-g))) * u;
            out_f16[(size_t)m * cols + n] = f32_to_f16_bits(v);
        } else {
            float y = 0.0f;
            for (int s = 0; s < nsplit; s++) y += part[((size_t)s * kMaxM + m) * N + n];
            if (scale) y = y * scale[n];
            if (epi == 1) out_f32[(size_t)m * N + n] = out_f32[(size_t)m * N + n] + y;
            else out_f32[(size_t)m * N + n] = y;
        }
    }
}

int plan_splits(int N, int K, int* chunks_per_split) {
    const int ntiles = (N + kNT - 1) / kNT;
    const int nkc = (K + kKC - 1) / kKC;
    int ns = (384 + ntiles - 1) / ntiles;
    if (ns > nkc) ns = nkc;
    if (ns < 1) ns = 1;
    const int cps = (nkc + ns - 1) / ns;
    *chunks_per_split = cps;
    return (nkc + cps - 1) / cps;
}

// QK-norm + RoPE + append for M rows (reference: src/matmul_decoder.c:1984-2034,
// rope via the table formula of :620-631, identical to apply_rope_batch_f32).
// grid = (nq + 2*nkv, M), 64 threads.
__global__ __launch_bounds__(64) void k_qk_rope_append_rows(
    const mdx_state* st, const float* qkv, const float* q_norm, const float* k_norm, float eps,
    const float* cos_t, const float* sin_t, int nq, int nkv, int hd, int style, float* q_out,
    uint16_t* k_cache, uint16_t* v_cache) {
    const int b = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int pos = st->pos + t;
    const int half = hd / 2;
    const int qd = nq * hd, kvd = nkv * hd;
    const float* row = qkv + (size_t)t * (qd + 2 * kvd);
    if (b >= nq + nkv) {
        const int h = b - nq - nkv;
        const float* src = row + qd + kvd + h * hd;
        uint16_t* dst = v_cache + (size_t)pos * kvd + h * hd;
        for (int e = lane; e < hd; e += 64) dst[e] = f32_to_f16_bits(src[e]);
        return;
    }
    const bool is_q = b < nq;
    const float* src = is_q ? row + b * hd : row + qd + (b - nq) * hd;
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
            q_out[(size_t)t * qd + b * hd + i0] = o0;
            q_out[(size_t)t * qd + b * hd + i1] = o1;
        } else {
            uint16_t* dst = k_cache + (size_t)pos * kvd + (b - nq) * hd;
            dst[i0] = f32_to_f16_bits(o0);
            dst[i1] = f32_to_f16_bits(o1);
        }
    }
}

// Causal attention for one query row and one KV head group (reference:
// src/cpu_ops.c:459-571, over the cache rows that already hold the batch's
// own K/V).  grid = (nkv, M), 256 threads; positions are streamed in tiles
// of 16 with a running max and sum.
template <int HD, int G>
__global__ __launch_bounds__(256) void k_attn_prefill(const mdx_state* st, const float* q,
                                                      const uint16_t* kc, const uint16_t* vc,
                                                      int nkv, uint16_t* out16) {
    constexpr int LP = HD / 8;
    constexpr int PPW = 64 / LP;
    constexpr int TILE = 4 * PPW;       // positions scored per tile
    constexpr int PG = 256 / LP;
    __shared__ float qs[G * HD];
    __shared__ float sc[G * TILE];
    __shared__ float mrun[G], lrun[G], fac[G];
    extern __shared__ float red[];      // [PG][G][HD]

    const int kvh = blockIdx.x, t = blockIdx.y;
    const int nq = nkv * G;
    const int L = st->pos + t + 1;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kvd = nkv * HD;
    const float scale = 1.0f / sqrtf((float)HD);
    for (int i = tid; i < G * HD; i += 256) qs[i] = q[(size_t)t * nq * HD + (size_t)kvh * G * HD + i];
    if (tid < G) { mrun[tid] = -1e30f; lrun[tid] = 0.0f; }
    __syncthreads();

    const int dsub = tid % LP, pg = tid / LP;
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.0f;

    for (int p0 = 0; p0 < L; p0 += TILE) {
        const int n = min(TILE, L - p0);
        {
            const int sub = lane % LP, slot = lane / LP;
            const int pi = wave * PPW + slot;
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
                if (act && sub == 0) sc[g * TILE + pi] = pd * scale;
            }
        }
        __syncthreads();
        if (wave == 0) {
            for (int g = 0; g < G; g++) {
                float m = lane < n ? sc[g * TILE + lane] : -1e30f;
                m = wave_max(m);
                const float mnew = fmaxf(mrun[g], m);
                float e = 0.0f;
                if (lane < n) {
                    e = expf(sc[g * TILE + lane] - mnew);
                    sc[g * TILE + lane] = e;
                }
                const float lsum = wave_sum(e);
                if (lane == 0) {
                    const float f = expf(mrun[g] - mnew);
                    fac[g] = f;
                    lrun[g] = lrun[g] * f + lsum;
                    mrun[g] = mnew;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] = acc[g][e] * fac[g];
        for (int pi = pg; pi < n; pi += PG) {
            const uint4 vv = *reinterpret_cast<const uint4*>(vc + (size_t)(p0 + pi) * kvd + kvh * HD + dsub * 8);
            const half2_t v01 = as_h2(vv.x), v23 = as_h2(vv.y), v45 = as_h2(vv.z), v67 = as_h2(vv.w);
            const float vf[8] = {(float)v01.x, (float)v01.y, (float)v23.x, (float)v23.y,
                                 (float)v45.x, (float)v45.y, (float)v67.x, (float)v67.y};
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float p = sc[g * TILE + pi];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[g][e] = acc[g][e] + vf[e] * p;
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) red[(pg * G + g) * HD + dsub * 8 + e] = acc[g][e];
    __syncthreads();
    for (int i = tid; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        float s = 0.0f;
        for (int k = 0; k < PG; k++) s += red[(k * G + g) * HD + d];
        out16[(size_t)t * nq * HD + (size_t)(kvh * G + g) * HD + d] = f32_to_f16_bits(s / lrun[g]);
    }
}

__global__ void k_copy_row(const float* x, int row, int d, float* dst) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < d; i += gridDim.x * blockDim.x)
        dst[i] = x[(size_t)row * d + i];
}

}  // namespace

extern "C" {

int mdx_launch_rmsnorm_rows(const float* x, const float* w, float eps, int M, int d,
                            uint16_t* x16, void* stream) {
    if (M <= 0) return -1;
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(M), dim3(256), 0, (hipStream_t)stream, x, w, eps, d, x16);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int mdx_launch_to_f16(const float* x, int n, uint16_t* x16, void* stream) {
    int blocks = (n + 255) / 256;
    if (blocks > 2048) blocks = 2048;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_to_f16, dim3(blocks), dim3(256), 0, (hipStream_t)stream, x, n, x16);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

size_t mdx_gemm_scratch_floats(int M, int N, int K) {
    (void)M;
    int cps;
    const int ns = plan_splits(N, K, &cps);
    return (size_t)ns * kMaxM * N;
}

int mdx_launch_gemm(const uint16_t* x16, int M, const mdx_wdesc* w, int epilogue, void* out,
                    float* scratch, void* stream) {
    if (M <= 0 || M > kMaxM || w->K % 32 != 0) return -1;
    if (epilogue == 2 && w->N % 2) return -1;
    if (w->kind == MDX_W_I4 && w->K % kKC != 0) return -1;   // int4 pieces are whole 16-byte words
    int cps;
    const int ns = plan_splits(w->N, w->K, &cps);
    dim3 grid((w->N + kNT - 1) / kNT, ns);
    const uint8_t* wp = (const uint8_t*)w->w;
    switch (w->kind) {
        case MDX_W_F16:
            hipLaunchKernelGGL(k_gemm<MDX_W_F16>, grid, dim3(256), 0, (hipStream_t)stream, x16, M, wp,
                               w->K, w->N, cps, scratch);
            break;
        case MDX_W_I8:
            hipLaunchKernelGGL(k_gemm<MDX_W_I8>, grid, dim3(256), 0, (hipStream_t)stream, x16, M, wp,
                               w->K, w->N, cps, scratch);
            break;
        case MDX_W_I4:
            hipLaunchKernelGGL(k_gemm<MDX_W_I4>, grid, dim3(256), 0, (hipStream_t)stream, x16, M, wp,
                               w->K, w->N, cps, scratch);
            break;
        default:
            return -5;
    }
    if (hipGetLastError() != hipSuccess) return -4;
    const int cols = epilogue == 2 ? w->N / 2 : w->N;
    int blocks = (M * cols + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(k_gemm_reduce, dim3(blocks), dim3(256), 0, (hipStream_t)stream, scratch, ns, M,
                       w->N, w->scale, epilogue, (float*)out, (uint16_t*)out);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int mdx_launch_qk_rope_append_rows(const mdx_state* state, const float* qkv, int M,
                                   const float* q_norm, const float* k_norm, float eps,
                                   const float* cos_t, const float* sin_t, int nq, int nkv,
                                   int hd, int rope_style, float* q_out, uint16_t* k_cache,
                                   uint16_t* v_cache, void* stream) {
    if (hd % 2 || M <= 0) return -1;
    hipLaunchKernelGGL(k_qk_rope_append_rows, dim3(nq + 2 * nkv, M), dim3(64), 0, (hipStream_t)stream,
                       state, qkv, q_norm, k_norm, eps, cos_t, sin_t, nq, nkv, hd, rope_style, q_out,
                       k_cache, v_cache);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int mdx_launch_attn_prefill(const mdx_state* state, const float* q, int M,
                            const uint16_t* k_cache, const uint16_t* v_cache, int nq, int nkv,
                            int hd, uint16_t* out16, void* stream) {
    if (nkv <= 0 || nq % nkv || M <= 0) return -1;
    const int G = nq / nkv;
    const int LP = hd / 8;
    const int PG = 256 / (LP > 0 ? LP : 1);
    const size_t lds = (size_t)PG * G * hd * 4;
    if (lds > 48 * 1024) return -5;
    dim3 grid(nkv, M);
#define MDX_PATTN(HD_, G_)                                                                          \
    if (hd == HD_ && G == G_) {                                                                     \
        hipLaunchKernelGGL((k_attn_prefill<HD_, G_>), grid, dim3(256), lds, (hipStream_t)stream,    \
                           state, q, k_cache, v_cache, nkv, out16);                                 \
        return hipGetLastError() == hipSuccess ? 0 : -4;                                            \
    }
    MDX_PATTN(64, 1) MDX_PATTN(64, 2) MDX_PATTN(64, 4)
    MDX_PATTN(128, 1) MDX_PATTN(128, 2) MDX_PATTN(128, 4) MDX_PATTN(128, 8)
    MDX_PATTN(256, 1) MDX_PATTN(256, 2) MDX_PATTN(256, 4)
#undef MDX_PATTN
    return -5;
}

int mdx_launch_copy_row(const float* x, int row, int d, float* dst, void* stream) {
    hipLaunchKernelGGL(k_copy_row, dim3((d + 255) / 256), dim3(256), 0, (hipStream_t)stream, x, row, d,
                       dst);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // extern "C"
