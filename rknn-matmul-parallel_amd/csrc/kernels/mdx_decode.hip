// mdx_decode.hip — M = 1 decode kernels for gfx950.
//
// Projections (reference: src/matmul_decoder.c:382-445, the NPU call sites
// K1/K2; CPU GEMVs :511-616) run as bandwidth-bound GEMVs over the W^T
// device layout: each wave owns RW weight rows, every lane streams 16-byte
// chunks of each row (one wave load instruction reads 1 KiB contiguous),
// dequantises in registers, accumulates with v_dot2_f32_f16 and reduces with
// lane shuffles.  The weight loads are issued before the activation prologue
// (they do not depend on it), so HBM latency overlaps the RMSNorm that
// builds the fp16 activation vector in LDS (reference: src/cpu_ops.c:18-55).
//
// Attention (reference: src/cpu_ops.c:202-264 and the QK-norm/RoPE/KV-append
// steps of src/matmul_decoder.c:1493-1520) is one kernel per layer: every
// block normalises and rotates its query heads itself, the block holding the
// newest position appends that position's K/V to the fp16 cache, blocks
// split the positions, and the last block to finish merges the splits.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>

#include "mdx_common.h"
#include "mdx_device.h"

using namespace mdx;

namespace {

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

enum XMode { XM_NORM = 0, XM_F16 = 1, XM_F32 = 2, XM_EMBED = 3 };
enum Epi { EP_STORE = 0, EP_ADD = 1, EP_SWIGLU = 2, EP_LOGITS = 3 };
// KF16/KI8/KI4: fp16 activations (the NPU input).  KF32X: fp32 rows with fp32
// activations, KF16X: fp16 rows with fp32 activations (the CPU GEMVs).
enum Kind { KF16 = 0, KI8 = 1, KI4 = 2, KF32X = 3, KF16X = 4 };

struct GemvArgs {
    const uint8_t* w;
    const float* scale;
    int K, N;             // N weight rows
    int n_units;          // unit u uses rows u (and u + n_units when unit_rows == 2)
    int unit_rows;
    int xmode;
    const float* xf32;    // XM_NORM/XM_F32 input, XM_EMBED uploaded embedding
    const uint16_t* x16;
    const float* norm_w;
    float eps;
    int epi;
    float* out_f32;
    uint16_t* out_f16;
    // XM_EMBED: input row chosen by state->mode / state->token, copied to hidden_out
    const mdx_state* st_in;
    const float* emb_table;
    int vocab;
    float* hidden_out;
    // EP_LOGITS: fused argmax and step bookkeeping
    mdx_state* st;
    unsigned long long* amax_key;
    unsigned int* done;
    int* out_tokens;
    int advance;
};

template <int KIND> struct KindTraits;
template <> struct KindTraits<KF16> { static constexpr int E = 8; static constexpr bool XF32 = false; static constexpr int EB2 = 4; };
template <> struct KindTraits<KI8> { static constexpr int E = 16; static constexpr bool XF32 = false; static constexpr int EB2 = 2; };
template <> struct KindTraits<KI4> { static constexpr int E = 32; static constexpr bool XF32 = false; static constexpr int EB2 = 1; };
template <> struct KindTraits<KF32X> { static constexpr int E = 4; static constexpr bool XF32 = true; static constexpr int EB2 = 8; };
template <> struct KindTraits<KF16X> { static constexpr int E = 8; static constexpr bool XF32 = true; static constexpr int EB2 = 4; };
// E = elements per 16-byte chunk; EB2 = row bytes per element, times 2.

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

// x is read as 4-element vectors (K is a multiple of 4 for every kind),
// kXV per thread at a time, all loads of a batch issued before the first is
// used (indexes clamped to the last vector, so no load needs a branch):
// staging costs one cache round trip per batch, where a load-use loop would
// wait on each element for every earlier load, the weights included.
constexpr int kXV = 2;

// The row that supplies x (the embedding row of the current token in
// XM_EMBED mode, unless the embedding was uploaded).
__device__ __forceinline__ const float* x_source(const GemvArgs& a) {
    const float* src = a.xf32;
    if (a.xmode == XM_EMBED && a.st_in->mode != 1) {
        int tok = a.st_in->token;
        tok = tok < 0 ? 0 : (tok >= a.vocab ? a.vocab - 1 : tok);
        src = a.emb_table + (size_t)tok * a.K;
    }
    return src;
}

// The first batch of build_x's loads, issued on its own so that a kernel can
// request x before its weights: loads complete in issue order, so staging x
// then waits for x alone while the weights are still arriving.
struct XFirst {
    float4 v[kXV], g[kXV];
    uint2 h[kXV];
};
__device__ __forceinline__ void build_x_first(const GemvArgs& a, XFirst& f) {
    const int tid = threadIdx.x, nt = blockDim.x, nv = a.K / 4;
    if (a.xmode == XM_F16) {
        const uint2* x16 = reinterpret_cast<const uint2*>(a.x16);
#pragma unroll
        for (int i = 0; i < kXV; i++) f.h[i] = x16[min(tid + i * nt, nv - 1)];
        return;
    }
    const float4* s4 = reinterpret_cast<const float4*>(x_source(a));
#pragma unroll
    for (int i = 0; i < kXV; i++) f.v[i] = s4[min(tid + i * nt, nv - 1)];
    if (a.xmode == XM_NORM || a.xmode == XM_EMBED) {
        const float4* g4 = reinterpret_cast<const float4*>(a.norm_w);
#pragma unroll
        for (int i = 0; i < kXV; i++) f.g[i] = g4[min(tid + i * nt, nv - 1)];
    }
}

// Builds the activation vector in LDS: fp16 for the NPU-style kinds, fp32 for
// the CPU-GEMV kinds.  XM_NORM / XM_EMBED apply the reference RMSNorm first.
// With `first`, the first batch comes from build_x_first instead of new loads.
template <bool XF32>
__device__ __forceinline__ void build_x(const GemvArgs& a, void* xs_raw, float* red,
                                        const XFirst* first = nullptr) {
    const int tid = threadIdx.x, nt = blockDim.x;
    const int K = a.K, nv = K / 4, step = kXV * nt;
    float4* xs32 = reinterpret_cast<float4*>(xs_raw);
    uint2* xs16 = reinterpret_cast<uint2*>(xs_raw);
    if (a.xmode == XM_F16) {
        const uint2* x16 = reinterpret_cast<const uint2*>(a.x16);
        for (int q0 = tid; q0 < nv; q0 += step) {
            uint2 h[kXV];
#pragma unroll
            for (int i = 0; i < kXV; i++) h[i] = first && q0 == tid ? first->h[i] : x16[min(q0 + i * nt, nv - 1)];
#pragma unroll
            for (int i = 0; i < kXV; i++) {
                const int q = q0 + i * nt;
                if (q >= nv) break;
                if constexpr (XF32)
                    xs32[q] = make_float4(f16_bits_to_f32(h[i].x & 0xffff), f16_bits_to_f32(h[i].x >> 16),
                                          f16_bits_to_f32(h[i].y & 0xffff), f16_bits_to_f32(h[i].y >> 16));
                else xs16[q] = h[i];
            }
        }
        __syncthreads();
        return;
    }
    const float* src = x_source(a);
    const bool embed = a.xmode == XM_EMBED;
    const bool norm = a.xmode == XM_NORM || embed;
    const bool copy = embed && blockIdx.x == 0;
    const float4* s4 = reinterpret_cast<const float4*>(src);
    const float4* g4 = reinterpret_cast<const float4*>(a.norm_w);
    float4 v[kXV], g[kXV];
    if (first) {
#pragma unroll
        for (int i = 0; i < kXV; i++) {
            v[i] = first->v[i];
            g[i] = first->g[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < kXV; i++) v[i] = s4[min(tid + i * nt, nv - 1)];
        if (norm) {
#pragma unroll
            for (int i = 0; i < kXV; i++) g[i] = g4[min(tid + i * nt, nv - 1)];
        }
    }
    float rms = 1.0f;
    if (norm) {
        float ss = 0.0f;
        for (int q0 = tid; q0 < nv; q0 += step) {
            float4 u[kXV];
#pragma unroll
            for (int i = 0; i < kXV; i++) u[i] = q0 == tid ? v[i] : s4[min(q0 + i * nt, nv - 1)];
#pragma unroll
            for (int i = 0; i < kXV; i++) {
                const int q = q0 + i * nt;
                if (q >= nv) break;
                if (copy) reinterpret_cast<float4*>(a.hidden_out)[q] = u[i];
                ss += u[i].x * u[i].x;
                ss += u[i].y * u[i].y;
                ss += u[i].z * u[i].z;
                ss += u[i].w * u[i].w;
            }
        }
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int wv = 0; wv < (nt >> 6); wv++) tot += red[wv];
        rms = 1.0f / sqrtf(tot / (float)K + a.eps);
    }
    for (int q0 = tid; q0 < nv; q0 += step) {
        if (q0 != tid) {
#pragma unroll
            for (int i = 0; i < kXV; i++) {
                const int q = min(q0 + i * nt, nv - 1);
                v[i] = s4[q];
                if (norm) g[i] = g4[q];
            }
        }
#pragma unroll
        for (int i = 0; i < kXV; i++) {
            const int q = q0 + i * nt;
            if (q >= nv) break;
            float4 x = v[i];
            if (norm) {
                x.x = (x.x * rms) * g[i].x;
                x.y = (x.y * rms) * g[i].y;
                x.z = (x.z * rms) * g[i].z;
                x.w = (x.w * rms) * g[i].w;
            }
            if constexpr (XF32) xs32[q] = x;
            else xs16[q] = make_uint2((uint32_t)f32_to_f16_bits(x.x) | ((uint32_t)f32_to_f16_bits(x.y) << 16),
                                      (uint32_t)f32_to_f16_bits(x.z) | ((uint32_t)f32_to_f16_bits(x.w) << 16));
        }
    }
    __syncthreads();
}

template <int KIND, int RW, int U>
struct RowSet {
    int rows[RW];
    bool valid[RW];
    float sc[RW];   // per-row scales, requested with the row set (not after the reduction)
    __device__ __forceinline__ void init(const GemvArgs& a, int blk, int wave) {
        const int slot0 = (blk * 4 + wave) * RW;
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const int slot = slot0 + r;
            // unit_rows is 1 or 2
            const int unit = slot >> (a.unit_rows - 1), which = slot & (a.unit_rows - 1);
            valid[r] = unit < a.n_units;
            rows[r] = unit + which * a.n_units;
            sc[r] = (a.scale && valid[r]) ? a.scale[rows[r]] : 1.0f;
        }
    }
    __device__ __forceinline__ void load(const GemvArgs& a, size_t row_bytes, int nchunks, int base,
                                         int lane, uint4 (&wv)[RW][U]) const {
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const uint4* rp = reinterpret_cast<const uint4*>(a.w + (size_t)rows[r] * row_bytes);
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int j = base + u * 64 + lane;
                wv[r][u] = (valid[r] && j < nchunks) ? ld_nt(rp + j) : make_uint4(0, 0, 0, 0);
            }
        }
    }
};

// The stores of a wave's RW reduced rows (lane r stores row r).
template <int KIND, int RW, int U>
__device__ __forceinline__ void store_rows(const GemvArgs& a, const RowSet<KIND, RW, U>& cur,
                                           const float (&y)[RW], int lane) {
    if (a.epi == EP_SWIGLU) {
        // slots come in (gate, up) pairs: slot 2c is row unit, 2c+1 row unit + F
#pragma unroll
        for (int r = 0; r + 1 < RW; r += 2) {
            if (cur.valid[r] && lane == r) {
                const int unit = cur.rows[r];
                const float g = y[r], u = y[r + 1];
                float v;
                if (unit < (a.n_units & ~3)) v = silu_mul(g, u);
                else v = (g / (1.0f + expf(-g))) * u;     // reference tail formula
                a.out_f16[unit] = f32_to_f16_bits(v);
            }
        }
    } else {     // EP_STORE, EP_ADD, and the logits of EP_LOGITS
#pragma unroll
        for (int r = 0; r < RW; r++) {
            if (cur.valid[r] && lane == r) {
                if (a.epi == EP_ADD) a.out_f32[cur.rows[r]] = a.out_f32[cur.rows[r]] + y[r];
                else a.out_f32[cur.rows[r]] = y[r];
            }
        }
    }
}

// The GEMV.  Blocks of 256 threads (4 waves x RW rows) walk the row blocks
// with a grid stride; the next row block's weights are requested before the
// current one is reduced.
template <int KIND, int RW, int U>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
    using T = KindTraits<KIND>;
    extern __shared__ uint4 xs[];
    __shared__ float red[4];
    __shared__ unsigned long long bkey[4];
    __shared__ int last_block;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int nchunks = a.K / T::E;
    const size_t row_bytes = (size_t)a.K * T::EB2 / 2;
    const long slots = (long)a.n_units * a.unit_rows;
    const int nblk = (int)((slots + 4L * RW - 1) / (4L * RW));
    const bool single = nchunks <= 64 * U;

    int blk = blockIdx.x;
    RowSet<KIND, RW, U> rs;
    uint4 wv[RW][U];
    if (blk < nblk) {
        rs.init(a, blk, wave);
        rs.load(a, row_bytes, nchunks, 0, lane, wv);
    }
    build_x<T::XF32>(a, xs, red);

    unsigned long long best = 0ull;
    for (; blk < nblk; blk += gridDim.x) {
        float acc[RW];
#pragma unroll
        for (int r = 0; r < RW; r++) acc[r] = 0.0f;
        for (int base = 0; base < nchunks; base += 64 * U) {
            if (base > 0) rs.load(a, row_bytes, nchunks, base, lane, wv);
#pragma unroll
            for (int r = 0; r < RW; r++)
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const int j = base + u * 64 + lane;
                    if (j < nchunks) acc[r] = chunk_dot<KIND>(wv[r][u], xs, j, acc[r]);
                }
        }
        RowSet<KIND, RW, U> cur = rs;
        const int nb = blk + gridDim.x;
        if (nb < nblk) {                    // request the next row block now
            rs.init(a, nb, wave);
            if (single) rs.load(a, row_bytes, nchunks, 0, lane, wv);
        }

        float y[RW];
#pragma unroll
        for (int r = 0; r < RW; r++) {
            y[r] = wave_sum_dpp(acc[r]);
            if (a.scale && cur.valid[r]) y[r] = y[r] * cur.sc[r];
        }
        store_rows<KIND, RW, U>(a, cur, y, lane);
        if (a.epi == EP_LOGITS) {
#pragma unroll
            for (int r = 0; r < RW; r++) {
                if (cur.valid[r]) {
                    const unsigned long long k = ref_argmax_key(y[r], cur.rows[r]);
                    if (k > best) best = k;
                }
            }
        }
        if (!single && nb < nblk) rs.load(a, row_bytes, nchunks, 0, lane, wv);
    }

    if (a.epi == EP_LOGITS) {
        if (lane == 0) bkey[wave] = best;
        __syncthreads();
        if (tid == 0) {
            unsigned long long b = bkey[0];
            for (int w = 1; w < 4; w++) b = bkey[w] > b ? bkey[w] : b;
            // device-scope atomics throughout, the maximum completed before
            // the arrival is counted: no cache write-back is needed
            if (b) __hip_atomic_fetch_max(a.amax_key, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);
            const unsigned prev = __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_block = prev == gridDim.x - 1;
        }
        __syncthreads();
        if (last_block && tid == 0) {
            const unsigned long long k = atomicExch(a.amax_key, 0ull);
            atomicExch(a.done, 0u);
            const int tok = ref_argmax_index(k);
            mdx_state* st = a.st;
            st->argmax = tok;
            st->token = tok;
            st->mode = 0;
            if (a.out_tokens) {
                a.out_tokens[st->n_out] = tok;
                st->n_out = st->n_out + 1;
            }
            st->pos = st->pos + a.advance;
        }
    }
}

// The GEMV when every workgroup takes exactly one row block and a lane's
// loads cover the whole row in one round (K <= 64 * U * E): the same weight
// requests, staging and sums as k_gemv, in a straight-line kernel without
// the grid-stride loop and the argmax tail.  A launch this small is bound by
// its fixed costs (dispatch and one HBM round trip), and the shorter code
// leaves fewer instruction-cache lines to fetch after the launch.
template <int KIND, int RW, int U>
__global__ __launch_bounds__(256) void k_gemv_once(GemvArgs a) {
    using T = KindTraits<KIND>;
    extern __shared__ uint4 xs[];
    __shared__ float red[4];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int nchunks = a.K / T::E;
    const size_t row_bytes = (size_t)a.K * T::EB2 / 2;
    RowSet<KIND, RW, U> rs;
    uint4 wv[RW][U];
    rs.init(a, blockIdx.x, wave);
    // x first, then the weights: staging x waits for x alone while the
    // weights arrive (config 2's four launches 17.51 -> 17.14 us, the INT8
    // 1 x 1024 x 4096 tile 3.02 -> 2.97 us)
    XFirst xf;
    build_x_first(a, xf);
    rs.load(a, row_bytes, nchunks, 0, lane, wv);
    build_x<T::XF32>(a, xs, red, &xf);
    float y[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        float acc = 0.0f;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = u * 64 + lane;
            if (j < nchunks) acc = chunk_dot<KIND>(wv[r][u], xs, j, acc);
        }
        y[r] = wave_sum_dpp(acc);
        if (a.scale && rs.valid[r]) y[r] = y[r] * rs.sc[r];
    }
    store_rows<KIND, RW, U>(a, rs, y, lane);
}

// INT8 lm_head with K = 1024 (one 16-byte chunk per lane is a whole row):
// block b streams rows [b*N/grid, (b+1)*N/grid); each wave takes batches of
// 16 rows, 4 batches apart, with three batches in registers (two in flight
// while one is multiplied).  x = fp16(RMSNorm(hidden)).  Each block stores its
// argmax key; arrival is counted in 8 group counters (so no single address
// takes all the atomics) and the last block reduces the keys and does the
// step bookkeeping of k_gemv's EP_LOGITS.
constexpr int kLmRows = 16;
constexpr int kLmBlocks = 256;
constexpr int kLmGroups = 8;
__global__ __launch_bounds__(256) void k_lmhead_i8_1k(GemvArgs a) {
    constexpr int U = kLmRows;
    constexpr int PER = 64 / U;
    __shared__ uint4 xs[128];
    __shared__ float red[4];
    __shared__ unsigned long long bkey[4];
    __shared__ int last_block;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int rb = (int)(((long long)blockIdx.x * a.N) / gridDim.x);
    const int re = (int)(((long long)(blockIdx.x + 1) * a.N) / gridDim.x);
    auto load = [&](uint4 (&w)[U], float& sc, int base) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int r = min(base + u, re - 1);
            w[u] = *reinterpret_cast<const uint4*>(a.w + (size_t)r * 1024 + lane * 16);
        }
        sc = a.scale ? a.scale[min(base + lane / PER, re - 1)] : 1.0f;
    };
    uint4 w0[U], w1[U], w2[U];
    float sc0 = 0.0f, sc1 = 0.0f, sc2 = 0.0f;
    const int first = rb + wave * U;
    if (first < re) load(w0, sc0, first);
    if (first + 4 * U < re) load(w1, sc1, first + 4 * U);
    build_x<false>(a, xs, red);
    __syncthreads();
    const uint4 x0 = xs[2 * lane], x1 = xs[2 * lane + 1];
    unsigned long long best = 0ull;
    auto consume = [&](const uint4 (&w)[U], float sc, int base) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = dot16_i8(w[u], x0, x1, 0.0f);
        const float tot = reduce_scatter<U, 64>(v, lane);
        const int r = base + lane / PER;
        if ((lane % PER) == 0 && r < re) {
            const float y = tot * sc;
            a.out_f32[r] = y;
            const unsigned long long k = ref_argmax_key(y, r);
            best = k > best ? k : best;
        }
    };
    for (int base = first; base < re; base += 12 * U) {
        if (base + 8 * U < re) load(w2, sc2, base + 8 * U);
        consume(w0, sc0, base);
        if (base + 4 * U >= re) break;
        if (base + 12 * U < re) load(w0, sc0, base + 12 * U);
        consume(w1, sc1, base + 4 * U);
        if (base + 8 * U >= re) break;
        if (base + 16 * U < re) load(w1, sc1, base + 16 * U);
        consume(w2, sc2, base + 8 * U);
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const unsigned lo = __shfl_xor((unsigned)(best & 0xffffffffull), off, 64);
        const unsigned hi = __shfl_xor((unsigned)(best >> 32), off, 64);
        const unsigned long long k = ((unsigned long long)hi << 32) | lo;
        best = k > best ? k : best;
    }
    if (lane == 0) bkey[wave] = best;
    __syncthreads();
    // scratch: [16, 48) group counters, [48, 52) group-done counter, [64, ...) keys
    unsigned* cnt = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(a.amax_key) + 16);
    unsigned* top = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(a.amax_key) + 48);
    unsigned long long* keys = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(a.amax_key) + 64);
    if (tid == 0) {
        unsigned long long bk = bkey[0];
        for (int w = 1; w < 4; w++) bk = bkey[w] > bk ? bkey[w] : bk;
        // the key goes out with a device-scope store that completes before
        // the arrival is counted, and the last block reads the keys with
        // device-scope loads: no cache write-back or invalidate is needed
        __hip_atomic_store(&keys[blockIdx.x], bk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        const int grp = blockIdx.x % kLmGroups;
        const unsigned in_grp = (gridDim.x - grp + kLmGroups - 1) / kLmGroups;
        int last = 0;
        if (__hip_atomic_fetch_add(&cnt[grp], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == in_grp - 1)
            last = __hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kLmGroups - 1;
        last_block = last;
    }
    __syncthreads();
    if (last_block) {
        unsigned long long k = 0ull;
        for (int i = tid; i < (int)gridDim.x; i += 256) {
            const unsigned long long v = __hip_atomic_load(&keys[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            k = v > k ? v : k;
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const unsigned lo = __shfl_xor((unsigned)(k & 0xffffffffull), off, 64);
            const unsigned hi = __shfl_xor((unsigned)(k >> 32), off, 64);
            const unsigned long long k2 = ((unsigned long long)hi << 32) | lo;
            k = k2 > k ? k2 : k;
        }
        if (lane == 0) bkey[wave] = k;
        __syncthreads();
        if (tid < kLmGroups) __hip_atomic_store(&cnt[tid], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (last_block && tid == 0) {
        unsigned long long k = bkey[0];
        for (int w = 1; w < 4; w++) k = bkey[w] > k ? bkey[w] : k;
        __hip_atomic_store(top, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int tok = ref_argmax_index(k);
        mdx_state* st = a.st;
        st->argmax = tok;
        st->token = tok;
        st->mode = 0;
        if (a.out_tokens) {
            a.out_tokens[st->n_out] = tok;
            st->n_out = st->n_out + 1;
        }
        st->pos = st->pos + a.advance;
    }
}

typedef void (*GemvKernel)(GemvArgs);

// The instantiated shapes: RW = 1 or 2 rows per wave with U = 1, 2, 3, 4, 6
// or 8 chunks per lane, and RW = 8 with U = 1 or 2 (RW * U <= 16, the
// choices of rows_per_wave_for and pick_u).  ONCE selects k_gemv_once.
template <int KIND, bool ONCE, int RW, int U>
constexpr GemvKernel gemv_fn() {
    if constexpr (ONCE) return k_gemv_once<KIND, RW, U>;
    else return k_gemv<KIND, RW, U>;
}

template <int KIND, bool ONCE, int RW>
GemvKernel pick_u_kernel(int u) {
    if constexpr (RW == 8) {
        return u == 1 ? gemv_fn<KIND, ONCE, 8, 1>() : gemv_fn<KIND, ONCE, 8, 2>();
    } else {
        switch (u) {
            case 1: return gemv_fn<KIND, ONCE, RW, 1>();
            case 2: return gemv_fn<KIND, ONCE, RW, 2>();
            case 3: return gemv_fn<KIND, ONCE, RW, 3>();
            case 4: return gemv_fn<KIND, ONCE, RW, 4>();
            case 6: return gemv_fn<KIND, ONCE, RW, 6>();
            default: return gemv_fn<KIND, ONCE, RW, 8>();
        }
    }
}

template <int KIND, bool ONCE>
GemvKernel pick_kernel(int rw, int u) {
    switch (rw) {
        case 1: return pick_u_kernel<KIND, ONCE, 1>(u);
        case 2: return pick_u_kernel<KIND, ONCE, 2>(u);
        default: return pick_u_kernel<KIND, ONCE, 8>(u);
    }
}

template <bool ONCE>
GemvKernel pick_kind(int kind, int rw, int u) {
    switch (kind) {
        case KF16: return pick_kernel<KF16, ONCE>(rw, u);
        case KI8: return pick_kernel<KI8, ONCE>(rw, u);
        case KI4: return pick_kernel<KI4, ONCE>(rw, u);
        case KF32X: return pick_kernel<KF32X, ONCE>(rw, u);
        default: return pick_kernel<KF16X, ONCE>(rw, u);
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

// chunks per lane per round: the smallest of {1,2,3,4,6,8} covering the row,
// with at most 16 outstanding 16-byte loads per lane (RW*U <= 16).
int pick_u(int nchunks, int rw) {
    static const int opts[6] = {1, 2, 3, 4, 6, 8};
    const int need = (nchunks + 63) / 64;
    int cap = 16 / rw;
    int best = 1;
    for (int i = 0; i < 6; i++) {
        if (opts[i] > cap) break;
        best = opts[i];
        if (opts[i] >= need) break;
    }
    return best;
}

// One row per wave up to 4096 rows (more blocks: an INT8 1024 x 4096 GEMV
// takes 3.9 us against 4.1 us with two rows per wave).
int rows_per_wave_for(int rows) {
    if (rows >= 65536) return 8;
    if (rows > 4096) return 2;
    return 1;
}

int launch_gemv(int kind, GemvArgs a, int rw, int max_grid, void* stream) {
    const int E = elems_per_chunk(kind);
    if (a.K <= 0 || a.K % E != 0 || a.n_units <= 0) return -1;
    if (rw != 1 && rw != 2 && rw != 8) return -1;   // the instantiated row counts
    const int nchunks = a.K / E;
    const int u = pick_u(nchunks, rw);
    const long slots = (long)a.n_units * a.unit_rows;
    long grid = (slots + 4L * rw - 1) / (4L * rw);
    if (max_grid > 0 && grid > max_grid) grid = max_grid;
    const bool xf32 = kind == KF32X || kind == KF16X;
    const size_t lds = (size_t)a.K * (xf32 ? 4 : 2);
    if (lds > 64 * 1024) return -5;
    // one row block per workgroup and one round of loads per row: the
    // straight-line kernel
    const long nblk = (slots + 4L * rw - 1) / (4L * rw);
    const bool once = a.epi != EP_LOGITS && grid == nblk && nchunks <= 64 * u;
    GemvKernel k = once ? pick_kind<true>(kind, rw, u) : pick_kind<false>(kind, rw, u);
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

GemvArgs base_args(const mdx_wdesc* w) {
    GemvArgs a = {};
    a.w = (const uint8_t*)w->w;
    a.scale = w->scale;
    a.K = w->K;
    a.N = w->N;
    a.n_units = w->N;
    a.unit_rows = 1;
    return a;
}

// ---- attention ---------------------------------------------------------------

struct AttnArgs {
    const mdx_state* st;
    const float* qkv;         // [nq*hd | nkv*hd | nkv*hd] fp32 projection output
    const float* q_norm;
    const float* k_norm;
    float eps;
    const float* cos_t;
    const float* sin_t;
    int style;
    uint16_t* kc;             // layer cache [max_seq][nkv*hd] fp16
    uint16_t* vc;
    int nkv;
    int max_splits;
    int chunk_cap;
    float* part;              // [nkv][max_splits][G][hd + 4]
    unsigned int* done;       // [nkv], zero between launches
    uint16_t* out16;          // [nq*hd]
};

// Splits of up to kAttnChunk positions (more when L exceeds max_splits of
// them): fewer split records to merge, and a block's tiles are requested
// together (k_attn_decode issues its first kAttnPf tiles before anything else).
constexpr int kAttnChunk = 64, kAttnPf = 4;
__device__ __forceinline__ void attn_plan(int L, int max_splits, int& splits, int& chunk) {
    int s = (L + kAttnChunk - 1) / kAttnChunk;
    if (s > max_splits) s = max_splits;
    chunk = (L + s - 1) / s;
    splits = (L + chunk - 1) / chunk;
}

// Per-head RMSNorm (optional) + RoPE of one head vector, one wave.  Writes the
// rotated fp32 values to dst (LDS) and, when cache != NULL, their fp16
// roundings to cache (and the rounded values to dst, the fp16 KV semantic).
// hd <= 256: a lane holds elements lane + 64k (k < 4) for the sum of squares
// (summed in that order) and pairs i = lane + 64k (k < 2); every load is
// issued before the first is used (indexes clamped into the head).
__device__ __forceinline__ void rope_head(const float* src, const float* nw, float eps,
                                          const float* cr, const float* sr, int hd, int style,
                                          float* dst, uint16_t* cache, int lane) {
    const int half = hd / 2;
    float xe[4], x0[2], x1[2], w0[2], w1[2], cv[2], sv[2];
#pragma unroll
    for (int k = 0; k < 4; k++) xe[k] = src[min(lane + 64 * k, hd - 1)];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int i = min(lane + 64 * k, half - 1);
        const int i0 = style == 0 ? 2 * i : i;
        const int i1 = style == 0 ? 2 * i + 1 : i + half;
        x0[k] = src[i0];
        x1[k] = src[i1];
        w0[k] = nw ? nw[i0] : 1.0f;
        w1[k] = nw ? nw[i1] : 1.0f;
        cv[k] = cr[i];
        sv[k] = sr[i];
    }
    float rms = 1.0f;
    if (nw) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (lane + 64 * k < hd) ss += xe[k] * xe[k];
        ss = wave_sum(ss);
        rms = 1.0f / sqrtf(ss / (float)hd + eps);
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int i = lane + 64 * k;
        if (i >= half) break;
        const int i0 = style == 0 ? 2 * i : i;
        const int i1 = style == 0 ? 2 * i + 1 : i + half;
        float a0 = x0[k], a1 = x1[k];
        if (nw) {
            a0 = (a0 * rms) * w0[k];
            a1 = (a1 * rms) * w1[k];
        }
        const float c = cv[k], sn = sv[k];
        float o0 = a0 * c - a1 * sn;
        float o1 = a1 * c + a0 * sn;
        if (cache) {
            const uint16_t h0 = f32_to_f16_bits(o0), h1 = f32_to_f16_bits(o1);
            cache[i0] = h0;
            cache[i1] = h1;
            o0 = f16_bits_to_f32(h0);
            o1 = f16_bits_to_f32(h1);
        }
        dst[i0] = o0;
        dst[i1] = o1;
    }
}

// grid = (nkv, max_splits), 256 threads.  Block (h, s) covers positions
// [s*chunk, min(L, (s+1)*chunk)) of KV head h for its G query heads.
template <int HD, int G>
__global__ __launch_bounds__(256) void k_attn_decode(AttnArgs a) {
    constexpr int LP = HD / 8;          // lanes per position (16-byte chunks)
    constexpr int PPW = 64 / LP;        // positions per wave per tile
    constexpr int TILE = 4 * PPW;       // positions per tile
    constexpr int PG = 256 / LP;        // position groups in P.V
    constexpr int GD4 = G * HD / 4;     // float4 slices of the G output heads
    constexpr int SG = 256 / GD4 > 0 ? 256 / GD4 : 1;   // split groups in the merge
    extern __shared__ float smem[];
    float* qs = smem;                   // [G][HD]
    float* kn = qs + G * HD;            // [HD] newest K (fp16-rounded)
    float* vn = kn + HD;                // [HD] newest V (fp16-rounded)
    float* sc = vn + HD;                // [G][chunk_cap]
    __shared__ float ml[2 * G];
    __shared__ int is_last;

    const int pos = a.st->pos;
    const int L = pos + 1;
    int splits, chunk;
    attn_plan(L, a.max_splits, splits, chunk);
    const int s = blockIdx.y;
    if (s >= splits) return;
    const int kvh = blockIdx.x;
    const int p0 = s * chunk;
    const int p1 = min(L, p0 + chunk);
    const int n = p1 - p0;
    const bool has_new = p1 == L;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nq = a.nkv * G, qd = nq * HD, kvd = a.nkv * HD;
    const int half = HD / 2;
    const float scale = 1.0f / sqrtf((float)HD);
    const int sub = lane % LP, slot = lane / LP;
    const int dsub = tid % LP, pg = tid / LP;

    // the first kAttnPf K tiles and V position groups: the cache loads are
    // issued before anything else (the newest row, pos, comes from LDS)
    uint4 kpre[kAttnPf], vpre[kAttnPf];
#pragma unroll
    for (int t = 0; t < kAttnPf; t++) {
        const int pik = t * TILE + wave * PPW + slot, piv = t * PG + pg;
        kpre[t] = make_uint4(0, 0, 0, 0);
        vpre[t] = make_uint4(0, 0, 0, 0);
        if (pik < n && p0 + pik < pos)
            kpre[t] = *reinterpret_cast<const uint4*>(a.kc + (size_t)(p0 + pik) * kvd + kvh * HD + sub * 8);
        if (piv < n && p0 + piv < pos)
            vpre[t] = *reinterpret_cast<const uint4*>(a.vc + (size_t)(p0 + piv) * kvd + kvh * HD + dsub * 8);
    }

    // QK-norm + RoPE of the G query heads (every block), and of the newest
    // K/V row (the block that holds position pos, which also appends it)
    const float* cr = a.cos_t + (size_t)pos * half;
    const float* sr = a.sin_t + (size_t)pos * half;
    for (int t = wave; t < G + 2; t += 4) {
        if (t < G) {
            rope_head(a.qkv + (size_t)(kvh * G + t) * HD, a.q_norm, a.eps, cr, sr, HD, a.style,
                      qs + t * HD, nullptr, lane);
        } else if (has_new && t == G) {
            rope_head(a.qkv + qd + kvh * HD, a.k_norm, a.eps, cr, sr, HD, a.style, kn,
                      a.kc + (size_t)pos * kvd + kvh * HD, lane);
        } else if (has_new) {
            const float* src = a.qkv + qd + kvd + kvh * HD;
            uint16_t* dst = a.vc + (size_t)pos * kvd + kvh * HD;
            for (int e = lane; e < HD; e += 64) {
                const uint16_t hv = f32_to_f16_bits(src[e]);
                dst[e] = hv;
                vn[e] = f16_bits_to_f32(hv);
            }
        }
    }
    __syncthreads();

    // scores: tile t0 (positions t0 .. t0 + TILE - 1 of the split)
    auto score_tile = [&](int t0, uint4 kv) {
        const int pi = t0 + wave * PPW + slot;
        const bool act = pi < n;
        const int p = p0 + pi;
        float kf[8];
        if (act && p == pos) {
#pragma unroll
            for (int e = 0; e < 8; e++) kf[e] = kn[sub * 8 + e];
        } else {
            const half2_t k01 = as_h2(kv.x), k23 = as_h2(kv.y), k45 = as_h2(kv.z), k67 = as_h2(kv.w);
            kf[0] = (float)k01.x; kf[1] = (float)k01.y; kf[2] = (float)k23.x; kf[3] = (float)k23.y;
            kf[4] = (float)k45.x; kf[5] = (float)k45.y; kf[6] = (float)k67.x; kf[7] = (float)k67.y;
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float* qq = qs + g * HD + sub * 8;
            float pd = qq[0] * kf[0];
#pragma unroll
            for (int e = 1; e < 8; e++) pd = pd + qq[e] * kf[e];
            if constexpr (LP == 16) pd = row_sum16(pd);   // DPP within the 16-lane row
            else pd = group_sum(pd, LP);
            if (act && sub == 0) sc[g * a.chunk_cap + pi] = pd * scale;
        }
    };
#pragma unroll
    for (int t = 0; t < kAttnPf; t++)
        if (t * TILE < n) score_tile(t * TILE, kpre[t]);
    for (int t0 = kAttnPf * TILE; t0 < n; t0 += TILE) {
        const int pi = t0 + wave * PPW + slot;
        uint4 kv = make_uint4(0, 0, 0, 0);
        if (pi < n && p0 + pi < pos) kv = *reinterpret_cast<const uint4*>(a.kc + (size_t)(p0 + pi) * kvd + kvh * HD + sub * 8);
        score_tile(t0, kv);
    }
    __syncthreads();

    for (int g = wave; g < G; g += 4) {
        float m = -1e30f;
        for (int i = lane; i < n; i += 64) m = fmaxf(m, sc[g * a.chunk_cap + i]);
        m = wave_max_dpp(m);
        float l = 0.0f;
        for (int i = lane; i < n; i += 64) {
            const float e = expf(sc[g * a.chunk_cap + i] - m);
            sc[g * a.chunk_cap + i] = e;
            l += e;
        }
        l = wave_sum_dpp(l);
        if (lane == 0) {
            ml[2 * g] = m;
            ml[2 * g + 1] = l;
        }
    }
    __syncthreads();

    // P.V: thread = (position group, 8-wide slice of the head dimension)
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.0f;
    auto pv_row = [&](int pi, uint4 vv) {
        const int p = p0 + pi;
        float vf[8];
        if (p == pos) {
#pragma unroll
            for (int e = 0; e < 8; e++) vf[e] = vn[dsub * 8 + e];
        } else {
            const half2_t v01 = as_h2(vv.x), v23 = as_h2(vv.y), v45 = as_h2(vv.z), v67 = as_h2(vv.w);
            vf[0] = (float)v01.x; vf[1] = (float)v01.y; vf[2] = (float)v23.x; vf[3] = (float)v23.y;
            vf[4] = (float)v45.x; vf[5] = (float)v45.y; vf[6] = (float)v67.x; vf[7] = (float)v67.y;
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float pw = sc[g * a.chunk_cap + pi];
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] = acc[g][e] + vf[e] * pw;
        }
    };
#pragma unroll
    for (int t = 0; t < kAttnPf; t++)
        if (t * PG + pg < n) pv_row(t * PG + pg, vpre[t]);
    for (int pi = kAttnPf * PG + pg; pi < n; pi += PG)
        pv_row(pi, *reinterpret_cast<const uint4*>(a.vc + (size_t)(p0 + pi) * kvd + kvh * HD + dsub * 8));
    __syncthreads();   // scores no longer needed: smem is reused for the cross-group sum
    float* red = smem; // [PG][G][HD]
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) red[(pg * G + g) * HD + dsub * 8 + e] = acc[g][e];
    __syncthreads();
    if (splits == 1) {
        // the only split: its sums are final (the merge of one record
        // computes the same quotient), so no record, arrival or merge
        for (int i = tid; i < G * HD; i += 256) {
            const int g = i / HD, d = i % HD;
            float sum = 0.0f;
            for (int k = 0; k < PG; k++) sum += red[(k * G + g) * HD + d];
            a.out16[(size_t)(kvh * G + g) * HD + d] = f32_to_f16_bits(sum / ml[2 * g + 1]);
        }
        return;
    }
    // The split's record ([G][HD + 4] floats: the HD sums, then m, l and two
    // unused words, so every head starts on 16 bytes) goes out as 16-byte
    // stores with the sc1 policy (what an agent-scope atomic store compiles
    // to: past the per-XCD L2s); each thread waits for its own stores, and
    // only then is the arrival counted (agent-scope atomic).  The last block
    // reads the records with 16-byte sc1 loads.  No cache write-back or
    // invalidate is needed.
    constexpr int RH = HD + 4;              // floats per head in a record
    const auto prs = __builtin_amdgcn_make_buffer_rsrc(a.part, (short)0, 0x7fffffff, 0x00020000);
    const unsigned rec0 = (unsigned)(((size_t)kvh * a.max_splits + s) * G * RH * 4);
    for (int i4 = tid; i4 < G * HD / 4; i4 += 256) {
        const int g = (4 * i4) / HD, d = (4 * i4) % HD;
        float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int k = 0; k < PG; k++) {
            const float4 r = *reinterpret_cast<const float4*>(red + (k * G + g) * HD + d);
            sum.x += r.x; sum.y += r.y; sum.z += r.z; sum.w += r.w;
        }
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, sum), prs,
                                               rec0 + (unsigned)(g * RH + d) * 4, 0, 16);
    }
    if (tid < G) {
        const float4 t4 = make_float4(ml[2 * tid], ml[2 * tid + 1], 0.f, 0.f);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, t4), prs,
                                               rec0 + (unsigned)(tid * RH + HD) * 4, 0, 16);
    }

    // the last block of this KV head merges all splits
    wait_all();
    __syncthreads();
    if (tid == 0)
        is_last = __hip_atomic_fetch_add(&a.done[kvh], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                  (unsigned)(splits - 1);
    __syncthreads();
    if (!is_last) return;
    const unsigned base = (unsigned)((size_t)kvh * a.max_splits * G * RH * 4);
    const unsigned stride = (unsigned)(G * RH * 4);
    float m = -INFINITY, l = 0.0f, o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int gd = tid % GD4, sg = tid / GD4;
    const int g = gd / (HD / 4), d4 = (gd % (HD / 4)) * 4;
    if (sg < SG) {
        // records sp = sg, sg + SG, ... merged in that order; the loads of a
        // batch of kMergeB records are issued before the first is used
        constexpr int kMergeB = 12;
        for (int sp0 = sg; sp0 < splits; sp0 += kMergeB * SG) {
            u32x4_t ml4[kMergeB], os4[kMergeB];
#pragma unroll
            for (int j = 0; j < kMergeB; j++) {
                const int sp = min(sp0 + j * SG, splits - 1);
                const unsigned ps = base + (unsigned)sp * stride + (unsigned)(g * RH) * 4;
                ml4[j] = __builtin_amdgcn_raw_buffer_load_b128(prs, ps + HD * 4, 0, 16);
                os4[j] = __builtin_amdgcn_raw_buffer_load_b128(prs, ps + (unsigned)d4 * 4, 0, 16);
            }
#pragma unroll
            for (int j = 0; j < kMergeB; j++) {
                if (sp0 + j * SG >= splits) break;
                const float msj = __uint_as_float(ml4[j].x), lsj = __uint_as_float(ml4[j].y);
                const float mn = fmaxf(m, msj);
                const float fa = expf(m - mn), fb = expf(msj - mn);
                l = l * fa + lsj * fb;
                o[0] = o[0] * fa + __uint_as_float(os4[j].x) * fb;
                o[1] = o[1] * fa + __uint_as_float(os4[j].y) * fb;
                o[2] = o[2] * fa + __uint_as_float(os4[j].z) * fb;
                o[3] = o[3] * fa + __uint_as_float(os4[j].w) * fb;
                m = mn;
            }
        }
    }
    __syncthreads();
    float* mr = smem;                       // [SG][GD4][6]
    if (sg < SG) {
        float* r = mr + (sg * GD4 + gd) * 6;
        r[0] = m; r[1] = l; r[2] = o[0]; r[3] = o[1]; r[4] = o[2]; r[5] = o[3];
    }
    __syncthreads();
    if (sg == 0) {
        float M = -INFINITY;
        for (int k = 0; k < SG; k++) M = fmaxf(M, mr[(k * GD4 + gd) * 6]);
        float Ls = 0.0f, O[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int k = 0; k < SG; k++) {
            const float* r = mr + (k * GD4 + gd) * 6;
            if (r[0] == -INFINITY) continue;
            const float f = expf(r[0] - M);
            Ls = Ls + r[1] * f;
            for (int e = 0; e < 4; e++) O[e] = O[e] + r[2 + e] * f;
        }
        uint16_t* dst = a.out16 + (size_t)(kvh * G + g) * HD + d4;
        for (int e = 0; e < 4; e++) dst[e] = f32_to_f16_bits(O[e] / Ls);
    }
    if (tid == 0) __hip_atomic_store(&a.done[kvh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void k_advance(mdx_state* st, int advance) {
    if (threadIdx.x == 0) st->pos = st->pos + advance;
}

}  // namespace

extern "C" {

int mdx_launch_norm_gemv(const float* hidden, const float* norm_w, float eps, const mdx_wdesc* w,
                         int epilogue, void* out, void* stream) {
    GemvArgs a = base_args(w);
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
        a.epi = EP_STORE;
        a.out_f32 = (float*)out;
    }
    const int kind = kind_from(w, 0);
    int rw = rows_per_wave_for(a.n_units * a.unit_rows);
    if (a.unit_rows == 2 && rw < 2) rw = 2;
    return launch_gemv(kind, a, rw, 0, stream);
}

int mdx_launch_embed_norm_gemv(const mdx_state* state, const float* emb_table, const float* emb_in,
                               int vocab, float* hidden, const float* norm_w, float eps,
                               const mdx_wdesc* w, float* out, void* stream) {
    GemvArgs a = base_args(w);
    a.xmode = XM_EMBED;
    a.st_in = state;
    a.emb_table = emb_table;
    a.xf32 = emb_in;
    a.vocab = vocab;
    a.hidden_out = hidden;
    a.norm_w = norm_w;
    a.eps = eps;
    a.epi = EP_STORE;
    a.out_f32 = out;
    const int kind = kind_from(w, 0);
    return launch_gemv(kind, a, rows_per_wave_for(w->N), 0, stream);
}

int mdx_launch_gemv_add(const uint16_t* x16, const mdx_wdesc* w, float* out, void* stream) {
    GemvArgs a = base_args(w);
    a.xmode = XM_F16;
    a.x16 = x16;
    a.epi = EP_ADD;
    a.out_f32 = out;
    const int kind = kind_from(w, 0);
    return launch_gemv(kind, a, rows_per_wave_for(a.N), 0, stream);
}

int mdx_launch_gemv_f16in(const uint16_t* x16, const mdx_wdesc* w, float* y, void* stream) {
    GemvArgs a = base_args(w);
    a.xmode = XM_F16;
    a.x16 = x16;
    a.epi = EP_STORE;
    a.out_f32 = y;
    const int kind = kind_from(w, 0);
    return launch_gemv(kind, a, rows_per_wave_for(a.N), 0, stream);
}

int mdx_launch_gemv(const float* x, const mdx_wdesc* w, int x_fp32_exact, float* y, void* stream) {
    GemvArgs a = base_args(w);
    a.xmode = XM_F32;
    a.xf32 = x;
    a.epi = EP_STORE;
    a.out_f32 = y;
    const int kind = kind_from(w, x_fp32_exact);
    return launch_gemv(kind, a, rows_per_wave_for(a.N), 0, stream);
}

size_t mdx_lmhead_scratch_bytes(void) { return 64 + 8 * kLmBlocks; }

int mdx_launch_lmhead(const float* hidden, const float* norm_w, float eps, const mdx_wdesc* w,
                      float* logits, void* scratch, mdx_state* state, int* out_tokens, int advance,
                      void* stream) {
    GemvArgs a = base_args(w);
    a.xmode = XM_NORM;
    a.xf32 = hidden;
    a.norm_w = norm_w;
    a.eps = eps;
    a.epi = EP_LOGITS;
    a.out_f32 = logits;
    a.amax_key = (unsigned long long*)scratch;
    a.done = (unsigned int*)((char*)scratch + 8);
    a.st = state;
    a.out_tokens = out_tokens;
    a.advance = advance;
    // fp16 rows take fp32 activations here (the reference's CPU lm_head)
    const int kind = kind_from(w, 1);
    if (kind == KI8 && w->K == 1024 && w->N >= kLmBlocks * kLmRows) {
        hipLaunchKernelGGL(k_lmhead_i8_1k, dim3(kLmBlocks), dim3(256), 0, (hipStream_t)stream, a);
        return hipGetLastError() == hipSuccess ? 0 : -4;
    }
    return launch_gemv(kind, a, rows_per_wave_for(w->N), 1024, stream);
}

int mdx_launch_advance(mdx_state* state, int advance, void* stream) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, (hipStream_t)stream, state, advance);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int mdx_attn_max_splits(int max_seq) {
    (void)max_seq;
    return 64;
}

size_t mdx_attn_decode_scratch_bytes(int nq, int nkv, int hd, int max_splits) {
    return (size_t)nq * max_splits * (hd + 4) * 4 + (size_t)nkv * 4;
}

int mdx_launch_attn_decode(const mdx_state* state, const float* qkv, const float* q_norm,
                           const float* k_norm, float eps, const float* cos_t, const float* sin_t,
                           int rope_style, int nq, int nkv, int hd, int max_seq, int max_splits,
                           uint16_t* k_cache, uint16_t* v_cache, void* scratch, uint16_t* attn_out16,
                           void* stream) {
    if (nkv <= 0 || nq % nkv || max_splits <= 0 || hd % 8) return -1;
    const int G = nq / nkv;
    AttnArgs a;
    a.st = state;
    a.qkv = qkv;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.eps = eps;
    a.cos_t = cos_t;
    a.sin_t = sin_t;
    a.style = rope_style;
    a.kc = k_cache;
    a.vc = v_cache;
    a.nkv = nkv;
    a.max_splits = max_splits;
    a.chunk_cap = (max_seq + max_splits - 1) / max_splits;
    if (a.chunk_cap < kAttnChunk) a.chunk_cap = kAttnChunk;
    a.part = (float*)scratch;
    a.done = (unsigned int*)((char*)scratch + (size_t)nq * max_splits * (hd + 4) * 4);
    a.out16 = attn_out16;
    const int LP = hd / 8;
    const int PG = 256 / LP;
    const size_t lds_a = (size_t)(G * hd + 2 * hd + G * a.chunk_cap) * 4;
    const size_t lds_b = (size_t)PG * G * hd * 4;
    const size_t lds_c = (size_t)256 * 6 * 4;
    size_t lds = lds_a > lds_b ? lds_a : lds_b;
    if (lds_c > lds) lds = lds_c;
    if (lds > 64 * 1024) return -5;
    dim3 grid(nkv, max_splits);
#define MDX_ATTN(HD_, G_)                                                                          \
    if (hd == HD_ && G == G_) {                                                                    \
        hipLaunchKernelGGL((k_attn_decode<HD_, G_>), grid, dim3(256), lds, (hipStream_t)stream, a); \
        return hipGetLastError() == hipSuccess ? 0 : -4;                                           \
    }
    MDX_ATTN(64, 1) MDX_ATTN(64, 2) MDX_ATTN(64, 4) MDX_ATTN(64, 8)
    MDX_ATTN(128, 1) MDX_ATTN(128, 2) MDX_ATTN(128, 4) MDX_ATTN(128, 8)
    MDX_ATTN(256, 1) MDX_ATTN(256, 2) MDX_ATTN(256, 4)
#undef MDX_ATTN
    return -5;
}

}  // extern "C"
