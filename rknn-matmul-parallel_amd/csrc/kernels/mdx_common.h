// mdx_common.h — device helpers shared by the gfx950 kernels.
//
// Conversions follow round-to-nearest-even (the hardware default mode).
// All code is compiled with -ffp-contract=off, so `a*b + c` rounds twice
// unless a fused builtin is written explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mdx {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

// Non-temporal 16-byte load, for data read once per step or per launch
// (weights streamed past the caches): it does not evict what is read again.
__device__ __forceinline__ uint4 ld_nt(const void* p) {
    typedef unsigned u32x4_nt __attribute__((ext_vector_type(4)));
    const u32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t h2_bits(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// Data exchanged between workgroups of one kernel goes through agent-coherent
// 32-bit accesses (relaxed agent-scope atomics): they bypass the per-XCD L2,
// so no device-wide cache write-back / invalidate (fence) is needed.  The
// writer waits for its stores to complete (wait_all) before it signals with
// an atomic; the reader only loads after it has observed that signal.
__device__ __forceinline__ void st_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_coherent_u32(const unsigned* p) {
    return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until every memory operation this thread issued has completed.
__device__ __forceinline__ void wait_all() { __builtin_amdgcn_s_waitcnt(0); }

// Sum over all 64 lanes; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Sum over aligned groups of `width` lanes (power of two <= 64).
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Cross-lane reductions with DPP moves (a few cycles each, unlike LDS-routed
// shuffles).  row_sum16: every lane of each 16-lane row gets the row's sum.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float row_sum16(float v) {
    v = v + dpp<0xB1>(v);    // quad_perm [1,0,3,2]
    v = v + dpp<0x4E>(v);    // quad_perm [2,3,0,1]
    v = v + dpp<0x124>(v);   // row_ror:4
    v = v + dpp<0x128>(v);   // row_ror:8
    return v;
}
// Sum over the 64 lanes, returned to every lane (through lane 63).
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = row_sum16(v);
    v = v + dpp<0x142, 0xA>(v);   // row_bcast:15 into rows 1, 3
    v = v + dpp<0x143, 0xC>(v);   // row_bcast:31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Maximum over the 64 lanes, returned to every lane (through lane 63).
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp<0xB1>(v));          // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp<0x4E>(v));          // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp<0x124>(v));         // row_ror:4
    v = fmaxf(v, dpp<0x128>(v));         // row_ror:8
    v = fmaxf(v, dpp<0x142, 0xA>(v));    // row_bcast:15 into rows 1, 3
    v = fmaxf(v, dpp<0x143, 0xC>(v));    // row_bcast:31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Lanes 0..31 only (lanes 32..63 are ignored), returned to every lane.
__device__ __forceinline__ float half_sum_dpp(float v) {
    v = row_sum16(v);
    v = v + dpp<0x142, 0xA>(v);   // row_bcast:15 into rows 1, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
}
__device__ __forceinline__ float half_max_dpp(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x124>(v));
    v = fmaxf(v, dpp<0x128>(v));
    v = fmaxf(v, dpp<0x142, 0xA>(v));   // row 1 (read below) takes row 0's maximum
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
}
// Sum / maximum over the four 16-lane rows of a wave, per column (lane & 15),
// returned to every lane: the gfx950 row swaps (odd rows of one operand with
// even rows of the other; upper half with lower half) run on the VALU.
__device__ __forceinline__ float rows_sum4(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}
__device__ __forceinline__ float rows_max4(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Argmax key of logit v at index idx, reproducing argmax_f32
// (src/cpu_ops.c:575-586: max starts at x[0], strict '>' over i = 1..n-1):
// the largest key wins, equal values pick the lower index, -0 and +0 are
// equal, a NaN never wins (key 0, which no number has) except at index 0,
// where the reference's running maximum starts and no later '>' can replace
// it, so it takes the largest key.
__device__ __forceinline__ unsigned long long ref_argmax_key(float v, int idx) {
    if (v != v) return idx == 0 ? ~0ull : 0ull;
    unsigned u = __float_as_uint(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)idx);
}
// The index a key was made from (0 for "no key").
__device__ __forceinline__ int ref_argmax_index(unsigned long long k) {
    return (k && k != ~0ull) ? (int)(0xFFFFFFFFu - (unsigned)(k & 0xFFFFFFFFull)) : 0;
}

// fp16 x fp16 products (exact in fp32) accumulated into fp32.
__device__ __forceinline__ float dot8_f16(uint4 w, uint4 x, float acc) {
    acc = __builtin_amdgcn_fdot2(as_h2(w.x), as_h2(x.x), acc, false);
    acc = __builtin_amdgcn_fdot2(as_h2(w.y), as_h2(x.y), acc, false);
    acc = __builtin_amdgcn_fdot2(as_h2(w.z), as_h2(x.z), acc, false);
    acc = __builtin_amdgcn_fdot2(as_h2(w.w), as_h2(x.w), acc, false);
    return acc;
}

// Four signed int8 (one word, k ascending from the low byte) -> two half2
// holding (q0,q1) and (q2,q3), exactly: (0x6400 | (q+128)) is 1024+q+128.
__device__ __forceinline__ void i8x4_to_h2x2(uint32_t w, half2_t& a, half2_t& b) {
    const uint32_t u = w ^ 0x80808080u;
    const half2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    a = as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
    b = as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
}

// One int4 word of the device layout (8 consecutive k, nibble pairs
// interleaved so that (w >> 4i) & 0x000f000f holds k=2i and k=2i+1) ->
// half2 (q_{2i}, q_{2i+1}) exactly: (0x6400 | (q+8)) is 1024+q+8.
__device__ __forceinline__ half2_t i4_pair(uint32_t u, int i) {
    const half2_t bias = {(_Float16)1032.0f, (_Float16)1032.0f};
    return as_h2(((u >> (4 * i)) & 0x000f000fu) | 0x64006400u) - bias;
}

__device__ __forceinline__ float dot16_i8(uint4 w, uint4 x0, uint4 x1, float acc) {
    half2_t a, b;
    i8x4_to_h2x2(w.x, a, b);
    acc = __builtin_amdgcn_fdot2(a, as_h2(x0.x), acc, false);
    acc = __builtin_amdgcn_fdot2(b, as_h2(x0.y), acc, false);
    i8x4_to_h2x2(w.y, a, b);
    acc = __builtin_amdgcn_fdot2(a, as_h2(x0.z), acc, false);
    acc = __builtin_amdgcn_fdot2(b, as_h2(x0.w), acc, false);
    i8x4_to_h2x2(w.z, a, b);
    acc = __builtin_amdgcn_fdot2(a, as_h2(x1.x), acc, false);
    acc = __builtin_amdgcn_fdot2(b, as_h2(x1.y), acc, false);
    i8x4_to_h2x2(w.w, a, b);
    acc = __builtin_amdgcn_fdot2(a, as_h2(x1.z), acc, false);
    acc = __builtin_amdgcn_fdot2(b, as_h2(x1.w), acc, false);
    return acc;
}

__device__ __forceinline__ float dot8_i4(uint32_t w, uint4 x, float acc) {
    const uint32_t u = w ^ 0x88888888u;
    acc = __builtin_amdgcn_fdot2(i4_pair(u, 0), as_h2(x.x), acc, false);
    acc = __builtin_amdgcn_fdot2(i4_pair(u, 1), as_h2(x.y), acc, false);
    acc = __builtin_amdgcn_fdot2(i4_pair(u, 2), as_h2(x.z), acc, false);
    acc = __builtin_amdgcn_fdot2(i4_pair(u, 3), as_h2(x.w), acc, false);
    return acc;
}

// Reference-style SiLU-gated product: g * (1 / (1 + expf(-g))) * u.
__device__ __forceinline__ float silu_mul(float g, float u) {
    float sig = 1.0f / (1.0f + expf(-g));
    return (g * sig) * u;
}

// The value of the partner lane at distance O (a symmetric pairing that
// flips lane bit log2(O) and keeps the higher bits): DPP within a 16-lane
// row, the gfx950 row swaps across rows.
template <int O>
__device__ __forceinline__ float partner(float v) {
    if constexpr (O == 1) return dpp<0xB1>(v);        // quad_perm [1,0,3,2]
    else if constexpr (O == 2) return dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    else if constexpr (O == 4) return dpp<0x141>(v);  // row_half_mirror: i <-> 7-i
    else return dpp<0x128>(v);                        // row_ror:8 (i <-> i^8)
}

// One butterfly step at distance O over nv live values: the lane with bit O
// clear keeps the low half, its partner the high half; each adds the other's
// copy of the half it keeps.
template <int O, int NV>
__device__ __forceinline__ void rs_step(float (&v)[NV], int nv, int lane) {
    const int half = nv / 2;
    if constexpr (O >= 16) {
        // row swaps: (lo, hi) -> (own lo, partner lo) below, (partner hi, own hi) above
#pragma unroll
        for (int k = 0; k < NV / 2; k++) {
            if (k < half) {
                if constexpr (O == 32) {
                    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[k]),
                                                                    __float_as_uint(v[k + half]), false, false);
                    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
                } else {
                    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]),
                                                                    __float_as_uint(v[k + half]), false, false);
                    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
                }
            }
        }
    } else {
        // bitwise select: keeps both reads static (a select of two array
        // elements would otherwise become a dynamically indexed read)
        const unsigned up = (lane & O) ? 0xffffffffu : 0u;
#pragma unroll
        for (int k = 0; k < NV / 2; k++) {
            if (k < half) {
                const unsigned lo = __float_as_uint(v[k]), hi = __float_as_uint(v[k + half]);
                const float send = __uint_as_float((lo & up) | (hi & ~up));
                const float keep = __uint_as_float((hi & up) | (lo & ~up));
                v[k] = keep + partner<O>(send);
            }
        }
    }
}
template <int O>
__device__ __forceinline__ float sum_step(float v) {
    if constexpr (O == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
        return v + partner<O>(v);
    }
}

// Reduce-scatter of NV per-lane values over aligned groups of G lanes: on
// return lane l holds the group total of value (l % G) / (G / NV).
constexpr int ilog2(int x) { return x <= 1 ? 0 : 1 + ilog2(x / 2); }

template <int NV, int G, int O = G / 2>
__device__ __forceinline__ float reduce_scatter_from(float (&v)[NV], int nv, int lane) {
    if constexpr (O == 0) {
        return v[0];
    } else {
        if (nv > 1) {
            rs_step<O, NV>(v, nv, lane);
            return reduce_scatter_from<NV, G, O / 2>(v, nv / 2, lane);
        }
        v[0] = sum_step<O>(v[0]);
        return reduce_scatter_from<NV, G, O / 2>(v, 1, lane);
    }
}
template <int NV, int G>
__device__ __forceinline__ float reduce_scatter(float (&v)[NV], int lane) {
    return reduce_scatter_from<NV, G>(v, NV, lane);
}

}  // namespace mdx
