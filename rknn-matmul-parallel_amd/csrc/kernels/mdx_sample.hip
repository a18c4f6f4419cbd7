// mdx_sample.hip — token sampling on the device, from the logits a decode step
// leaves in HBM, so that non-greedy decoding needs no copy of the V logits to
// the host.  For top_k <= 64 (the usual sampling settings) two launches:
// 256 workgroups each keep the 64 best of their contiguous index range as
// 64-bit ranking keys, sorted with wave-level bitonic networks in registers;
// 16 workgroups merge 16 lists each the same way, and the last of them to
// finish merges their 16 results: the first k keys are the candidates in rank
// order.  Larger k: seven short
// launches, a scratch clear, four radix-select levels and a gather over 128
// workgroups (each owns a contiguous index range), and one finishing
// workgroup that ranks the candidates with a bitonic sort in LDS.
//
//   1. (separate tiny kernel) repetition penalty on the listed tokens, once
//      per distinct token: a positive logit is divided by the penalty, any
//      other multiplied by it.  The reference declares the parameter
//      (include/matmul_decoder.h:395-397) and applies it nowhere.
//   2. v_i = logits_i / T when T != 1 (src/cpu_ops.c:597-601 divides).
//   3. the k largest v, ties to the lower index: the reference's insertion
//      (src/cpu_ops.c:604-624) takes an element only when it is strictly
//      greater, so an equal value never displaces an earlier index.  Its k
//      slots start as (index 0, -1e30) and only v > -1e30 displaces them, so
//      NaN and values <= -1e30 never become candidates and missing slots stay
//      (0, -1e30); the same rule holds here (such values get key 0).  Found by
//      a radix select over an order-preserving 32-bit key (4 levels of 8
//      bits; per-block LDS histograms summed in device memory), then the
//      keys above the threshold are appended and the ties at it taken in
//      index order (per-range counts, then a rescan of only the ranges that
//      hold the first ones), then ranked by (value desc, index asc).
//   4. e_j = expf(v_j - v_0) and sum = sum of e_j in rank order
//      (src/cpu_ops.c:626-632).
//   5. top_p < 1 keeps the shortest prefix whose running sum reaches
//      top_p * sum (nucleus restriction of the top-k candidates; the
//      reference's top_p_sample_f32, src/cpu_ops.c:650-665, returns the
//      argmax instead).
//   6. r = u * sum with the caller's uniform u in [0,1] in place of
//      rand() / RAND_MAX; the token is the first candidate whose running sum
//      exceeds r, else the last (src/cpu_ops.c:634-646).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <mutex>

#include "mdx_device.h"

namespace {

constexpr int kThreads = 1024;          // the finishing workgroup
constexpr int kBlocks = 128;            // histogram / gather grid
constexpr int kBT = 256;                // threads per grid block
constexpr int kMaxK = MDX_SAMPLE_MAX_TOP_K;
constexpr int kLB = 256;                // per-range selection blocks (small-k path)
constexpr int kSmallK = 64;             // the small-k path serves top_k up to this
constexpr int kRange = 1024;            // values of one block range (small-k path: V <= kLB * kRange)

static_assert(kMaxK <= kThreads, "one candidate per thread in the ranking");
static_assert(kSmallK == 64 && kLB == 16 * 16, "16 merging workgroups of 16 lists");

// Scratch in device memory, cleared by k_sample_clear at the start of a call.
struct SampleScratch {
    uint32_t hist[4][256];      // per radix level
    int n_gt;                   // keys above the threshold, appended so far
    int pad[63];
    int tiecount[kBlocks];      // keys equal to the threshold, per block range
    int cand_idx[kMaxK];
    float cand_val[kMaxK];
    // small-k path: block b's 64 best candidates as ranking keys (rank_key),
    // in ranking order; 0 fills the slots past its eligible values
    unsigned long long loc_top[kLB][kSmallK];
    unsigned long long grp_top[kLB / 16][kSmallK];   // merged lists of 16 ranges each
    unsigned merge_arrived;                           // zero between calls
};

// The reference's empty-slot value: only v > kFloor can become a candidate.
constexpr float kFloor = -1e30f;

// Larger float -> larger key.  -0 and +0 share the key of +0 (they compare
// equal as floats).  Values that can never be candidates (NaN, <= -1e30)
// take key 0, which no candidate has.
__device__ inline uint32_t order_key(float v) {
    if (!(v > kFloor)) return 0u;
    const uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ inline float tempered(float l, float temp) { return temp != 1.0f ? l / temp : l; }

// Block b's contiguous index range (ranges follow index order).
__device__ inline void block_range(int V, int b, int& r0, int& r1) {
    const int chunk = (V + kBlocks - 1) / kBlocks;
    r0 = b * chunk < V ? b * chunk : V;
    r1 = r0 + chunk < V ? r0 + chunk : V;
}

// One radix level resolved from its 256-bin histogram by the 64 lanes of one
// wave: the digit d whose bin holds the need-th largest remaining key,
// above(d) < need <= above(d) + hist[d], above(d) being the count in the bins
// above d (a suffix sum over the lanes, four bins per lane); need drops by
// above(d).  With fewer than need keys in all bins the digit is 0.
__device__ inline uint32_t resolve_level(const uint32_t* hist, uint32_t& need) {
    const int lane = threadIdx.x & 63;
    {
        const uint4 h = *reinterpret_cast<const uint4*>(&hist[4 * lane]);
        const uint32_t loc = h.x + h.y + h.z + h.w;
        uint32_t incl = loc;                        // bins of lanes >= this one
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t o = __shfl_down(incl, off);
            if (lane + off < 64) incl += o;
        }
        uint32_t a = incl - loc;                    // bins above this lane's four
        int found = -1;
        uint32_t at = 0u;
        if (a < need && need <= a + h.w) { found = 4 * lane + 3; at = a; }
        a += h.w;
        if (found < 0 && a < need && need <= a + h.z) { found = 4 * lane + 2; at = a; }
        a += h.z;
        if (found < 0 && a < need && need <= a + h.y) { found = 4 * lane + 1; at = a; }
        a += h.y;
        if (found < 0 && a < need && need <= a + h.x) { found = 4 * lane; at = a; }
        const unsigned long long bal = __ballot(found >= 0);
        int d = 0;
        uint32_t above = __shfl(incl, 0) - __shfl(h.x, 0);   // no bin found: digit 0
        if (bal) {
            const int src = __ffsll((long long)bal) - 1;
            d = __shfl(found, src);
            above = __shfl(at, src);
        }
        need -= above;
        return (uint32_t)d;
    }
}

// The radix levels [0, levels) resolved from the histograms in scratch: the
// key prefix they fix and how many keys equal to the full threshold are still
// needed.
__device__ inline void resolve(const SampleScratch* sc, int levels, int k, uint32_t& prefix,
                               uint32_t& need) {
    prefix = 0u;
    need = (uint32_t)k;
    for (int lv = 0; lv < levels; lv++) prefix |= resolve_level(sc->hist[lv], need) << (24 - 8 * lv);
}

// Ranking key of a candidate: its order key above the complemented index, so
// that a descending order is (value desc, index asc).  Key 0 sorts last.
__device__ inline unsigned long long rank_key(uint32_t key, int idx) {
    return ((unsigned long long)key << 32) | (0xffffffffu - (uint32_t)idx);
}
__device__ inline int rank_index(unsigned long long rk) { return (int)(0xffffffffu - (uint32_t)rk); }

// Descending bitonic sort of N (a power of two) keys in LDS, one per thread.
template <int N>
__device__ inline void bitonic_desc(unsigned long long* a, int tid) {
    for (int size = 2; size <= N; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const int o = tid ^ stride;
            if (tid < N && o > tid) {
                const unsigned long long x = a[tid], y = a[o];
                const bool desc = (tid & size) == 0;
                if (desc ? x < y : x > y) {
                    a[tid] = y;
                    a[o] = x;
                }
            }
            __syncthreads();
        }
    }
}

// The draw from k ranked candidates (sidx/sval by value desc, index asc;
// empty slots (0, -1e30)): e_j = expf(v_j - v_0), running sums in rank order
// (the reference's sequential float sum), the nucleus prefix and the draw as
// the first crossing of a threshold, found in parallel (running sums of
// non-negative terms never decrease, so each crossing is unique).  ebuf holds
// k floats of workgroup scratch, 16-byte aligned, its length a multiple of 4.
// Called by every thread of the workgroup.
__device__ inline void finish(int k, const int* sidx, const float* sval, float* ebuf, float top_p,
                              float u, int* out, int* top_idx, float* top_val) {
    __shared__ __align__(16) float run[kMaxK];
    __shared__ int s_m, s_pick;
    const int tid = threadIdx.x;
    if (tid < k) ebuf[tid] = expf(sval[tid] - sval[0]);
    __syncthreads();
    if (tid == 0) {
        // one term after another (16-byte LDS reads and writes; the terms and
        // sums past k are never read)
        float acc = 0.0f;
        for (int j = 0; j < k; j += 4) {
            const float4 e = *reinterpret_cast<const float4*>(ebuf + j);
            float4 r;
            acc += e.x; r.x = acc;
            acc += e.y; r.y = acc;
            acc += e.z; r.z = acc;
            acc += e.w; r.w = acc;
            *reinterpret_cast<float4*>(run + j) = r;
        }
        s_m = k;
    }
    __syncthreads();
    if (top_p < 1.0f && tid < k) {
        const float lim = top_p * run[k - 1];
        if (run[tid] >= lim && (tid == 0 || run[tid - 1] < lim)) s_m = tid + 1;
    }
    __syncthreads();
    const int m = s_m;
    if (tid == 0) s_pick = m - 1;       // no crossing (u = 1): the last kept
    __syncthreads();
    const float r = u * run[m - 1];
    if (tid < m && r < run[tid] && (tid == 0 || !(r < run[tid - 1]))) s_pick = tid;
    __syncthreads();
    if (tid == 0) {
        out[0] = sidx[s_pick];
        out[1] = m;
    }
    if (top_idx && tid < k) top_idx[tid] = sidx[tid];
    if (top_val && tid < k) top_val[tid] = sval[tid];
}

// Inclusive scan of one int per thread over a workgroup of NT threads: within
// each wave by shuffles, then over the wave totals (wsum: NT/64 ints of LDS).
// *total receives the workgroup's sum.
template <int NT>
__device__ inline int scan_incl(int* wsum, int v, int* total) {
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    if (wave == 0) {
        int w = lane < NW ? wsum[lane] : 0;
#pragma unroll
        for (int off = 1; off < NW; off <<= 1) {
            const int y = __shfl_up(w, off, 64);
            if (lane >= off) w += y;
        }
        if (lane < NW) wsum[lane] = w;
    }
    __syncthreads();
    const int r = x + (wave ? wsum[wave - 1] : 0);
    *total = wsum[NW - 1];
    __syncthreads();   // wsum is reused by the next scan
    return r;
}

// ---- small-k path: wave-level bitonic top-64 ------------------------------
//
// A wave holds 64 ranking keys, one per lane.  wave_sort_desc sorts them in
// descending order across the lanes (lane 0 the best); wave_merge_top keeps
// the best 64 of two such sorted sets (the lane-wise maximum of one set and
// the other reversed is bitonic and holds the best 64, which six merge steps
// sort).  The ranking key is a total order, so the result is the exact top-64
// of the values seen, in the reference's order (value desc, index asc).
// Lane exchanges on the VALU: the value of lane l ^ J (DPP moves within a
// 16-lane row, the gfx950 row swaps across rows), and of lane 63 - l.
template <int CTRL>
__device__ inline uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int J>
__device__ inline uint32_t xor_lane(uint32_t v) {
    const int lane = threadIdx.x & 63;
    if constexpr (J == 1) return dpp_u32<0xB1>(v);            // quad_perm [1,0,3,2]
    else if constexpr (J == 2) return dpp_u32<0x4E>(v);       // quad_perm [2,3,0,1]
    else if constexpr (J == 4) {
        const uint32_t up = dpp_u32<0x104>(v);                // row_shl:4: lane l + 4
        const uint32_t dn = dpp_u32<0x114>(v);                // row_shr:4: lane l - 4
        return (lane & 4) ? dn : up;
    } else if constexpr (J == 8) return dpp_u32<0x128>(v);    // row_ror:8
    else if constexpr (J == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16) ? r[0] : r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane & 32) ? r[0] : r[1];
    }
}
template <int J>
__device__ inline unsigned long long xor_lane_u64(unsigned long long v) {
    const uint32_t lo = xor_lane<J>((uint32_t)v), hi = xor_lane<J>((uint32_t)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}
__device__ inline unsigned long long reverse_lanes_u64(unsigned long long v) {
    // row_mirror (c -> 15 - c), then rows r -> r ^ 3
    uint32_t lo = dpp_u32<0x140>((uint32_t)v), hi = dpp_u32<0x140>((uint32_t)(v >> 32));
    lo = xor_lane<16>(xor_lane<32>(lo));
    hi = xor_lane<16>(xor_lane<32>(hi));
    return ((unsigned long long)hi << 32) | lo;
}
// One compare-exchange step at distance J: keep_max lanes keep the larger key.
template <int J>
__device__ inline unsigned long long cmpx(unsigned long long v, bool keep_max) {
    const unsigned long long o = xor_lane_u64<J>(v);
    return keep_max ? (v > o ? v : o) : (v < o ? v : o);
}
template <int SIZE, int J>
__device__ inline unsigned long long sort_stage(unsigned long long v, int lane) {
    if constexpr (J == 0) {
        return v;
    } else {
        // the lower lane of a descending pair keeps the larger key
        v = cmpx<J>(v, ((lane & J) == 0) == ((lane & SIZE) == 0));
        return sort_stage<SIZE, J / 2>(v, lane);
    }
}
template <int SIZE>
__device__ inline unsigned long long sort_from(unsigned long long v, int lane) {
    if constexpr (SIZE > 64) {
        return v;
    } else {
        v = sort_stage<SIZE, SIZE / 2>(v, lane);
        return sort_from<SIZE * 2>(v, lane);
    }
}
__device__ inline unsigned long long wave_sort_desc(unsigned long long v) {
    return sort_from<2>(v, threadIdx.x & 63);
}
template <int J>
__device__ inline unsigned long long clean_desc(unsigned long long v, int lane) {
    if constexpr (J == 0) {
        return v;
    } else {
        v = cmpx<J>(v, (lane & J) == 0);
        return clean_desc<J / 2>(v, lane);
    }
}
__device__ inline unsigned long long wave_merge_top(unsigned long long a, unsigned long long b) {
    const int lane = threadIdx.x & 63;
    const unsigned long long rb = reverse_lanes_u64(b);
    const unsigned long long v = a > rb ? a : rb;
    return clean_desc<32>(v, lane);
}
// The best 64 of N sorted sets, merged as a tree: the merges of one level are
// independent, so their instruction streams interleave.
template <int N>
__device__ inline unsigned long long tree_merge(unsigned long long (&x)[N]) {
#pragma unroll
    for (int step = 1; step < N; step *= 2)
#pragma unroll
        for (int i = 0; i + step < N; i += 2 * step) x[i] = wave_merge_top(x[i], x[i + step]);
    return x[0];
}

// Small-k path, step 1: block b keeps the 64 best ranking keys of its
// contiguous range (at most kRange values): each wave sorts its chunks of 64
// and merges them, then wave 0 merges the four waves' sets.  The loops are
// kept rolled: each sort or merge is one copy of straight-line code that
// every iteration reuses (unrolled, the instruction fetch of code that runs
// once per launch dominated the kernel).
__global__ __launch_bounds__(kBT) void k_sample_local(const float* __restrict__ logits, int V, float temp,
                                                      SampleScratch* sc) {
    constexpr int NW = kBT / 64;
    constexpr int PER = kRange / kBT;
    __shared__ unsigned long long wl[NW][64];
    __shared__ float vs[NW][PER][64];
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (b == 0 && tid == 0) sc->merge_arrived = 0u;   // the merge launch that follows counts from zero
    const int chunk = (V + kLB - 1) / kLB;
    const int r0 = min(V, b * chunk), r1 = min(V, r0 + chunk);
    const int n = r1 - r0;
    // element 64 (wave + NW c) + lane of the range; every load issued first
    float v[PER];
#pragma unroll
    for (int c = 0; c < PER; c++) {
        const int i = 64 * (wave + NW * c) + lane;
        v[c] = i < n ? logits[r0 + i] : 0.0f;
    }
#pragma unroll
    for (int c = 0; c < PER; c++) vs[wave][c][lane] = v[c];
    unsigned long long top = 0ull;
#pragma unroll 1
    for (int c = 0; c < PER; c++) {
        const int i = 64 * (wave + NW * c) + lane;
        if (64 * (wave + NW * c) >= n) break;            // uniform over the wave
        const uint32_t key = i < n ? order_key(tempered(vs[wave][c][lane], temp)) : 0u;
        const unsigned long long x = wave_sort_desc(key ? rank_key(key, r0 + i) : 0ull);
        top = c == 0 ? x : wave_merge_top(top, x);
    }
    wl[wave][lane] = top;
    __syncthreads();
    if (wave == 0) {
        unsigned long long t = wl[0][lane];
#pragma unroll 1
        for (int w = 1; w < NW; w++) t = wave_merge_top(t, wl[w][lane]);
        sc->loc_top[b][lane] = t;
    }
}

// Small-k path, step 2: 16 workgroups of 16 waves each merge 16 of the 256
// range lists as a tree across their waves (four levels through LDS), store
// the result and count their arrival; the last to arrive merges the 16
// results the same way.  Its first k ranking keys are the reference's k
// candidates in rank order; keys 0 (fewer than k eligible values) are the
// empty slots (index 0, -1e30).
constexpr int kMergeBlocks = kLB / 16;

// The best 64 of the 16 waves' sets by a tree through LDS: on return wave 0
// holds them.  set: 16 x 64 keys of LDS.
__device__ inline unsigned long long tree_across_waves(unsigned long long t, unsigned long long (*set)[64]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int step = 1; step < 16; step *= 2) {
        if (wave % (2 * step) == step) set[wave][lane] = t;
        __syncthreads();
        if (wave % (2 * step) == 0) t = wave_merge_top(t, set[wave + step][lane]);
        __syncthreads();
    }
    return t;
}

__global__ __launch_bounds__(kThreads) void k_sample_merge(const float* __restrict__ logits, float temp,
                                                           int k, float top_p, float u,
                                                           SampleScratch* sc, int* __restrict__ out,
                                                           int* __restrict__ top_idx,
                                                           float* __restrict__ top_val) {
    static_assert(kThreads == 16 * 64, "one list per wave");
    __shared__ unsigned long long set[16][64];
    __shared__ int s_last;
    __shared__ int sidx[kSmallK];
    __shared__ float sval[kSmallK];
    __shared__ __align__(16) float ebuf[kSmallK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = blockIdx.x;
    unsigned long long t = tree_across_waves(sc->loc_top[16 * g + wave][lane], set);
    // the result goes out with device-scope stores that complete before the
    // arrival is counted, and the last block reads with device-scope loads:
    // no cache write-back or invalidate is needed (a __threadfence pair here,
    // which writes back the whole L2 of the XCD, took the kernel to 16.5 us)
    if (wave == 0) __hip_atomic_store(&sc->grp_top[g][lane], t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(&sc->merge_arrived, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (unsigned)(kMergeBlocks - 1);
    __syncthreads();
    if (!s_last) return;
    if (tid == 0) __hip_atomic_store(&sc->merge_arrived, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    t = tree_across_waves(__hip_atomic_load(&sc->grp_top[wave][lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                          set);
    if (wave == 0 && lane < k) {
        const bool real = (t >> 32) != 0ull;
        const int i = real ? rank_index(t) : 0;
        sidx[lane] = i;
        sval[lane] = real ? tempered(logits[i], temp) : kFloor;
    }
    __syncthreads();
    finish(k, sidx, sval, ebuf, top_p, u, out, top_idx, top_val);
}

__global__ __launch_bounds__(256) void k_repeat_penalty(float* logits, const int* toks, int n,
                                                       float penalty) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const int t = toks[i];
    const float l = logits[t];
    logits[t] = l > 0.0f ? l / penalty : l * penalty;
}

__global__ __launch_bounds__(256) void k_sample_clear(SampleScratch* sc) {
    uint32_t* h = &sc->hist[0][0];
    for (int i = threadIdx.x; i < 4 * 256; i += 256) h[i] = 0u;
    if (threadIdx.x == 0) sc->n_gt = 0;
}

// One radix level: every block histograms the digit of its range's keys that
// match the prefix of the levels before, and adds its bins to the level's.
__global__ __launch_bounds__(kBT) void k_sample_hist(const float* __restrict__ logits, int V,
                                                     float temp, int k, int level,
                                                     SampleScratch* sc) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_prefix, s_mask;
    const int tid = threadIdx.x;
    hist[tid] = 0u;
    if (tid < 64) {
        uint32_t prefix, need;
        resolve(sc, level, k, prefix, need);
        if (tid == 0) {
            s_prefix = prefix;
            s_mask = level ? 0xffffffffu << (32 - 8 * level) : 0u;
        }
    }
    __syncthreads();
    const uint32_t prefix = s_prefix, mask = s_mask;
    const int shift = 24 - 8 * level;
    int r0, r1;
    block_range(V, blockIdx.x, r0, r1);
    for (int i = r0 + tid; i < r1; i += kBT) {
        const uint32_t key = order_key(tempered(logits[i], temp));
        if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    const uint32_t h = hist[tid];
    if (h) atomicAdd(&sc->hist[level][tid], h);
}

// Keys above the threshold are appended (any order); keys equal to it are
// counted per block range.
__global__ __launch_bounds__(kBT) void k_sample_gather(const float* __restrict__ logits, int V,
                                                       float temp, int k, SampleScratch* sc) {
    __shared__ uint32_t s_kstar;
    __shared__ int s_ties;
    const int tid = threadIdx.x;
    if (tid < 64) {
        uint32_t prefix, need;
        resolve(sc, 4, k, prefix, need);
        if (tid == 0) {
            s_kstar = prefix;
            s_ties = 0;
        }
    }
    __syncthreads();
    const uint32_t kstar = s_kstar;
    int r0, r1;
    block_range(V, blockIdx.x, r0, r1);
    int ties = 0;
    for (int i = r0 + tid; i < r1; i += kBT) {
        const float v = tempered(logits[i], temp);
        const uint32_t key = order_key(v);
        if (key > kstar) {   // kstar may be 0 (fewer than k candidates): key 0 never passes
            const int slot = atomicAdd(&sc->n_gt, 1);
            if (slot < kMaxK) {
                sc->cand_idx[slot] = i;
                sc->cand_val[slot] = v;
            }
        }
        ties += key == kstar && kstar != 0u;
    }
    if (ties) atomicAdd(&s_ties, ties);
    __syncthreads();
    if (tid == 0) sc->tiecount[blockIdx.x] = s_ties;
}

// The finishing workgroup: the candidates above the threshold, the first
// `need` ties in index order (rescanning only the block ranges that hold
// them), the ranking, softmax, top-p and the draw.
__global__ __launch_bounds__(kThreads) void k_sample_final(const float* __restrict__ logits, int V,
                                                           float temp, int k, float top_p, float u,
                                                           const SampleScratch* sc,
                                                           int* __restrict__ out,
                                                           int* __restrict__ top_idx,
                                                           float* __restrict__ top_val) {
    __shared__ uint32_t s_kstar;
    __shared__ int s_need;
    __shared__ int wsum[kThreads / 64];
    __shared__ int cidx[kMaxK], sidx[kMaxK];
    __shared__ __align__(16) float cval[kMaxK];
    __shared__ float sval[kMaxK];
    const int tid = threadIdx.x;
    if (tid < 64) {
        uint32_t prefix, need;
        resolve(sc, 4, k, prefix, need);
        if (tid == 0) {
            s_kstar = prefix;
            s_need = (int)need;
        }
    }
    __syncthreads();
    const uint32_t kstar = s_kstar;
    // kstar == 0: fewer than k values can be candidates; every one of them is
    // above the threshold and the other slots keep (index 0, -1e30)
    const int need = kstar ? s_need : 0;
    const int greater = k - s_need;
    const int nc = greater + need;     // candidates that are real values
    if (tid < greater) {
        cidx[tid] = sc->cand_idx[tid];
        cval[tid] = sc->cand_val[tid];
    }
    int base = 0;                       // ties taken so far (uniform)
    for (int b = 0; b < kBlocks && base < need; b++) {
        if (sc->tiecount[b] == 0) continue;
        int r0, r1;
        block_range(V, b, r0, r1);
        for (int c0 = r0; c0 < r1 && base < need; c0 += kThreads) {
            const int i = c0 + tid;
            float v = 0.0f;
            int flag = 0;
            if (i < r1) {
                v = tempered(logits[i], temp);
                flag = order_key(v) == kstar;
            }
            int tot;
            const int incl = scan_incl<kThreads>(wsum, flag, &tot);
            const int pos = base + incl - flag;
            if (flag && pos < need) {
                cidx[greater + pos] = i;
                cval[greater + pos] = v;
            }
            base += tot;
        }
    }
    __syncthreads();

    // rank by (value desc, index asc): a bitonic sort of 64-bit keys (the
    // order key of the value above the complemented index; the pairs are
    // distinct); the empty slots follow as (index 0, -1e30)
    __shared__ unsigned long long sk[kThreads];
    sk[tid] = tid < nc ? rank_key(order_key(cval[tid]), cidx[tid]) : 0ull;
    __syncthreads();
    bitonic_desc<kThreads>(sk, tid);
    if (tid < k) {
        const int i = tid < nc ? rank_index(sk[tid]) : 0;
        sidx[tid] = i;
        sval[tid] = tid < nc ? tempered(logits[i], temp) : kFloor;
    }
    __syncthreads();
    finish(k, sidx, sval, cval, top_p, u, out, top_idx, top_val);
}

// The sampler scratch of mdx_sample_topk_noalloc, for callers that cannot
// allocate: one copy per device, held until the process ends.  Host code
// never passes the name itself to a kernel (on the host it is only a handle);
// it uses the device address hipGetSymbolAddress returns for the current
// device, looked up once per device.
static __device__ __align__(256) unsigned char scratch[sizeof(SampleScratch)];
constexpr int kMaxDevices = 64;
void* g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of this device's scratch, or nullptr (with a message).
void* noalloc_scratch() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        fprintf(stderr, "mdx_sample_topk_noalloc: no usable current device (%d)\n", dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fprintf(stderr, "mdx_sample_topk_noalloc: hipGetSymbolAddress: %s\n", hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_addr[dev] = p;
    }
    return g_scratch_addr[dev];
}

}  // namespace

extern "C" {

size_t mdx_sample_scratch_bytes(void) { return sizeof(SampleScratch); }

int mdx_sample_topk_noalloc(const float* logits, int V, float temperature, int top_k, float top_p,
                            float uniform, int* out, int* top_idx, float* top_val, void* stream) {
    if (top_k > kMaxK) {
        fprintf(stderr, "mdx_sample_topk_noalloc: top_k=%d exceeds the scratch capacity of %d candidates\n",
                top_k, kMaxK);
        return -1;
    }
    if (!logits || V <= 0 || top_k < 1 || top_k > V || !(temperature > 0.0f) || !(uniform >= 0.0f) ||
        !(uniform <= 1.0f) || !out)
        return -1;
    void* sc = noalloc_scratch();
    if (!sc) return -4;
    return mdx_launch_topk_sample(logits, V, temperature, top_k, top_p, uniform, sc, out, top_idx, top_val,
                                  stream);
}

int mdx_launch_repeat_penalty(float* logits, const int* tokens, int n, float penalty, void* stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_repeat_penalty, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       logits, tokens, n, penalty);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int mdx_launch_topk_sample(const float* logits, int V, float temperature, int k, float top_p,
                           float uniform, void* scratch, int* out, int* top_idx, float* top_val,
                           void* stream) {
    if (V <= 0 || k < 1 || k > kMaxK || k > V || !(temperature > 0.0f) || !(uniform >= 0.0f) ||
        !(uniform <= 1.0f) || !scratch || !out)
        return -1;
    hipStream_t s = (hipStream_t)stream;
    SampleScratch* sc = (SampleScratch*)scratch;
    if (k <= kSmallK && V <= kLB * kRange) {
        hipLaunchKernelGGL(k_sample_local, dim3(kLB), dim3(kBT), 0, s, logits, V, temperature, sc);
        hipLaunchKernelGGL(k_sample_merge, dim3(kMergeBlocks), dim3(kThreads), 0, s, logits, temperature, k,
                           top_p, uniform, sc, out, top_idx, top_val);
        return hipGetLastError() == hipSuccess ? 0 : -4;
    }
    hipLaunchKernelGGL(k_sample_clear, dim3(1), dim3(256), 0, s, sc);
    for (int level = 0; level < 4; level++)
        hipLaunchKernelGGL(k_sample_hist, dim3(kBlocks), dim3(kBT), 0, s, logits, V, temperature, k,
                           level, sc);
    hipLaunchKernelGGL(k_sample_gather, dim3(kBlocks), dim3(kBT), 0, s, logits, V, temperature, k, sc);
    hipLaunchKernelGGL(k_sample_final, dim3(1), dim3(kThreads), 0, s, logits, V, temperature, k, top_p,
                       uniform, (const SampleScratch*)sc, out, top_idx, top_val);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // extern "C"
