// mdx_sample.hip — token sampling on the device, from the logits a decode step
// leaves in HBM, so that non-greedy decoding needs no copy of the V logits to
// the host.  Seven short launches: a scratch clear, four radix-select levels
// and a gather over 128 workgroups (each owns a contiguous index range), and
// one finishing workgroup of 1024 threads.
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

static_assert(kMaxK <= kThreads, "one candidate per thread in the ranking");

// Scratch in device memory, cleared by k_sample_clear at the start of a call.
struct SampleScratch {
    uint32_t hist[4][256];      // per radix level
    int n_gt;                   // keys above the threshold, appended so far
    int pad[63];
    int tiecount[kBlocks];      // keys equal to the threshold, per block range
    int cand_idx[kMaxK];
    float cand_val[kMaxK];
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

// The radix levels [0, levels) resolved from the histograms, by the 64 lanes
// of one wave: the key prefix they fix and how many keys equal to the full
// threshold are still needed.  At each level the digit d is the one whose
// bin holds the need-th largest remaining key: above(d) < need <= above(d) +
// hist[d], above(d) being the count in the bins above d (a suffix sum over
// the lanes, four bins per lane).
__device__ inline void resolve(const SampleScratch* sc, int levels, int k, uint32_t& prefix,
                               uint32_t& need) {
    const int lane = threadIdx.x & 63;
    prefix = 0u;
    need = (uint32_t)k;
    for (int lv = 0; lv < levels; lv++) {
        const uint4 h = *reinterpret_cast<const uint4*>(&sc->hist[lv][4 * lane]);
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
        prefix |= (uint32_t)d << (24 - 8 * lv);
    }
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

// Inclusive scan of one int per thread over the workgroup.
__device__ inline int block_scan(int* buf, int v) {
    const int tid = threadIdx.x;
    buf[tid] = v;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
        const int a = tid >= off ? buf[tid - off] : 0;
        __syncthreads();
        buf[tid] += a;
        __syncthreads();
    }
    return buf[tid];
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
    __shared__ int scan[kThreads];
    __shared__ int cidx[kMaxK], sidx[kMaxK];
    __shared__ float cval[kMaxK], sval[kMaxK];
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
            const int incl = block_scan(scan, flag);
            const int pos = base + incl - flag;
            if (flag && pos < need) {
                cidx[greater + pos] = i;
                cval[greater + pos] = v;
            }
            base += scan[kThreads - 1];
            __syncthreads();
        }
    }
    __syncthreads();

    // rank by (value desc, index asc); the pairs are distinct, so the ranks
    // are a permutation of 0..nc-1; the empty slots follow
    __shared__ uint32_t ckey[kMaxK];
    if (tid < nc) ckey[tid] = order_key(cval[tid]);
    __syncthreads();
    if (tid < nc) {
        const uint32_t kj = ckey[tid];
        const int ij = cidx[tid];
        int r = 0;
        for (int m = 0; m < nc; m++) {
            const uint32_t km = ckey[m];
            r += km > kj || (km == kj && cidx[m] < ij);
        }
        sidx[r] = ij;
        sval[r] = cval[tid];
    } else if (tid < k) {
        sidx[tid] = 0;
        sval[tid] = kFloor;
    }
    __syncthreads();

    // softmax over the candidates: running sums in rank order (the
    // reference's sequential float sum), then the nucleus prefix and the draw
    // as the first crossing of a threshold, found in parallel (running sums
    // of non-negative terms never decrease, so each crossing is unique)
    __shared__ float run[kMaxK];
    __shared__ int s_m, s_pick;
    if (tid < k) cval[tid] = expf(sval[tid] - sval[0]);
    __syncthreads();
    if (tid == 0) {
        float acc = 0.0f;
#pragma unroll 8
        for (int j = 0; j < k; j++) {
            acc += cval[j];
            run[j] = acc;
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
