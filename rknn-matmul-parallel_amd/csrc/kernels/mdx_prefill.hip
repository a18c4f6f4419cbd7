// mdx_prefill.hip — batch prefill (M <= 64 rows) kernels for gfx950.
//
// Projections (reference: src/matmul_decoder.c:1841-1899, run_batch_matmul)
// run on MFMA v_mfma_f32_16x16x32_f16: the qkv and gate/up projections one
// block per 64 x 32 output tile with the K range split over its waves
// (k_gemm, or k_gemm_p with the block's activation panel staged in LDS), the
// o and down projections split over blocks along K with the activation panel
// staged in LDS (k_gemm_s).
#include <hip/hip_runtime.h>

#include <cmath>

#include "mdx_common.h"
#include "mdx_device.h"
#include "mdx_gemm_tile.h"

using namespace mdx;

namespace {

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

// Weights are read once per prefill: non-temporal loads keep them from
// evicting the activation panels and split-K partials that the following
// kernels read again (measured: 1.139 -> 1.089 ms for the M=60 INT8 prefill).
__device__ __forceinline__ uint4 ld_w(const void* p) { return ld_nt(p); }

constexpr int kMaxM = 64;
constexpr int kNT = 32;        // weight rows (output columns) per block

// fp32 GEMM results (split partials, projection outputs) are stored
// write-through (agent-scope store, sc1): the next kernel reads them from
// memory anyway, and less dirty data is left in L2 when the kernel ends
// (measured on the M=60 INT8 prefill: 1.456 -> 1.423 ms).
__device__ __forceinline__ void store_wt(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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

// ---- projections: register-direct MFMA GEMM ----------------------------------
//
// Block = GemmKind::WAVES waves (8: two per SIMD with up to 256 registers
// each), one 64 x 32 output tile (all M
// rows, two 16-column MFMA tiles; for SwiGLU the gate and up columns of the
// same 16 features).  The K
// range is split over the waves in contiguous runs of K-blocks; a wave keeps
// several rounds of K-blocks of weights and activations in flight in registers (the MFMA
// fragments are loaded straight from memory, the int8/int4 weights widened to
// fp16 exactly in registers), so a block's loads are not serialised behind
// barriers.  The waves' partial tiles are summed in LDS in wave order, then the
// scale and the epilogue are applied.
//
// K-block layout: a weight load is 16 bytes per lane = EPL consecutive k of
// one weight row (EPL = 8 fp16, 16 int8, 32 int4), lane group g = lane/16
// takes k [g*EPL, (g+1)*EPL) of the block, and MFMA step s of the block uses
// k g*EPL + 8s .. +7; the activations are loaded with the same k mapping.

// Weight row of tile column c: 32 consecutive rows, or for SwiGLU the 16 gate
// rows f0.. and the 16 up rows N/2+f0.. of the same features.
__device__ __forceinline__ int tile_row(int tile, int c, int swiglu, int N) {
    if (!swiglu) return tile * kNT + c;
    const int f0 = tile * (kNT / 2);
    return c < kNT / 2 ? f0 + c : N / 2 + f0 + (c - kNT / 2);
}

template <int KIND>
struct GemmRound {
    uint4 bw[GemmKind<KIND>::NKB][2];
    uint4 av[GemmKind<KIND>::NKB][4][GemmKind<KIND>::EPL / 8];
};

// Requests the NKB K-blocks of a round starting at K-block kb (blocks past
// the wave's range re-read block kb_last; gemm_compute skips them).
// K need not be a multiple of the K-block: a lane group whose k range lies at
// or past K (K is a multiple of EPL) loads zero weights and zero activations.
template <int KIND>
__device__ __forceinline__ void gemm_issue(GemmRound<KIND>& R, int kb, int kb_last, int K,
                                           const uint8_t* const (&wrow)[2], const bool (&wvalid)[2],
                                           const uint16_t* const (&arow)[4], int g) {
    using GK = GemmKind<KIND>;
    constexpr int EPL = GK::EPL, KB = 4 * EPL;
#pragma unroll
    for (int j = 0; j < GK::NKB; j++) {
        const int k = min(kb + j, kb_last) * KB + g * EPL;
        const bool kin = k < K;
#pragma unroll
        for (int t = 0; t < 2; t++)
            R.bw[j][t] = (wvalid[t] && kin) ? ld_w(wrow[t] + (size_t)k * 16 / EPL)
                                            : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int s = 0; s < EPL / 8; s++)
                R.av[j][r][s] = kin ? *reinterpret_cast<const uint4*>(arow[r] + k + 8 * s)
                                    : make_uint4(0u, 0u, 0u, 0u);
    }
}

template <int KIND>
__device__ __forceinline__ void gemm_compute(const GemmRound<KIND>& R, int kb, int kb_end,
                                             float4_t (&acc)[2][4]) {
    using GK = GemmKind<KIND>;
    constexpr int STEPS = GK::EPL / 8;
#pragma unroll
    for (int j = 0; j < GK::NKB; j++) {
        if (kb + j >= kb_end) break;
        half8_t b[2][STEPS];
#pragma unroll
        for (int t = 0; t < 2; t++) widen_b<KIND>(R.bw[j][t], b[t]);
#pragma unroll
        for (int s = 0; s < STEPS; s++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const half8_t a = __builtin_bit_cast(half8_t, R.av[j][r][s]);
#pragma unroll
                for (int t = 0; t < 2; t++)
                    acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[t][s], acc[t][r], 0, 0, 0);
            }
    }
}

// The epilogue shared by k_gemm and k_gemm_p: the waves' partial tiles (the
// MFMA accumulators) are summed in LDS in wave order; then split partials go
// to part (write-through), or the scale and the epilogue are applied.
template <int NW>
__device__ __forceinline__ void gemm_epilogue(const float4_t (&acc)[2][4], float (*red)[kMaxM * kNT], int tid,
                                              int M, int N, int tile, int swiglu, int epi, float sc_a,
                                              float sc_b, float* out_f32, uint16_t* out_f16, float* part) {
    const int wave = tid >> 6, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
    // D fragment: lane holds column c16 of MFMA tile t, rows 16r + 4g + i
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                red[wave][(16 * r + 4 * g + i) * kNT + 16 * t + c16] = acc[t][r][i];
    __syncthreads();
    // 2048 outputs over 256 threads, summed in wave order
    for (int o = tid; o < kMaxM * kNT; o += NW * 64) {
        const int row = o / kNT, col = o % kNT;
        if (row >= M) continue;
        float v = red[0][o];
#pragma unroll
        for (int wv = 1; wv < NW; wv++) v = v + red[wv][o];
        if (part) {
            const int n = tile * kNT + col;
            if (n < N) store_wt(&part[((size_t)blockIdx.y * kMaxM + row) * N + n], v);
            continue;
        }
        if (swiglu) {
            if (col >= kNT / 2) continue;
            const int cols = N / 2;
            const int f = tile * (kNT / 2) + col;
            if (f >= cols) continue;
            float u = red[0][row * kNT + col + kNT / 2];
#pragma unroll
            for (int wv = 1; wv < NW; wv++) u = u + red[wv][row * kNT + col + kNT / 2];
            const float gs = v * sc_a, us = u * sc_b;
            float act;
            if (f < (cols & ~3)) act = silu_mul(gs, us);
            else act = (gs / (1.0f + expf(-gs))) * us;     // reference tail formula
            out_f16[(size_t)row * cols + f] = f32_to_f16_bits(act);
        } else {
            const int n = tile * kNT + col;
            if (n >= N) continue;
            const float y = v * sc_a;
            float* dst = out_f32 + (size_t)row * N + n;
            store_wt(dst, epi == 1 ? *dst + y : y);
        }
    }
}

// With part != NULL each block covers K split blockIdx.y (of gridDim.y,
// possibly 1) and stores its raw partial tile to part[blockIdx.y][row][N]
// for k_residual_norm; with part == NULL gridDim.y is 1 and the epilogue
// writes out_f32 / out_f16.
template <int KIND>
__global__ __launch_bounds__(GemmKind<KIND>::WAVES * 64) void k_gemm(const uint16_t* x16, int M,
                                                          const uint8_t* w, int K, int N,
                                                          const float* scale, int epi,
                                                          float* out_f32, uint16_t* out_f16,
                                                          float* part) {
    using GK = GemmKind<KIND>;
    constexpr int EPL = GK::EPL, KB = 4 * EPL;
    constexpr int NW = GK::WAVES;
    __shared__ float red[NW][kMaxM * kNT];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tile = blockIdx.x;
    const int swiglu = epi == 2;
    const int g = lane >> 4, c16 = lane & 15;
    const size_t row_bytes = KIND == MDX_W_F16 ? (size_t)K * 2 : (KIND == MDX_W_I8 ? (size_t)K : (size_t)K / 2);
    // this block's K-blocks (split blockIdx.y of gridDim.y), then this wave's: [kb0, kb1)
    const int nkb_all = (K + KB - 1) / KB;   // the last K-block may be partial
    const int per_split = (nkb_all + gridDim.y - 1) / gridDim.y;
    const int sb0 = min(nkb_all, (int)blockIdx.y * per_split);
    const int sb1 = min(nkb_all, sb0 + per_split);
    const int per = (sb1 - sb0 + NW - 1) / NW;
    const int kb0 = min(sb1, sb0 + wave * per), kb1 = min(sb1, kb0 + per);

    const uint8_t* wrow_[2];
#pragma unroll
    for (int t = 0; t < 2; t++) wrow_[t] = w + (size_t)tile_row(tile, 16 * t + c16, swiglu, N) * row_bytes;
    const uint8_t* const wrow[2] = {wrow_[0], wrow_[1]};
    const bool wvalid[2] = {tile_row(tile, c16, swiglu, N) < N, tile_row(tile, 16 + c16, swiglu, N) < N};
    const uint16_t* const arow[4] = {x16 + (size_t)min(c16, M - 1) * K, x16 + (size_t)min(16 + c16, M - 1) * K,
                                     x16 + (size_t)min(32 + c16, M - 1) * K, x16 + (size_t)min(48 + c16, M - 1) * K};

    // The epilogue's outputs of this thread all lie in column tid % kNT (2048
    // outputs over a multiple of kNT threads): its scales are requested now,
    // not after the sums.
    float sc_a = 1.0f, sc_b = 1.0f;
    if (!part && scale) {
        const int col = tid % kNT;
        if (swiglu) {
            const int f = tile * (kNT / 2) + col;
            if (col < kNT / 2 && f < N / 2) {
                sc_a = scale[f];
                sc_b = scale[N / 2 + f];
            }
        } else if (tile * kNT + col < N) {
            sc_a = scale[tile * kNT + col];
        }
    }

    float4_t acc[2][4];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[t][r] = float4_t{0.f, 0.f, 0.f, 0.f};

    if (kb0 < kb1) {
        constexpr int DP = GK::DEPTH;
        GemmRound<KIND> r[DP];
#pragma unroll
        for (int d = 0; d < DP - 1; d++)
            if (kb0 + d * GK::NKB < kb1) gemm_issue<KIND>(r[d], kb0 + d * GK::NKB, kb1 - 1, K, wrow, wvalid, arow, g);
        for (int kb = kb0; kb < kb1; kb += DP * GK::NKB) {
#pragma unroll
            for (int d = 0; d < DP; d++) {
                // request the round DP-1 ahead into the buffer freed last, then multiply round d
                const int ki = kb + (d + DP - 1) * GK::NKB;
                if (ki < kb1) gemm_issue<KIND>(r[(d + DP - 1) % DP], ki, kb1 - 1, K, wrow, wvalid, arow, g);
                if (kb + d * GK::NKB < kb1) gemm_compute<KIND>(r[d], kb + d * GK::NKB, kb1, acc);
            }
        }
    }

    gemm_epilogue<NW>(acc, red, tid, M, N, tile, swiglu, epi, sc_a, sc_b, out_f32, out_f16, part);
}

// ---- k_gemm_p: k_gemm with the activation panel staged in LDS -------------
//
// The same tiles, K partition and reduction as k_gemm (so the same sums, bit
// for bit), but the block first requests all of its waves' weights, then
// stages the 64-row activation panel of its K split (at most kPanelK wide)
// in LDS with every load issued at once, and the waves read their MFMA A
// fragments from there.  k_gemm loads those fragments per wave in dependent
// rounds, so each wave of a block fetches its own share of the panel as it
// goes; here one round trip brings the whole panel and the weights.  The
// reduction buffer reuses the panel's LDS (gfx950: 160 KB per CU).
constexpr int kPanelK = 1024;
constexpr int kPanelRS = kPanelK / 8 + 1;   // uint4 per LDS panel row (16-byte pad)

template <int KIND>
__global__ __launch_bounds__(GemmKind<KIND>::WAVES * 64) void k_gemm_p(const uint16_t* __restrict__ x16,
                                                            int M, const uint8_t* __restrict__ w, int K,
                                                            int N, const float* scale, int epi,
                                                            float* out_f32, uint16_t* out_f16, float* part) {
    using GK = GemmKind<KIND>;
    constexpr int EPL = GK::EPL, KB = 4 * EPL, STEPS = EPL / 8;
    constexpr int NW = GK::WAVES;
    constexpr int KPW = (kPanelK / KB + NW - 1) / NW;   // K-blocks per wave at most
    static_assert(kMaxM * kPanelRS * 16 >= NW * kMaxM * kNT * 4, "the reduction fits the panel");
    __shared__ uint4 xs4[kMaxM * kPanelRS];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tile = blockIdx.x;
    const int swiglu = epi == 2;
    const int g = lane >> 4, c16 = lane & 15;
    const size_t row_bytes = KIND == MDX_W_F16 ? (size_t)K * 2 : (KIND == MDX_W_I8 ? (size_t)K : (size_t)K / 2);
    const int nkb_all = (K + KB - 1) / KB;   // the last K-block may be partial
    const int per_split = (nkb_all + gridDim.y - 1) / gridDim.y;
    const int sb0 = min(nkb_all, (int)blockIdx.y * per_split);
    const int sb1 = min(nkb_all, sb0 + per_split);
    const int per = (sb1 - sb0 + NW - 1) / NW;
    const int kb0 = min(sb1, sb0 + wave * per), kb1 = min(sb1, kb0 + per);

    // this wave's weights: K-blocks kb0 .. kb1-1 of the tile's two 16-row groups
    uint4 bw[KPW][2];
    {
        bool wvalid[2];
        const uint8_t* wrow[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int r = tile_row(tile, 16 * t + c16, swiglu, N);
            wvalid[t] = r < N;
            wrow[t] = w + (size_t)(wvalid[t] ? r : 0) * row_bytes;
        }
#pragma unroll
        for (int j = 0; j < KPW; j++) {
            const int kb = min(kb0 + j, kb1 - 1);
            const int k = (kb < kb0 ? kb0 : kb) * KB + g * EPL;
#pragma unroll
            for (int t = 0; t < 2; t++)
                bw[j][t] = (wvalid[t] && kb0 + j < kb1 && k < K) ? ld_w(wrow[t] + (size_t)k * 16 / EPL)
                                                                 : make_uint4(0u, 0u, 0u, 0u);
        }
    }
    float sc_a = 1.0f, sc_b = 1.0f;
    if (!part && scale) {
        const int col = tid % kNT;
        if (swiglu) {
            const int f = tile * (kNT / 2) + col;
            if (col < kNT / 2 && f < N / 2) {
                sc_a = scale[f];
                sc_b = scale[N / 2 + f];
            }
        } else if (tile * kNT + col < N) {
            sc_a = scale[tile * kNT + col];
        }
    }
    // the panel: 64 rows (rows >= M repeat row M-1) x this split's K range;
    // columns at or past K (a partial last K-block) are staged as zeros.  The
    // host never launches an empty split, so cpr >= 1.
    const int ks0 = sb0 * KB, kw = (sb1 - sb0) * KB;
    {
        constexpr int PER = kMaxM * (kPanelK / 8) / (NW * 64);
        static_assert(kMaxM * (kPanelK / 8) % (NW * 64) == 0, "panel split");
        const int cpr = kw / 8;                  // uint4 per panel row
        uint4 v[PER];
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int c = tid + i * NW * 64;
            const int row = c / cpr, col = c % cpr;
            const int rr = row < M ? row : M - 1;
            v[i] = (row < kMaxM && ks0 + 8 * col < K)
                       ? *reinterpret_cast<const uint4*>(x16 + (size_t)rr * K + ks0 + 8 * col)
                       : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int c = tid + i * NW * 64;
            const int row = c / cpr, col = c % cpr;
            if (row < kMaxM) xs4[row * kPanelRS + col] = v[i];
        }
    }
    __syncthreads();

    float4_t acc[2][4];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[t][r] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KPW; j++) {
        if (kb0 + j >= kb1) break;
        const int kl = (kb0 + j - sb0) * KB + g * EPL;   // k within the panel
        half8_t b[2][STEPS];
#pragma unroll
        for (int t = 0; t < 2; t++) widen_b<KIND>(bw[j][t], b[t]);
#pragma unroll
        for (int s = 0; s < STEPS; s++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const half8_t a = __builtin_bit_cast(half8_t, xs4[(16 * r + c16) * kPanelRS + kl / 8 + s]);
#pragma unroll
                for (int t = 0; t < 2; t++)
                    acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[t][s], acc[t][r], 0, 0, 0);
            }
    }
    __syncthreads();   // the panel's LDS is reused for the reduction
    gemm_epilogue<NW>(acc, reinterpret_cast<float (*)[kMaxM * kNT]>(xs4), tid, M, N, tile, swiglu, epi, sc_a,
                      sc_b, out_f32, out_f16, part);
}

// ---- projections, split-K over blocks: k_gemm_s -------------------------------
//
// The o and down projections (K a multiple of kKS, K / kKS <= kMaxSplits
// splits).  Block (tile, split) stages the activation panel X[64][kKS] of its
// split in LDS once (all 16-byte loads issued together), then each of its NW
// waves owns 16 output columns (weight rows) over the whole panel: no
// cross-wave reduction.  The weights of a wave are requested before the
// panel, so their HBM latency overlaps the staging.  The raw fp32 sums go to
// part[split][row][N] for k_residual_norm (which sums the splits in split
// order and applies the column scales), written as whole 256-byte row
// segments through LDS with 16-byte device-scope stores: in a standalone
// timeline of this kernel, 4-byte device-scope stores of the MFMA fragments
// took ~4 us per launch, these ~0.5 us.
constexpr int kKS = 256;

template <int KIND, int NW>
__global__ __launch_bounds__(NW * 64) void k_gemm_s(const uint16_t* __restrict__ x16, int M, int K,
                                                    const uint8_t* __restrict__ w, int N, float* part) {
    using GK = GemmKind<KIND>;
    constexpr int EPL = GK::EPL;               // k per 16-byte weight load
    constexpr int CK = 4 * EPL;                // k per chunk (4 lane groups)
    constexpr int NCH = kKS / CK;              // chunks per split
    constexpr int STEPS = EPL / 8;             // MFMA k-steps per chunk
    constexpr int RS = kKS / 8 + 1;            // uint4 per LDS panel row (16-byte pad)
    constexpr int OW = 16 * NW + 4;            // floats per LDS output row
    static_assert(kMaxM * RS * 16 >= kMaxM * OW * 4, "output tile fits the panel");
    __shared__ uint4 xs4[kMaxM * RS];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    // Blocks id, id + 8, id + 16, ... run on one XCD (one L2).  Each XCD takes a
    // contiguous run of (split, tile) pairs, so it fetches one or two splits'
    // activation panels instead of all of them.
    const int ntile = N / (16 * NW), nb = gridDim.x, id = blockIdx.x;
    const int gi = (nb & 7) ? id : (id & 7) * (nb >> 3) + (id >> 3);
    const int tile = gi % ntile, split = gi / ntile;
    const int k0 = split * kKS;
    const size_t row_bytes = KIND == MDX_W_F16 ? (size_t)K * 2 : (KIND == MDX_W_I8 ? (size_t)K : (size_t)K / 2);
    const int wrow = (tile * NW + wave) * 16 + c16;      // this lane's weight row
    uint4 wv[NCH];
    {
        const uint8_t* wr = w + (size_t)wrow * row_bytes + (size_t)(k0 + g * EPL) * 16 / EPL;
#pragma unroll
        for (int j = 0; j < NCH; j++) wv[j] = ld_w(wr + (size_t)j * CK * 16 / EPL);
    }
    // the panel: 64 rows (rows >= M repeat row M-1) x kKS fp16
    {
        constexpr int CHUNKS = kMaxM * (kKS / 8);
        constexpr int PER = CHUNKS / (NW * 64);
        static_assert(CHUNKS % (NW * 64) == 0, "panel split");
        uint4 v[PER];
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int c = tid + i * NW * 64;
            const int row = c / (kKS / 8), col = c % (kKS / 8);
            const int rr = row < M ? row : M - 1;
            v[i] = *reinterpret_cast<const uint4*>(x16 + (size_t)rr * K + k0 + 8 * col);
        }
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int c = tid + i * NW * 64;
            xs4[(c / (kKS / 8)) * RS + c % (kKS / 8)] = v[i];
        }
    }
    __syncthreads();
    float4_t acc[4];
#pragma unroll
    for (int r = 0; r < 4; r++) acc[r] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        half8_t b[STEPS];
        widen_b<KIND>(wv[j], b);
#pragma unroll
        for (int s = 0; s < STEPS; s++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                // A fragment: row 16r + c16, k = j*CK + g*EPL + 8s .. +7
                const half8_t a = __builtin_bit_cast(half8_t, xs4[(16 * r + c16) * RS + (j * CK + g * EPL) / 8 + s]);
                acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[s], acc[r], 0, 0, 0);
            }
    }
    __syncthreads();   // the panel is reused for the output tile
    float* ot = reinterpret_cast<float*>(xs4);
    // D fragment: lane holds column c16 of this wave's 16, rows 16r + 4g + i
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) ot[(16 * r + 4 * g + i) * OW + 16 * wave + c16] = acc[r][i];
    __syncthreads();
    constexpr int F4 = 4 * NW;                 // float4 per output row
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(part, (short)0, 0x7fffffff, 0x00020000);
    for (int idx = tid; idx < kMaxM * F4; idx += NW * 64) {
        const int row = idx / F4, c4 = idx % F4;
        if (row >= M) continue;
        const float4 v = *reinterpret_cast<const float4*>(ot + row * OW + 4 * c4);
        const size_t off = (((size_t)split * kMaxM + row) * N + (size_t)tile * 16 * NW + 4 * c4) * 4;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), rs, (unsigned)off, 0, 16);
    }
}

// Split-K finish for the o and down projections: y = sum of the split
// partials (split order) x scale; hidden += y (the residual); then the next
// RMSNorm of the row, x16 = fp16((hidden * rms) * norm_w) (skipped when norm_w
// is NULL).  grid = M rows, 256 threads.
constexpr int kMaxSplits = 16;

// R > 0: N == 1024 * R, thread t owns columns 4t..4t+3 (+1024 per round), and
// its hidden values stay in registers between the sum and the norm; the norm
// weights are requested with the partials, so the block waits for memory once.
// R == 0: any N (a multiple of 4), rounds looped at run time.
template <int R>
__global__ __launch_bounds__(256) void k_residual_norm(const float* part, int ns, int N,
                                                       const float* scale, float* hidden,
                                                       const float* norm_w, float eps,
                                                       uint16_t* x16) {
    __shared__ float ws[4];
    const int m = blockIdx.x, tid = threadIdx.x;
    float* hr = hidden + (size_t)m * N;
    float ss = 0.0f;
    constexpr int RK = R > 0 ? R : 1;
    float4 hv[RK], nwv[RK];
    // every load of a round is issued before any of them is used
#pragma unroll RK
    for (int r = 0, c = 4 * tid; R > 0 ? r < R : c < N; r++, c += 1024) {
        const int ri = R > 0 ? r : 0;
        if (norm_w) nwv[ri] = *reinterpret_cast<const float4*>(norm_w + c);
        float4 p[kMaxSplits];
#pragma unroll
        for (int sp = 0; sp < kMaxSplits; sp++)
            if (sp < ns) p[sp] = *reinterpret_cast<const float4*>(part + ((size_t)sp * kMaxM + m) * N + c);
        const float4 h0 = *reinterpret_cast<const float4*>(hr + c);
        const float4 sc = scale ? *reinterpret_cast<const float4*>(scale + c) : make_float4(1.f, 1.f, 1.f, 1.f);
        float4 y = p[0];
#pragma unroll
        for (int sp = 1; sp < kMaxSplits; sp++)
            if (sp < ns) {
                y.x = y.x + p[sp].x; y.y = y.y + p[sp].y; y.z = y.z + p[sp].z; y.w = y.w + p[sp].w;
            }
        float4 h;
        h.x = h0.x + y.x * sc.x; h.y = h0.y + y.y * sc.y; h.z = h0.z + y.z * sc.z; h.w = h0.w + y.w * sc.w;
        *reinterpret_cast<float4*>(hr + c) = h;
        hv[ri] = h;
        ss += h.x * h.x + h.y * h.y + h.z * h.z + h.w * h.w;
    }
    if (!norm_w) return;
    ss = wave_sum(ss);
    if ((tid & 63) == 0) ws[tid >> 6] = ss;
    __syncthreads();
    const float tot = ws[0] + ws[1] + ws[2] + ws[3];
    const float rms = 1.0f / sqrtf(tot / (float)N + eps);
#pragma unroll RK
    for (int r = 0, c = 4 * tid; R > 0 ? r < R : c < N; r++, c += 1024) {
        const float4 h = R > 0 ? hv[r] : *reinterpret_cast<const float4*>(hr + c);
        const float4 w = R > 0 ? nwv[r] : *reinterpret_cast<const float4*>(norm_w + c);
        uint2 o;
        o.x = (uint32_t)f32_to_f16_bits((h.x * rms) * w.x) | ((uint32_t)f32_to_f16_bits((h.y * rms) * w.y) << 16);
        o.y = (uint32_t)f32_to_f16_bits((h.z * rms) * w.z) | ((uint32_t)f32_to_f16_bits((h.w * rms) * w.w) << 16);
        *reinterpret_cast<uint2*>(x16 + (size_t)m * N + c) = o;
    }
}

// QK-norm + RoPE + append for M rows (reference: src/matmul_decoder.c:1984-2034,
// rope via the table formula of :620-631, identical to apply_rope_batch_f32).
// grid = (nq + 2*nkv, M), 64 threads; hd <= 256 (at most two pairs per lane).
constexpr int kRopePairs = 2;
__global__ __launch_bounds__(64) void k_qk_rope_append_rows(
    const mdx_state* st, const float* qkv, const float* part, int ns, const float* pscale,
    const float* q_norm, const float* k_norm, float eps, const float* cos_t, const float* sin_t,
    int nq, int nkv, int hd, int style, float* q_out, uint16_t* k_cache, uint16_t* v_cache) {
    const int b = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int pos = st->pos + t;
    const int half = hd / 2;
    const int qd = nq * hd, kvd = nkv * hd, nn = qd + 2 * kvd;
    // this block's head: columns [c0, c0 + hd) of the row
    const int c0 = b < nq ? b * hd : (b < nq + nkv ? qd + (b - nq) * hd : qd + kvd + (b - nq - nkv) * hd);
    __shared__ float rowv[2 * 64 * kRopePairs];
    const float* slice;
    if (part) {
        // the qkv GEMM's K-split partials, summed in split order, times the
        // column scale.  Lane elements e = lane + 64k (k < kRopeE, hd <= 256);
        // every load of a batch of kRopeS splits is issued before any is used
        // (indexes clamped to the slice's last column), so the block waits for
        // memory once per batch instead of once per split and element.
        constexpr int kRopeE = 4, kRopeS = 4;
        float acc[kRopeE], ps[kRopeE];
#pragma unroll
        for (int k = 0; k < kRopeE; k++) {
            const int e = min(lane + 64 * k, hd - 1);
            acc[k] = part[(size_t)t * nn + c0 + e];
            ps[k] = pscale ? pscale[c0 + e] : 1.0f;
        }
        for (int sp0 = 1; sp0 < ns; sp0 += kRopeS) {
            float p[kRopeS][kRopeE];
#pragma unroll
            for (int s = 0; s < kRopeS; s++)
#pragma unroll
                for (int k = 0; k < kRopeE; k++) {
                    const int sp = min(sp0 + s, ns - 1), e = min(lane + 64 * k, hd - 1);
                    p[s][k] = part[((size_t)sp * kMaxM + t) * nn + c0 + e];
                }
#pragma unroll
            for (int s = 0; s < kRopeS; s++)
                if (sp0 + s < ns)
#pragma unroll
                    for (int k = 0; k < kRopeE; k++) acc[k] = acc[k] + p[s][k];
        }
#pragma unroll
        for (int k = 0; k < kRopeE; k++) {
            const int e = lane + 64 * k;
            if (e < hd) rowv[e] = pscale ? acc[k] * ps[k] : acc[k];
        }
        __syncthreads();
        slice = rowv;
    } else {
        slice = qkv + (size_t)t * nn + c0;
    }
    if (b >= nq + nkv) {
        const int h = b - nq - nkv;
        const float* src = slice;
        uint16_t* dst = v_cache + (size_t)pos * kvd + h * hd;
        for (int e = lane; e < hd; e += 64) dst[e] = f32_to_f16_bits(src[e]);
        return;
    }
    const bool is_q = b < nq;
    const float* src = slice;
    const float* nw = is_q ? q_norm : k_norm;
    const float* cr = cos_t + (size_t)pos * half;
    const float* sr = sin_t + (size_t)pos * half;
    // this lane's pairs i = lane + 64k: elements, norm weights and table
    // values are all requested before the sum of squares, so the block
    // waits for memory once (measured: -0.4 us per layer at M = 60)
    float xa[kRopePairs], xb[kRopePairs], wa[kRopePairs], wb[kRopePairs], ca[kRopePairs], sa[kRopePairs];
#pragma unroll
    for (int k = 0; k < kRopePairs; k++) {
        const int i = lane + 64 * k < half ? lane + 64 * k : 0;
        const int i0 = style == 0 ? 2 * i : i;
        const int i1 = style == 0 ? 2 * i + 1 : i + half;
        xa[k] = src[i0];
        xb[k] = src[i1];
        wa[k] = nw ? nw[i0] : 1.0f;
        wb[k] = nw ? nw[i1] : 1.0f;
        ca[k] = cr[i];
        sa[k] = sr[i];
    }
    float rms = 1.0f;
    if (nw) {
        float ss = 0.0f;
        for (int e = lane; e < hd; e += 64) ss += src[e] * src[e];
        ss = wave_sum(ss);
        rms = 1.0f / sqrtf(ss / (float)hd + eps);
    }
#pragma unroll
    for (int k = 0; k < kRopePairs; k++) {
        const int i = lane + 64 * k;
        if (i >= half) break;
        const int i0 = style == 0 ? 2 * i : i;
        const int i1 = style == 0 ? 2 * i + 1 : i + half;
        float x0 = xa[k], x1 = xb[k];
        if (nw) {
            x0 = (x0 * rms) * wa[k];
            x1 = (x1 * rms) * wb[k];
        }
        const float c = ca[k], s = sa[k];
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
// own K/V).  grid = (nkv, M), 256 threads.  Positions [0, pos+t] go in rounds
// of PP passes; a pass gives each position HD/8 lanes (8 dimensions each).
// Every K/V row of a round is requested before any is used; scores of all
// passes, one workgroup-wide max per head, P.V summed over the position
// groups in LDS, and the rounds merged with the usual rescaling.
template <int LP>
__device__ __forceinline__ float lanes_sum(float v) {
    if constexpr (LP == 16) return row_sum16(v);
    else return group_sum(v, LP);
}

template <int HD, int G>
__global__ __launch_bounds__(256) void k_attn_prefill(const mdx_state* st, const float* q,
                                                      const uint16_t* kc, const uint16_t* vc,
                                                      int nkv, uint16_t* out16) {
    constexpr int LP = HD / 8;          // lanes per position
    constexpr int PPP = 256 / LP;       // positions per pass
    constexpr int PP = 4;               // passes per round
    constexpr int OPT = (G * HD + 255) / 256;   // outputs per thread
    __shared__ float qs[G * HD];
    __shared__ float att_m[PPP][G];
    __shared__ float att_l[PPP][G];
    extern __shared__ float att_o[];    // [PPP][G][HD]

    const int kvh = blockIdx.x, t = blockIdx.y;
    const int nq = nkv * G;
    const int L = st->pos + t + 1;
    const int tid = threadIdx.x;
    const int kvd = nkv * HD;
    const int pl = tid / LP, dl = tid % LP;
    const float scale = 1.0f / sqrtf((float)HD);
    // q is requested first and the first round's K/V rows right after it, so
    // the loads overlap (-0.4 us per layer at M = 60 against staging q
    // first) and, loads completing in issue order, staging q into LDS waits
    // for q alone while the K/V rows are still in flight (M = 60 INT8 prefill
    // 1.0934 -> 1.0874 ms against requesting the K/V rows first)
    constexpr int QPT = (G * HD + 255) / 256;
    float qv[QPT];
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int i = tid + 256 * k;
        qv[k] = i < G * HD ? q[(size_t)t * nq * HD + (size_t)kvh * G * HD + i] : 0.0f;
    }
    uint4 kk[PP], vv[PP];
    auto load_round = [&](int r0) {
#pragma unroll
        for (int qq = 0; qq < PP; qq++) {
            const int p = r0 + qq * PPP + pl;
            const int pc = p < L ? p : 0;
            kk[qq] = *reinterpret_cast<const uint4*>(kc + (size_t)pc * kvd + kvh * HD + dl * 8);
            vv[qq] = *reinterpret_cast<const uint4*>(vc + (size_t)pc * kvd + kvh * HD + dl * 8);
        }
    };
    load_round(0);
#pragma unroll
    for (int k = 0; k < QPT; k++)
        if (tid + 256 * k < G * HD) qs[tid + 256 * k] = qv[k];
    __syncthreads();
    float qr[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) qr[g][e] = qs[g * HD + dl * 8 + e];

    float runM[OPT], runL[OPT], runO[OPT];
#pragma unroll
    for (int j = 0; j < OPT; j++) { runM[j] = -INFINITY; runL[j] = 0.0f; runO[j] = 0.0f; }

    for (int r0 = 0; r0 < L; r0 += PP * PPP) {
        if (r0 > 0) load_round(r0);
        float sc[PP][G], mx[G];
#pragma unroll
        for (int g = 0; g < G; g++) mx[g] = -INFINITY;
#pragma unroll
        for (int qq = 0; qq < PP; qq++) {
            const half2_t k01 = as_h2(kk[qq].x), k23 = as_h2(kk[qq].y), k45 = as_h2(kk[qq].z),
                          k67 = as_h2(kk[qq].w);
            const float kf[8] = {(float)k01.x, (float)k01.y, (float)k23.x, (float)k23.y,
                                 (float)k45.x, (float)k45.y, (float)k67.x, (float)k67.y};
            const bool valid = r0 + qq * PPP + pl < L;
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float* qh = qr[g];
                float sv = ((qh[0] * kf[0] + qh[1] * kf[1]) + (qh[2] * kf[2] + qh[3] * kf[3])) +
                           ((qh[4] * kf[4] + qh[5] * kf[5]) + (qh[6] * kf[6] + qh[7] * kf[7]));
                sv = lanes_sum<LP>(sv) * scale;
                sc[qq][g] = valid ? sv : -INFINITY;
                mx[g] = fmaxf(mx[g], sc[qq][g]);
            }
        }
        if (dl == 0)
#pragma unroll
            for (int g = 0; g < G; g++) att_m[pl][g] = mx[g];
        __syncthreads();
        float Mr[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float v = att_m[0][g];
            for (int i = 1; i < PPP; i++) v = fmaxf(v, att_m[i][g]);
            Mr[g] = v;
        }
        float ls[G], o[G][8];
#pragma unroll
        for (int g = 0; g < G; g++) {
            ls[g] = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) o[g][e] = 0.0f;
        }
#pragma unroll
        for (int qq = 0; qq < PP; qq++) {
            const half2_t v01 = as_h2(vv[qq].x), v23 = as_h2(vv[qq].y), v45 = as_h2(vv[qq].z),
                          v67 = as_h2(vv[qq].w);
            const float vf[8] = {(float)v01.x, (float)v01.y, (float)v23.x, (float)v23.y,
                                 (float)v45.x, (float)v45.y, (float)v67.x, (float)v67.y};
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float p = sc[qq][g] == -INFINITY ? 0.0f : expf(sc[qq][g] - Mr[g]);
                ls[g] = ls[g] + p;
#pragma unroll
                for (int e = 0; e < 8; e++) o[g][e] = o[g][e] + p * vf[e];
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
#pragma unroll
            for (int e = 0; e < 8; e++) att_o[(pl * G + g) * HD + dl * 8 + e] = o[g][e];
            if (dl == 0) att_l[pl][g] = ls[g];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < OPT; j++) {
            const int oi = tid + 256 * j;
            if (oi < G * HD) {
                const int g = oi / HD, d = oi % HD;
                float Ox = 0.0f, Lx = 0.0f;
                for (int i = 0; i < PPP; i++) {
                    Ox = Ox + att_o[(i * G + g) * HD + d];
                    Lx = Lx + att_l[i][g];
                }
                const float M2 = Mr[g];
                const float Mn = fmaxf(runM[j], M2);
                if (Mn != -INFINITY) {
                    const float a = runM[j] == -INFINITY ? 0.0f : expf(runM[j] - Mn);
                    const float b = M2 == -INFINITY ? 0.0f : expf(M2 - Mn);
                    runL[j] = runL[j] * a + Lx * b;
                    runO[j] = runO[j] * a + Ox * b;
                    runM[j] = Mn;
                }
            }
        }
        __syncthreads();   // att_* are rewritten by the next round
    }
#pragma unroll
    for (int j = 0; j < OPT; j++) {
        const int oi = tid + 256 * j;
        if (oi < G * HD) {
            const int g = oi / HD, d = oi % HD;
            out16[(size_t)t * nq * HD + (size_t)(kvh * G + g) * HD + d] = f32_to_f16_bits(runO[j] / runL[j]);
        }
    }
}

__global__ void k_copy_row(const float* x, int row, int d, float* dst) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < d; i += gridDim.x * blockDim.x)
        dst[i] = x[(size_t)row * d + i];
}

}  // namespace

// k_gemm_s serves the shape: K a multiple of kKS with at most kMaxSplits
// splits, N a multiple of the 64 columns of a block (4 waves).
static bool gemm_s_ok(int M, const mdx_wdesc* w) {
    return M > 0 && M <= kMaxM && w->K % kKS == 0 && w->K / kKS <= kMaxSplits && w->N % 64 == 0;
}

static int gemm_s_launch(const uint16_t* x16, int M, const mdx_wdesc* w, float* part, void* stream) {
    dim3 grid((w->N / 64) * (w->K / kKS));   // (split, tile) pairs, decoded in the kernel
    const uint8_t* wp = (const uint8_t*)w->w;
    hipStream_t s = (hipStream_t)stream;
    switch (w->kind) {
        case MDX_W_F16:
            hipLaunchKernelGGL((k_gemm_s<MDX_W_F16, 4>), grid, dim3(256), 0, s, x16, M, w->K, wp, w->N, part);
            break;
        case MDX_W_I8:
            hipLaunchKernelGGL((k_gemm_s<MDX_W_I8, 4>), grid, dim3(256), 0, s, x16, M, w->K, wp, w->N, part);
            break;
        case MDX_W_I4:
            hipLaunchKernelGGL((k_gemm_s<MDX_W_I4, 4>), grid, dim3(256), 0, s, x16, M, w->K, wp, w->N, part);
            break;
        default:
            return -5;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

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

static int gemm_tiles(int N, int swiglu) {
    return swiglu ? (N / 2 + kNT / 2 - 1) / (kNT / 2) : (N + kNT - 1) / kNT;
}

// K per K-block of k_gemm / k_gemm_p (4 lane groups of one 16-byte load).
static int gemm_kblock(int kind) { return kind == MDX_W_F16 ? 32 : (kind == MDX_W_I8 ? 64 : 128); }

// K splits of a residual projection: about 256 blocks in all, at least two
// K-blocks of the widest kind per split.  The count is then reduced so that
// no split is empty: the kernels give split s the K-blocks
// [s * per, (s + 1) * per) with per = ceil(nkb / ns), and every split's
// consumer sums exactly ns partials.
static int residual_splits(int kind, int N, int K) {
    const int tiles = gemm_tiles(N, 0);
    int ns = (256 + tiles - 1) / tiles;
    const int max_ns = K / 256 > 0 ? K / 256 : 1;
    if (ns > max_ns) ns = max_ns;
    if (ns > kMaxSplits) ns = kMaxSplits;
    if (ns < 1) ns = 1;
    const int kb = gemm_kblock(kind), nkb = (K + kb - 1) / kb;
    if (ns > nkb) ns = nkb;
    const int per = (nkb + ns - 1) / ns;
    return (nkb + per - 1) / per;
}

int mdx_debug_gemm_splits(int kind, int N, int K, int* per_split) {
    if (kind < MDX_W_F16 || kind > MDX_W_I4 || N <= 0 || K <= 0) return -1;
    const int ns = residual_splits(kind, N, K);
    const int kb = gemm_kblock(kind), nkb = (K + kb - 1) / kb;
    if (per_split) *per_split = (nkb + ns - 1) / ns;
    return ns;
}

size_t mdx_gemm_scratch_floats(int M, int N, int K) {
    (void)M;
    int nsm = 1;
    for (int kind = MDX_W_F16; kind <= MDX_W_I4; kind++) {
        const int ns = residual_splits(kind, N, K);
        if (ns > nsm) nsm = ns;
    }
    const size_t a = (size_t)nsm * kMaxM * N;
    const size_t b = K % kKS == 0 ? (size_t)(K / kKS) * kMaxM * N : 0;
    return a > b ? a : b;
}



// Test hook: 1 selects k_gemm (fragments loaded in rounds) where k_gemm_p
// would serve.  Not thread-safe: set it before the contexts it is meant for
// capture their prefill graphs.
static int g_gemm_rounds = 0;

static int gemm_launch(const uint16_t* x16, int M, const mdx_wdesc* w, int epilogue, void* out,
                       float* part, int ns, void* stream) {
    if (w->kind < MDX_W_F16 || w->kind > MDX_W_I4) return -5;
    const int kb = gemm_kblock(w->kind);
    // K a multiple of one lane group's 16-byte load (the last K-block may be partial)
    if (M <= 0 || M > kMaxM || w->K <= 0 || w->K % (kb / 4) != 0) return -1;
    // exactly one destination: split partials, or the epilogue's output
    if (part ? (ns < 1 || out != nullptr) : (ns != 1 || out == nullptr)) return -1;
    if (epilogue == 2 && w->N % 2) return -1;
    dim3 grid(gemm_tiles(w->N, epilogue == 2), ns);
    const int waves = w->kind == MDX_W_F16 ? GemmKind<MDX_W_F16>::WAVES
                      : w->kind == MDX_W_I8 ? GemmKind<MDX_W_I8>::WAVES : GemmKind<MDX_W_I4>::WAVES;
    dim3 block(waves * 64);
    const uint8_t* wp = (const uint8_t*)w->w;
    float* of = (float*)out;
    uint16_t* oh = (uint16_t*)out;
    // The panel kernel when every split's K range fits the LDS panel: for the
    // SwiGLU GEMM (M=60, one split of 1024: fp16 11.80 -> 10.58 us per launch,
    // int8 9.23 -> 8.96, int4 9.03 -> 8.46) and, with fp16 weights, for split
    // partials (qkv, two splits of 512: 7.42 -> 7.33 us; int8 and int4 6.03 ->
    // 6.39 and 6.01 -> 6.20, so those keep k_gemm).
    const int nkb = (w->K + kb - 1) / kb, per_split = (nkb + ns - 1) / ns;
    if ((ns - 1) * per_split >= nkb) return -1;   // an empty split
    const bool panel = per_split * kb <= kPanelK && (epilogue == 2 || w->kind == MDX_W_F16);
    if (panel && !g_gemm_rounds) {
        switch (w->kind) {
            case MDX_W_F16:
                hipLaunchKernelGGL(k_gemm_p<MDX_W_F16>, grid, block, 0, (hipStream_t)stream, x16, M, wp,
                                   w->K, w->N, w->scale, epilogue, of, oh, part);
                break;
            case MDX_W_I8:
                hipLaunchKernelGGL(k_gemm_p<MDX_W_I8>, grid, block, 0, (hipStream_t)stream, x16, M, wp,
                                   w->K, w->N, w->scale, epilogue, of, oh, part);
                break;
            case MDX_W_I4:
                hipLaunchKernelGGL(k_gemm_p<MDX_W_I4>, grid, block, 0, (hipStream_t)stream, x16, M, wp,
                                   w->K, w->N, w->scale, epilogue, of, oh, part);
                break;
            default:
                return -5;
        }
        return hipGetLastError() == hipSuccess ? 0 : -4;
    }
    switch (w->kind) {
        case MDX_W_F16:
            hipLaunchKernelGGL(k_gemm<MDX_W_F16>, grid, block, 0, (hipStream_t)stream, x16, M, wp, w->K,
                               w->N, w->scale, epilogue, of, oh, part);
            break;
        case MDX_W_I8:
            hipLaunchKernelGGL(k_gemm<MDX_W_I8>, grid, block, 0, (hipStream_t)stream, x16, M, wp, w->K,
                               w->N, w->scale, epilogue, of, oh, part);
            break;
        case MDX_W_I4:
            hipLaunchKernelGGL(k_gemm<MDX_W_I4>, grid, block, 0, (hipStream_t)stream, x16, M, wp, w->K,
                               w->N, w->scale, epilogue, of, oh, part);
            break;
        default:
            return -5;
    }
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int mdx_debug_gemm_rounds(int on) {
    const int old = g_gemm_rounds;
    g_gemm_rounds = on != 0;
    return old;
}

int mdx_launch_gemm(const uint16_t* x16, int M, const mdx_wdesc* w, int epilogue, void* out,
                    float* scratch, void* stream) {
    (void)scratch;
    return gemm_launch(x16, M, w, epilogue, out, nullptr, 1, stream);
}
int mdx_launch_gemm_residual_norm(const uint16_t* x16, int M, const mdx_wdesc* w, float* hidden,
                                  const float* norm_w, float eps, uint16_t* x16_out, float* scratch,
                                  void* stream) {
    if (w->N % 4) return -1;   // float4 rows in k_residual_norm
    int ns, rc;
    if (gemm_s_ok(M, w)) {
        ns = w->K / kKS;
        rc = gemm_s_launch(x16, M, w, scratch, stream);
    } else {
        ns = residual_splits(w->kind, w->N, w->K);
        rc = gemm_launch(x16, M, w, 0, nullptr, scratch, ns, stream);
    }
    if (rc) return rc;
    const int R = w->N % 1024 == 0 ? w->N / 1024 : 0;
    auto kern = R == 1 ? k_residual_norm<1> : R == 2 ? k_residual_norm<2> : R == 4 ? k_residual_norm<4>
                                                                                  : k_residual_norm<0>;
    hipLaunchKernelGGL(kern, dim3(M), dim3(256), 0, (hipStream_t)stream, scratch, ns, w->N, w->scale,
                       hidden, norm_w, eps, x16_out);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int mdx_launch_qk_rope_append_rows(const mdx_state* state, const float* qkv, int M,
                                   const float* q_norm, const float* k_norm, float eps,
                                   const float* cos_t, const float* sin_t, int nq, int nkv,
                                   int hd, int rope_style, float* q_out, uint16_t* k_cache,
                                   uint16_t* v_cache, void* stream) {
    if (hd % 2 || hd > 2 * 64 * kRopePairs || M <= 0) return -1;
    hipLaunchKernelGGL(k_qk_rope_append_rows, dim3(nq + 2 * nkv, M), dim3(64), 0, (hipStream_t)stream,
                       state, qkv, (const float*)nullptr, 0, (const float*)nullptr, q_norm, k_norm, eps,
                       cos_t, sin_t, nq, nkv, hd, rope_style, q_out, k_cache, v_cache);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int mdx_launch_qkv_rope_append_rows(const uint16_t* x16, int M, const mdx_wdesc* w, float* scratch,
                                    const mdx_state* state, const float* q_norm, const float* k_norm,
                                    float eps, const float* cos_t, const float* sin_t, int nq, int nkv,
                                    int hd, int rope_style, float* q_out, uint16_t* k_cache,
                                    uint16_t* v_cache, void* stream) {
    if (hd % 2 || hd > 2 * 64 * kRopePairs || M <= 0 || w->N != (nq + 2 * nkv) * hd) return -1;
    const int ns = residual_splits(w->kind, w->N, w->K);
    int rc = gemm_launch(x16, M, w, 0, nullptr, scratch, ns, stream);
    if (rc) return rc;
    hipLaunchKernelGGL(k_qk_rope_append_rows, dim3(nq + 2 * nkv, M), dim3(64), 0, (hipStream_t)stream,
                       state, (const float*)nullptr, (const float*)scratch, ns, w->scale, q_norm, k_norm,
                       eps, cos_t, sin_t, nq, nkv, hd, rope_style, q_out, k_cache, v_cache);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int mdx_launch_attn_prefill(const mdx_state* state, const float* q, int M,
                            const uint16_t* k_cache, const uint16_t* v_cache, int nq, int nkv,
                            int hd, uint16_t* out16, void* stream) {
    if (nkv <= 0 || nq % nkv || M <= 0) return -1;
    const int G = nq / nkv;
    const int LP = hd / 8;
    const int PPP = 256 / (LP > 0 ? LP : 1);
    const size_t lds = (size_t)PPP * G * hd * 4;
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
