// mdx_prefill_xg.hip — batch prefill (M <= 64 rows) of the Qwen3-0.6B layer
// shape (d 1024, 16 query / 8 KV heads of 128, FFN 3072) in two launches per
// layer, for gfx950.
//
// Reference: src/matmul_decoder.c:1841-2065 (matmul_decoder_prefill_batch):
// per layer RMSNorm, q|k|v projections, QK-norm, RoPE (table formula
// :620-631), K/V append, causal GQA attention (src/cpu_ops.c:459-571), o +
// residual, RMSNorm, gate|up, SwiGLU, down + residual.
//
// The 256 workgroups (one per CU, 8 waves each) form 8 groups: group j =
// b % 8 owns KV head j and FFN features [384j, 384j + 384).  Dispatch places
// workgroups b, b + 8, ... on one XCD, so a group's exchanges stay in that
// XCD's L2.  Each launch starts from the previous launch's 8 K-split
// partials (one per group), which every group sums for itself:
//
//   k_prefill_attn (one launch per layer)
//     N  workgroup c: rows 2c, 2c + 1: the previous down partials summed in
//        group order, x scale, + residual (layer 0: the input rows), the
//        input RMSNorm -> fp16 rows to the group; group 0 writes the new
//        residual rows
//     Q  workgroup (g, s): 64 of the group's 512 q|k|v columns (query heads
//        2j, 2j+1, KV head j) over K split s (256 of 1024), on MFMA from the
//        fp16 panel in LDS; fp32 partials to the group
//     R  workgroup (head slot, 8 rows): the 4 split partials summed in split
//        order, the column scale, QK-norm, RoPE, K/V appended to the cache
//     A  workgroup c: rows c (waves 0-3) and 63 - c (waves 4-7) at once,
//        both query heads, causal attention over the cache rows before the
//        chunk and the group's new K/V rows
//     O  workgroup c: 32 o columns over the group's 256 attention dimensions
//        (its K slice of o): the group's K-split partial of o
//   k_prefill_mlp (one launch per layer)
//     N  as above with the o partials and the post-attention RMSNorm
//     G  workgroup (tile group, s): gate and up rows of 48 of the group's 384
//        features over K split s; fp32 partials to the group
//     S  workgroup c: rows 2c, 2c + 1: splits summed, scales, SwiGLU, fp16
//     D  workgroup c: 32 down columns over the group's 384 features: the
//        group's K-split partial of down
// After the last layer k_residual_norm (mdx_prefill.hip) adds the down
// partials to the residual rows without a norm.
//
// Exchanges inside a launch use LL words: 32-bit words of 16 payload bits
// and a 16-bit epoch, written with plain stores (through the CU's
// write-through L1 into the L2) and polled with non-temporal loads (which do
// not hit a stale L1 line).  A reader accepts a word only when its epoch is
// the current one, so no flag, fence or barrier is needed; fp32 values take
// two words.  Every wait is bounded: a workgroup that gives up sets the status
// word, stops waiting, and the host runs the chunk again on the eight-launch
// path (which needs no co-location).  The epoch changes with every layer and
// every prefill (a counter that the end-of-prefill kernel advances).
#include <hip/hip_runtime.h>

#include <cmath>

#include "mdx_common.h"
#include "mdx_device.h"
#include "mdx_gemm_tile.h"

using namespace mdx;

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int D = 1024, NQ = 16, NKV = 8, HD = 128, FF = 3072;
constexpr int QD = NQ * HD, KVD = NKV * HD;
constexpr int NB = 256;          // workgroups
constexpr int NT = 512;          // threads per workgroup (8 waves)
constexpr int MR = 64;           // rows of a chunk (M padded)
constexpr int GF = FF / NKV;     // FFN features per group
constexpr unsigned kSpin = 1u << 18;   // polling rounds before a wait gives up

// ---- exchange words of one group --------------------------------------------
// XN [row 64][1024] fp16: the normed rows of the launch (both launches)
constexpr int X_XN = 0;
// QP [split 4][head slot 4][row 64][col 64][half 2][word 2]: Q partials; lane
//    i of an R wave reads columns i and 64 + i of one row in one 16-byte load
constexpr int X_QP = X_XN + MR * D;
constexpr int X_RQ = X_QP + 4 * 4 * MR * 64 * 2 * 2;   // [row][head 2][128][word 2]: q after RoPE
constexpr int X_KV = X_RQ + MR * 2 * HD * 2;           // [row][256] fp16: K (0..127) | V
constexpr int X_AO = X_KV + MR * 2 * HD;               // [row][256] fp16: attention output
constexpr int X_ATTN_END = X_AO + MR * 2 * HD;
// GP [split 4][row 64][feature 384][gate, up][word 2]: G partials
constexpr int X_GP = X_XN + MR * D;
constexpr int X_SA = X_GP + 4 * MR * GF * 2 * 2;       // [row][384] fp16: SwiGLU output
constexpr int X_MLP_END = X_SA + MR * GF;
constexpr int X_GROUP = X_ATTN_END > X_MLP_END ? X_ATTN_END : X_MLP_END;
// header: [0] prefill counter (epoch source), [1] status (1: a wait timed out),
// [2] polling rounds before a wait gives up (0: kSpin; a test hook)
constexpr int X_HDR = 64;
constexpr size_t X_BYTES = (size_t)(X_HDR + NKV * X_GROUP) * 4;
static_assert(X_QP % 4 == 0 && X_RQ % 4 == 0 && X_KV % 4 == 0 && X_AO % 4 == 0 && X_GP % 4 == 0 &&
              X_SA % 4 == 0 && X_GROUP % 4 == 0, "16-byte aligned regions");

// stage ids of the epochs
// (stage R writes the q rows and the K/V rows: one epoch, SID_R)
enum { SID_QP = 0, SID_R = 2, SID_AO = 3, SID_GP = 4, SID_SA = 5, SID_XA = 6, SID_XM = 7, SID_N = 8 };

__device__ __forceinline__ unsigned xg_epoch(unsigned E, int L, int layer, int sid) {
    const unsigned long long v = ((unsigned long long)E * (unsigned)L + (unsigned)layer) * SID_N + (unsigned)sid;
    return (unsigned)(v % 65535ull) + 1u;
}

__device__ __forceinline__ unsigned ll_word(unsigned payload, unsigned ep) { return (payload & 0xffffu) | (ep << 16); }
__device__ __forceinline__ u32x2 ll_f32x(float v, unsigned ep) {
    const unsigned u = __float_as_uint(v);
    u32x2 r;
    r.x = ll_word(u, ep);
    r.y = ll_word(u >> 16, ep);
    return r;
}
__device__ __forceinline__ float ll_f32(unsigned lo, unsigned hi) {
    return __uint_as_float((lo & 0xffffu) | (hi << 16));
}
__device__ __forceinline__ bool ll_ok4(u32x4 v, unsigned ep) {
    return ((v.x >> 16) == ep) & ((v.y >> 16) == ep) & ((v.z >> 16) == ep) & ((v.w >> 16) == ep);
}

// Plain stores into the group's words (the L2 of the XCD the group shares).
__device__ __forceinline__ void xst2(__amdgpu_buffer_rsrc_t rs, int word, u32x2 v) {
    __builtin_amdgcn_raw_buffer_store_b64(v, rs, word * 4, 0, 0);
}
__device__ __forceinline__ void xst1(__amdgpu_buffer_rsrc_t rs, int word, unsigned v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, rs, word * 4, 0, 0);
}
// Non-temporal 16-byte poll (aux 2): reads the L2, not a stale L1 line.
__device__ __forceinline__ u32x4 xld4(__amdgpu_buffer_rsrc_t rs, int word) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, word * 4, 0, 2);
}

// Polls N 16-byte groups until every word carries epoch ep.  Returns false
// after `limit` rounds (the caller marks itself dead and stops waiting).
template <int N>
__device__ __forceinline__ bool xwait(__amdgpu_buffer_rsrc_t rs, const int (&word)[N], u32x4 (&v)[N],
                                      unsigned ep, bool dead, unsigned limit) {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = xld4(rs, word[i]);
    if (dead) return true;
    for (unsigned spin = 0;; spin++) {
        asm volatile("" ::: "memory");
        bool all = true;
#pragma unroll
        for (int i = 0; i < N; i++) {
            if (!ll_ok4(v[i], ep)) {
                all = false;
                v[i] = xld4(rs, word[i]);
            }
        }
        if (all) return true;
        if (spin > limit) return false;
    }
}

// Polls the group word[P] alone until it carries epoch ep, then requests all
// N groups and waits for the rest.  A thread that needs many groups from
// producers that finish together keeps one request in flight while they
// work instead of re-requesting every group each round, which would flood
// the XCD's L2 with polls.
template <int N, int P = 0>
__device__ __forceinline__ bool xwait_probe(__amdgpu_buffer_rsrc_t rs, const int (&word)[N], u32x4 (&v)[N],
                                            unsigned ep, bool dead, unsigned limit) {
    if (!dead) {
        u32x4 p = xld4(rs, word[P]);
        for (unsigned spin = 0; !ll_ok4(p, ep); spin++) {
            asm volatile("" ::: "memory");
            if (spin > limit) return false;
            p = xld4(rs, word[P]);
        }
    }
    return xwait<N>(rs, word, v, ep, dead, limit);
}

__device__ __forceinline__ void store_wt(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- MFMA tiles ---------------------------------------------------------------

template <int KIND>
__device__ __forceinline__ size_t row_bytes_of(int K) {
    return KIND == MDX_W_F16 ? (size_t)K * 2 : (KIND == MDX_W_I8 ? (size_t)K : (size_t)K / 2);
}

// One wave's weights for one 16-column tile: NKB K-blocks from k0 (lane group
// g takes k0 + j*KB + g*EPL), non-temporal 16-byte loads.
template <int KIND, int NKB>
__device__ __forceinline__ void load_b(uint4 (&bw)[NKB], const uint8_t* w, int row, int K, int k0, int lane) {
    constexpr int EPL = GemmKind<KIND>::EPL, KB = 4 * EPL;
    const uint8_t* wr = w + (size_t)row * row_bytes_of<KIND>(K);
#pragma unroll
    for (int j = 0; j < NKB; j++) {
        const int k = k0 + j * KB + (lane >> 4) * EPL;
        bw[j] = ld_nt(wr + (size_t)k * 16 / EPL);
    }
}

// acc[r] (rows 16r.., the wave's 16 columns) += panel[64][kofs..] . B: A
// fragments from the fp16 panel in LDS (PITCH uint4 per row).
template <int KIND, int NKB, int PITCH>
__device__ __forceinline__ void wave_mma(float4_t (&acc)[4], const uint4 (&bw)[NKB], const uint4* panel, int kofs,
                                         int lane) {
    constexpr int EPL = GemmKind<KIND>::EPL, KB = 4 * EPL, STEPS = EPL / 8;
    const int g = lane >> 4, c16 = lane & 15;
#pragma unroll
    for (int j = 0; j < NKB; j++) {
        half8_t b[STEPS];
        widen_b<KIND>(bw[j], b);
        const int kl = kofs + j * KB + g * EPL;
#pragma unroll
        for (int s = 0; s < STEPS; s++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const half8_t a = __builtin_bit_cast(half8_t, panel[(16 * r + c16) * PITCH + kl / 8 + s]);
                acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[s], acc[r], 0, 0, 0);
            }
    }
}

__device__ __forceinline__ void zero_acc(float4_t (&acc)[4]) {
#pragma unroll
    for (int r = 0; r < 4; r++) acc[r] = float4_t{0.f, 0.f, 0.f, 0.f};
}

// Stages columns [c0, c0 + COLS) of an LL fp16 exchange region [64][RSTRIDE]
// (rows >= M as zeros) into an LDS panel of PITCH uint4 per row: NL 16-byte
// polls per thread (4 values each), issued together.
template <int COLS, int RSTRIDE, int PITCH>
__device__ __forceinline__ bool stage_ll_panel(uint4* panel, __amdgpu_buffer_rsrc_t rs, int base, int c0, int M,
                                               unsigned ep, bool dead, unsigned limit, int t) {
    constexpr int NL = MR * COLS / 4 / NT;
    static_assert(MR * COLS % (4 * NT) == 0, "panel split");
    int wd[NL];
    u32x4 v[NL];
    const int m4 = M * COLS / 4;    // groups of 4 words in the rows < M
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int q = t + NT * i, qq = q < m4 ? q : 0;
        wd[i] = base + ((4 * qq) / COLS) * RSTRIDE + c0 + (4 * qq) % COLS;
    }
    const bool ok = xwait_probe<NL, NL - 1>(rs, wd, v, ep, dead, limit);
    uint2* p2 = reinterpret_cast<uint2*>(panel);
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int q = t + NT * i, row = (4 * q) / COLS, col = (4 * q) % COLS;
        uint2 h;
        h.x = q < m4 ? ((v[i].x & 0xffffu) | (v[i].y << 16)) : 0u;
        h.y = q < m4 ? ((v[i].z & 0xffffu) | (v[i].w << 16)) : 0u;
        p2[(row * PITCH * 16 + col * 2) / 8] = h;
    }
    return ok;
}

struct XgArgs {
    const uint16_t* x16;      // plain mode: [M][1024] fp16 normed input rows (no N stage), else NULL
    const mdx_state* st;
    int M, n_layers, layer, rope_style;
    float eps;
    const float* h_in;        // [64][1024] residual rows entering the launch
    float* h_out;             // [64][1024] the rows after the residual add (group 0 writes them)
    const float* part_in;     // [8][64][1024] the previous half's K-split partials, or NULL (layer 0)
    const float* scale_in;    // their column scales, or NULL
    const float* norm_w;      // the RMSNorm of the launch's input rows
    const uint8_t* w1;        // q|k|v rows (attention half) or gate|up rows (FFN half)
    const float* s1;
    const uint8_t* w2;        // o rows or down rows
    const float* q_norm;
    const float* k_norm;
    const float* cos_t;
    const float* sin_t;
    uint16_t* kc;             // layer caches [max_seq][1024]
    uint16_t* vc;
    float* part_out;          // [8][64][1024] this half's K-split partials (group j: split j)
    unsigned* xbuf;           // header + 8 groups of exchange words
    unsigned long long* trace;   // optional [layer][2 launches][256][16] 100 MHz timestamps
};

// Timestamp ev of this workgroup (thread 0) when tracing: launch 0 is the
// attention half, 1 the FFN half.
#define XG_TRACE(half, ev)                                                                          \
    do {                                                                                            \
        if (a.trace && threadIdx.x == 0)                                                            \
            a.trace[(((size_t)a.layer * 2 + (half)) * NB + blockIdx.x) * 16 + (ev)] = wall_clock64(); \
    } while (0)

// N: rows 2c, 2c + 1 of h = h_in + (sum of the 8 partials in group order) x
// scale (src/cpu_ops.c:296-359 residual), then x16 = fp16((h * rms) * w)
// (src/cpu_ops.c:18-55) to the group's XN words; group 0 stores h to h_out.
// Thread t owns columns 4 (t & 255) .. +3 of row 2c + (t >> 8).  Split in two
// so that the partials are requested before the stage's weights: nload issues
// every load, nfinish uses them.
// Plain mode: stages x16[row][k0 .. k0 + 256) (rows >= M as zeros) into an LDS
// panel of PITCH uint4 per row: 4 uint4 per thread, all requested together.
template <int PITCH>
__device__ __forceinline__ void stage_plain256(uint4* panel, const uint16_t* x16, int M, int k0, int t) {
    uint4 v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = t + NT * i, row = q >> 5, col = q & 31;
        v[i] = row < M ? *reinterpret_cast<const uint4*>(x16 + (size_t)row * D + k0 + 8 * col)
                       : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = t + NT * i;
        panel[(q >> 5) * PITCH + (q & 31)] = v[i];
    }
}

struct NRows {
    float4 h, p[8], sc, nw;
};
__device__ __forceinline__ void stage_norm_load(const XgArgs& a, int c, int t, NRows& n) {
    const int col = 4 * (t & 255);
    const int row = min(2 * c + (t >> 8), a.M - 1);
    n.h = *reinterpret_cast<const float4*>(a.h_in + (size_t)row * D + col);
    if (a.part_in) {
#pragma unroll
        for (int sp = 0; sp < 8; sp++)
            n.p[sp] = *reinterpret_cast<const float4*>(a.part_in + ((size_t)sp * MR + row) * D + col);
    }
    n.sc = a.scale_in ? *reinterpret_cast<const float4*>(a.scale_in + col) : make_float4(1.f, 1.f, 1.f, 1.f);
    n.nw = *reinterpret_cast<const float4*>(a.norm_w + col);
}
__device__ __forceinline__ void stage_norm_finish(const XgArgs& a, __amdgpu_buffer_rsrc_t rs, unsigned ep, int j,
                                                  int c, int t, NRows& n, float (*ss_red)[4]) {
    const int col = 4 * (t & 255), rr = t >> 8, wave = t >> 6;
    const int row = 2 * c + rr;
    float4 h = n.h;
    if (a.part_in) {
        float4 y = n.p[0];
#pragma unroll
        for (int sp = 1; sp < 8; sp++) {
            y.x = y.x + n.p[sp].x;
            y.y = y.y + n.p[sp].y;
            y.z = y.z + n.p[sp].z;
            y.w = y.w + n.p[sp].w;
        }
        h.x = h.x + y.x * n.sc.x;
        h.y = h.y + y.y * n.sc.y;
        h.z = h.z + y.z * n.sc.z;
        h.w = h.w + y.w * n.sc.w;
    }
    const float ss = wave_sum(h.x * h.x + h.y * h.y + h.z * h.z + h.w * h.w);
    if ((t & 63) == 0) ss_red[rr][wave & 3] = ss;
    __syncthreads();
    if (row < a.M) {
        const float tot = (ss_red[rr][0] + ss_red[rr][1]) + (ss_red[rr][2] + ss_red[rr][3]);
        const float rms = 1.0f / sqrtf(tot / (float)D + a.eps);
        u32x2 o0, o1;
        o0.x = ll_word(f32_to_f16_bits((h.x * rms) * n.nw.x), ep);
        o0.y = ll_word(f32_to_f16_bits((h.y * rms) * n.nw.y), ep);
        o1.x = ll_word(f32_to_f16_bits((h.z * rms) * n.nw.z), ep);
        o1.y = ll_word(f32_to_f16_bits((h.w * rms) * n.nw.w), ep);
        xst2(rs, X_XN + row * D + col, o0);
        xst2(rs, X_XN + row * D + col + 2, o1);
        if (j == 0) {
            float* ho = a.h_out + (size_t)row * D + col;
            store_wt(ho, h.x);
            store_wt(ho + 1, h.y);
            store_wt(ho + 2, h.z);
            store_wt(ho + 3, h.w);
        }
    }
}

// ---- k_prefill_attn -----------------------------------------------------------

constexpr int PQ = 33;    // uint4 per LDS panel row of 256 k (16-byte pad)
constexpr int PD = 49;    // ... of 384 k

template <int KIND>
__global__ __launch_bounds__(NT) void k_prefill_attn(XgArgs a) {
    using GK = GemmKind<KIND>;
    constexpr int KB = 4 * GK::EPL;
    constexpr int NKB128 = 128 / KB;   // K-blocks in 128 k
    __shared__ uint4 panel[MR * PQ];   // 33.8 KB: Q panel, the Q reduction, the O panel
    __shared__ float att_m[8][2], att_l[8][2];
    __shared__ float att_o[8][2][HD];  // 8 KB
    __shared__ float red_o[2][MR][16]; // O reduction (8 KB)
    __shared__ float ss_red[2][4];
    __shared__ uint4 bo_lds[4][NKB128][64];   // the O weights between N and O (4-16 KB)
    __shared__ float qs[2][2 * HD];           // each attention row's two query heads

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int b = blockIdx.x, j = b & 7, c = b >> 3;
    const int M = a.M;
    const int start = a.st->pos;
    unsigned* gbuf = a.xbuf + X_HDR + (size_t)j * X_GROUP;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(gbuf, (short)0, X_GROUP * 4, 0x00020000);
    const unsigned E = a.xbuf[0];
    const unsigned ep_xn = xg_epoch(E, a.n_layers, a.layer, SID_XA);
    const unsigned ep_qp = xg_epoch(E, a.n_layers, a.layer, SID_QP);
    const unsigned ep_r = xg_epoch(E, a.n_layers, a.layer, SID_R);
    const unsigned ep_ao = xg_epoch(E, a.n_layers, a.layer, SID_AO);
    const unsigned lim = a.xbuf[2] ? a.xbuf[2] : kSpin;
    bool dead = false;
    auto timed_out = [&]() {
        __hip_atomic_store(a.xbuf + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    const int l4 = lane >> 4, c16 = lane & 15;
    XG_TRACE(0, 0);
    const bool plain = a.x16 != nullptr;
    NRows nr_;
    if (!plain) stage_norm_load(a, c, t, nr_);
    // stage R's operands: its head slot's column scales and norm weights, and
    // the RoPE table entries of its row (positions start + row)
    const int rh = c & 3, rrow = 8 * (c >> 2) + wave;
    const int rcol0 = (rh == 0 ? 2 * j * HD : rh == 1 ? (2 * j + 1) * HD : rh == 2 ? QD + j * HD
                                                                         : QD + KVD + j * HD);
    const int rpos = start + min(rrow, M - 1);
    float rsc0 = 1.0f, rsc1 = 1.0f, rnw0 = 1.0f, rnw1 = 1.0f, rc0 = 0.f, rs0 = 0.f, rc1 = 0.f, rs1 = 0.f;
    {
        const float* nw = rh == 0 || rh == 1 ? a.q_norm : rh == 2 ? a.k_norm : nullptr;
        if (a.s1) {
            rsc0 = a.s1[rcol0 + lane];
            rsc1 = a.s1[rcol0 + 64 + lane];
        }
        if (nw) {
            rnw0 = nw[lane];
            rnw1 = nw[64 + lane];
        }
        if (rh < 3) {
            const int m0 = a.rope_style == 0 ? lane >> 1 : lane, m1 = a.rope_style == 0 ? 32 + (lane >> 1) : lane;
            rc0 = a.cos_t[(size_t)rpos * (HD / 2) + m0];
            rs0 = a.sin_t[(size_t)rpos * (HD / 2) + m0];
            rc1 = a.cos_t[(size_t)rpos * (HD / 2) + m1];
            rs1 = a.sin_t[(size_t)rpos * (HD / 2) + m1];
        }
    }
    XG_TRACE(0, 1);

    // ================= N =================
    if (!plain) stage_norm_finish(a, rs, ep_xn, j, c, t, nr_, ss_red);

    // ---------- the weights of both projections, requested after the N stage's loads
    // have returned (requested earlier they queue in front of them) ----------
    // Q: col group g (64 of the group's 512 columns), K split s
    const int g = c & 7, s = c >> 3;
    const int hs = g >> 1, gh = g & 1;
    const int qrow0 = (hs == 0 ? 2 * j * HD : hs == 1 ? (2 * j + 1) * HD : hs == 2 ? QD + j * HD
                                                                          : QD + KVD + j * HD) + 64 * gh;
    const int ct = wave & 3, kh = wave >> 2;
    uint4 bq[NKB128];
    load_b<KIND, NKB128>(bq, a.w1, qrow0 + 16 * ct + c16, D, 256 * s + 128 * kh, lane);
    // O: columns 32c.., K = the group's 256 attention dimensions; waves 0..3
    const int oct = wave & 1, okh = (wave >> 1) & 1;
    uint4 bo[NKB128];
    if (wave < 4) load_b<KIND, NKB128>(bo, a.w2, 32 * c + 16 * oct + c16, QD, 256 * j + 128 * okh, lane);
    XG_TRACE(0, 2);

    // ================= Q =================
    if (plain) stage_plain256<PQ>(panel, a.x16, M, 256 * s, t);
    else if (!stage_ll_panel<256, D, PQ>(panel, rs, X_XN, 256 * s, M, ep_xn, dead, lim, t)) { dead = true; timed_out(); }
    __syncthreads();
    XG_TRACE(0, 4);
    float4_t acc[4];
    zero_acc(acc);
    wave_mma<KIND, NKB128, PQ>(acc, bq, panel, 128 * kh, lane);
    // the O weights wait in LDS, not in registers, through R and A
    if (wave < 4) {
#pragma unroll
        for (int jb = 0; jb < NKB128; jb++) bo_lds[wave][jb][lane] = bo[jb];
    }
    XG_TRACE(0, 5);
    __syncthreads();   // the panel is reused for the K-half reduction
    float* red = reinterpret_cast<float*>(panel);   // [4 ct][64 rows][16]
    if (kh == 1) {
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) red[(ct * MR + 16 * r + 4 * l4 + i) * 16 + c16] = acc[r][i];
    }
    __syncthreads();
    if (kh == 0) {
        const int col = 16 * ct + c16;
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = 16 * r + 4 * l4 + i;
                if (row < M) {
                    const float v = acc[r][i] + red[(ct * MR + row) * 16 + c16];
                    xst2(rs, X_QP + ((((s * 4 + hs) * MR + row) * 64 + col) * 2 + gh) * 2, ll_f32x(v, ep_qp));
                }
            }
    }
    XG_TRACE(0, 6);

    // ================= R: QK-norm, RoPE, K/V append =================
    {
        const int row = rrow, i = lane;
        if (row < M) {
            int wd[4];
#pragma unroll
            for (int sp = 0; sp < 4; sp++) wd[sp] = X_QP + (((sp * 4 + rh) * MR + row) * 64 + i) * 4;
            u32x4 v[4];
            if (!xwait_probe<4, 3>(rs, wd, v, ep_qp, dead, lim)) { dead = true; timed_out(); }
            XG_TRACE(0, 7);
            // split order, then the column scale
            float x0 = ll_f32(v[0].x, v[0].y), x1 = ll_f32(v[0].z, v[0].w);
#pragma unroll
            for (int sp = 1; sp < 4; sp++) {
                x0 = x0 + ll_f32(v[sp].x, v[sp].y);
                x1 = x1 + ll_f32(v[sp].z, v[sp].w);
            }
            if (a.s1) {
                x0 = x0 * rsc0;
                x1 = x1 * rsc1;
            }
            const int pos = start + row;
            if (rh == 3) {
                const uint16_t h0 = f32_to_f16_bits(x0), h1 = f32_to_f16_bits(x1);
                a.vc[(size_t)pos * KVD + j * HD + i] = h0;
                a.vc[(size_t)pos * KVD + j * HD + 64 + i] = h1;
                xst1(rs, X_KV + row * 256 + 128 + i, ll_word(h0, ep_r));
                xst1(rs, X_KV + row * 256 + 192 + i, ll_word(h1, ep_r));
            } else {
                if (rh < 2 ? a.q_norm != nullptr : a.k_norm != nullptr) {
                    const float ss = wave_sum(x0 * x0 + x1 * x1);
                    const float rms = 1.0f / sqrtf(ss / (float)HD + a.eps);
                    x0 = (x0 * rms) * rnw0;
                    x1 = (x1 * rms) * rnw1;
                }
                float o0, o1;
                if (a.rope_style == 0) {
                    // adjacent pairs (2m, 2m + 1): the partner is lane i ^ 1
                    const float p0 = dpp<0xB1>(x0), p1 = dpp<0xB1>(x1);
                    if ((i & 1) == 0) {
                        o0 = x0 * rc0 - p0 * rs0;
                        o1 = x1 * rc1 - p1 * rs1;
                    } else {
                        o0 = x0 * rc0 + p0 * rs0;
                        o1 = x1 * rc1 + p1 * rs1;
                    }
                } else {
                    // split halves (i, i + 64)
                    o0 = x0 * rc0 - x1 * rs0;
                    o1 = x1 * rc0 + x0 * rs0;
                }
                if (rh < 2) {
                    xst2(rs, X_RQ + ((row * 2 + rh) * HD + i) * 2, ll_f32x(o0, ep_r));
                    xst2(rs, X_RQ + ((row * 2 + rh) * HD + 64 + i) * 2, ll_f32x(o1, ep_r));
                } else {
                    const uint16_t h0 = f32_to_f16_bits(o0), h1 = f32_to_f16_bits(o1);
                    a.kc[(size_t)pos * KVD + j * HD + i] = h0;
                    a.kc[(size_t)pos * KVD + j * HD + 64 + i] = h1;
                    xst1(rs, X_KV + row * 256 + i, ll_word(h0, ep_r));
                    xst1(rs, X_KV + row * 256 + 64 + i, ll_word(h1, ep_r));
                }
            }
        }
    }
    XG_TRACE(0, 8);

    // ================= A: rows c (waves 0-3) and 63 - c (waves 4-7) at once =================
    {
        const int half = wave >> 2, ht = t & 255;
        const int ps = ht >> 4, dl = ht & 15;        // 16 position slots x 16 lanes (8 dims each)
        const int row = half == 0 ? c : MR - 1 - c;
        const bool live = row < M;
        const int Lr = live ? start + row + 1 : 0;
        const int L0 = c < M ? start + c + 1 : 0, L1 = MR - 1 - c < M ? start + MR - c : 0;
        const int rounds = ((L0 > L1 ? L0 : L1) + 63) / 64;   // the same for both halves
        const float scale = 1.0f / sqrtf((float)HD);
        float qa[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, qb[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        // threads t < 256 of each half merge output (head ht >> 7, dimension ht & 127)
        float runM = -INFINITY, runL = 0.0f, runO = 0.0f;
#pragma unroll 1
        for (int rd = 0; rd < rounds; rd++) {
            // four passes of 16 positions; LL rows of this chunk (the row's own
            // position stands in for slots past the row), cache rows before it
            bool valid[4];
            int wd[17];
            u32x4 v[17];
#pragma unroll
            for (int pp = 0; pp < 4; pp++) {
                const int p = 64 * rd + 16 * pp + ps;
                valid[pp] = p < Lr;
                const int nr = (valid[pp] && p >= start) ? p - start : row;
                wd[4 * pp + 0] = X_KV + nr * 256 + 8 * dl;
                wd[4 * pp + 1] = X_KV + nr * 256 + 8 * dl + 4;
                wd[4 * pp + 2] = X_KV + nr * 256 + 128 + 8 * dl;
                wd[4 * pp + 3] = X_KV + nr * 256 + 128 + 8 * dl + 4;
            }
            // the row's q (512 words): threads ht < 128 of the half poll 4 each
            wd[16] = X_RQ + row * 2 * HD * 2 + 4 * (ht & 127);
#pragma unroll
            for (int i = 0; i < 17; i++) v[i] = u32x4{0u, 0u, 0u, 0u};
            if (live) {
                bool ok;
                if (rd == 0 && ht < 128) {
                    ok = xwait_probe<17, 16>(rs, wd, v, ep_r, dead, lim);   // K/V rows and the row's q
                } else {
                    int wk[16];
                    u32x4 vk[16];
#pragma unroll
                    for (int i = 0; i < 16; i++) wk[i] = wd[i];
                    ok = xwait_probe<16>(rs, wk, vk, ep_r, dead, lim);
#pragma unroll
                    for (int i = 0; i < 16; i++) v[i] = vk[i];
                }
                if (!ok) { dead = true; timed_out(); }
                if (rd == 0) XG_TRACE(0, 9);
                // cache rows before the chunk, put in the words' form (payload in the low half)
#pragma unroll
                for (int pp = 0; pp < 4; pp++) {
                    const int p = 64 * rd + 16 * pp + ps;
                    if (valid[pp] && p < start) {
                        const uint4 kk = *reinterpret_cast<const uint4*>(a.kc + (size_t)p * KVD + j * HD + dl * 8);
                        const uint4 vv = *reinterpret_cast<const uint4*>(a.vc + (size_t)p * KVD + j * HD + dl * 8);
                        v[4 * pp + 0] = u32x4{kk.x, kk.x >> 16, kk.y, kk.y >> 16};
                        v[4 * pp + 1] = u32x4{kk.z, kk.z >> 16, kk.w, kk.w >> 16};
                        v[4 * pp + 2] = u32x4{vv.x, vv.x >> 16, vv.y, vv.y >> 16};
                        v[4 * pp + 3] = u32x4{vv.z, vv.z >> 16, vv.w, vv.w >> 16};
                    }
                }
            }
            if (rd == 0) {
                if (ht < 128) {
                    qs[half][2 * ht] = ll_f32(v[16].x, v[16].y);
                    qs[half][2 * ht + 1] = ll_f32(v[16].z, v[16].w);
                }
                __syncthreads();
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    qa[e] = qs[half][dl * 8 + e];
                    qb[e] = qs[half][HD + dl * 8 + e];
                }
            }
            auto lo16 = [](unsigned w) { return f16_bits_to_f32((uint16_t)(w & 0xffffu)); };
            float sc[4][2];
            float mx[2] = {-INFINITY, -INFINITY};
#pragma unroll
            for (int pp = 0; pp < 4; pp++) {
                // a pass wholly past the row (the same for the half's waves) is skipped
                sc[pp][0] = sc[pp][1] = -INFINITY;
                if (64 * rd + 16 * pp >= Lr) continue;
                const float k[8] = {lo16(v[4 * pp].x),     lo16(v[4 * pp].y),     lo16(v[4 * pp].z),
                                    lo16(v[4 * pp].w),     lo16(v[4 * pp + 1].x), lo16(v[4 * pp + 1].y),
                                    lo16(v[4 * pp + 1].z), lo16(v[4 * pp + 1].w)};
                float s0 = ((qa[0] * k[0] + qa[1] * k[1]) + (qa[2] * k[2] + qa[3] * k[3])) +
                           ((qa[4] * k[4] + qa[5] * k[5]) + (qa[6] * k[6] + qa[7] * k[7]));
                float s1 = ((qb[0] * k[0] + qb[1] * k[1]) + (qb[2] * k[2] + qb[3] * k[3])) +
                           ((qb[4] * k[4] + qb[5] * k[5]) + (qb[6] * k[6] + qb[7] * k[7]));
                s0 = row_sum16(s0) * scale;
                s1 = row_sum16(s1) * scale;
                sc[pp][0] = valid[pp] ? s0 : -INFINITY;
                sc[pp][1] = valid[pp] ? s1 : -INFINITY;
                mx[0] = fmaxf(mx[0], sc[pp][0]);
                mx[1] = fmaxf(mx[1], sc[pp][1]);
            }
            if (rd == 0) XG_TRACE(0, 10);
            // maximum over the round: the wave's four position rows, then the half's waves
#pragma unroll
            for (int h = 0; h < 2; h++) mx[h] = rows_max4(mx[h]);
            if (lane == 0) {
                att_m[wave][0] = mx[0];
                att_m[wave][1] = mx[1];
            }
            __syncthreads();
            float Mr[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                float m = att_m[4 * half][h];
#pragma unroll
                for (int w = 1; w < 4; w++) m = fmaxf(m, att_m[4 * half + w][h]);
                Mr[h] = m;
            }
            float ls[2] = {0.f, 0.f}, o[2][8];
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int e = 0; e < 8; e++) o[h][e] = 0.0f;
#pragma unroll
            for (int pp = 0; pp < 4; pp++) {
                if (64 * rd + 16 * pp >= Lr) continue;
                const float vf[8] = {lo16(v[4 * pp + 2].x), lo16(v[4 * pp + 2].y), lo16(v[4 * pp + 2].z),
                                     lo16(v[4 * pp + 2].w), lo16(v[4 * pp + 3].x), lo16(v[4 * pp + 3].y),
                                     lo16(v[4 * pp + 3].z), lo16(v[4 * pp + 3].w)};
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const float pr = sc[pp][h] == -INFINITY ? 0.0f : expf(sc[pp][h] - Mr[h]);
                    ls[h] = ls[h] + pr;
#pragma unroll
                    for (int e = 0; e < 8; e++) o[h][e] = o[h][e] + pr * vf[e];
                }
            }
            // sums over the position slots: the wave's four rows, then the half's waves in order
#pragma unroll
            for (int h = 0; h < 2; h++) {
                ls[h] = rows_sum4(ls[h]);
#pragma unroll
                for (int e = 0; e < 8; e++) o[h][e] = rows_sum4(o[h][e]);
            }
            if (lane < 16) {
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int e = 0; e < 8; e++) att_o[wave][h][dl * 8 + e] = o[h][e];
                if (lane == 0) {
                    att_l[wave][0] = ls[0];
                    att_l[wave][1] = ls[1];
                }
            }
            __syncthreads();
            {
                const int h = ht >> 7, d = ht & 127;
                float Ox = att_o[4 * half][h][d], Lx = att_l[4 * half][h];
#pragma unroll
                for (int w = 1; w < 4; w++) {
                    Ox = Ox + att_o[4 * half + w][h][d];
                    Lx = Lx + att_l[4 * half + w][h];
                }
                const float M2 = Mr[h];
                const float Mn = fmaxf(runM, M2);
                if (Mn != -INFINITY) {
                    const float fa = runM == -INFINITY ? 0.0f : expf(runM - Mn);
                    const float fb = M2 == -INFINITY ? 0.0f : expf(M2 - Mn);
                    runL = runL * fa + Lx * fb;
                    runO = runO * fa + Ox * fb;
                    runM = Mn;
                }
            }
            __syncthreads();   // att_* are rewritten by the next round
        }
        if (live) {
            const int h = ht >> 7, d = ht & 127;
            xst1(rs, X_AO + row * 256 + h * HD + d, ll_word(f32_to_f16_bits(runO / runL), ep_ao));
        }
    }
    XG_TRACE(0, 11);

    // ================= O: 32 columns over the group's K slice =================
    // (a workgroup whose two attention rows are both past M ran no round, so
    // no barrier since the Q reduction read the panel's LDS)
    __syncthreads();
    if (!stage_ll_panel<256, 256, PQ>(panel, rs, X_AO, 0, M, ep_ao, dead, lim, t)) { dead = true; timed_out(); }
    __syncthreads();
    XG_TRACE(0, 13);
    if (wave < 4) {
#pragma unroll
        for (int jb = 0; jb < NKB128; jb++) bo[jb] = bo_lds[wave][jb][lane];
        zero_acc(acc);
        wave_mma<KIND, NKB128, PQ>(acc, bo, panel, 128 * okh, lane);
        XG_TRACE(0, 14);
        if (okh == 1) {
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int i = 0; i < 4; i++) red_o[oct][16 * r + 4 * l4 + i][c16] = acc[r][i];
        }
    }
    __syncthreads();
    if (wave < 4 && okh == 0) {
        const int col = 32 * c + 16 * oct + c16;
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = 16 * r + 4 * l4 + i;
                if (row < M)
                    store_wt(&a.part_out[((size_t)j * MR + row) * D + col], acc[r][i] + red_o[oct][row][c16]);
            }
    }
    XG_TRACE(0, 15);
}

// ---- k_prefill_mlp --------------------------------------------------------------

template <int KIND>
__global__ __launch_bounds__(NT) void k_prefill_mlp(XgArgs a) {
    using GK = GemmKind<KIND>;
    constexpr int KB = 4 * GK::EPL;
    constexpr int NKB128 = 128 / KB, NKB256 = 256 / KB;
    __shared__ uint4 panel[MR * PD];        // 50 KB: G panel (256 k), D panel (384 k)
    __shared__ float red_d[2][2][MR][16];   // D reduction over its three K parts (16 KB)
    __shared__ float ss_red[2][4];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int b = blockIdx.x, j = b & 7, c = b >> 3;
    const int M = a.M;
    unsigned* gbuf = a.xbuf + X_HDR + (size_t)j * X_GROUP;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(gbuf, (short)0, X_GROUP * 4, 0x00020000);
    const unsigned E = a.xbuf[0];
    const unsigned ep_xn = xg_epoch(E, a.n_layers, a.layer, SID_XM);
    const unsigned ep_gp = xg_epoch(E, a.n_layers, a.layer, SID_GP);
    const unsigned ep_sa = xg_epoch(E, a.n_layers, a.layer, SID_SA);
    const unsigned lim = a.xbuf[2] ? a.xbuf[2] : kSpin;
    bool dead = false;
    auto timed_out = [&]() {
        __hip_atomic_store(a.xbuf + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    const int l4 = lane >> 4, c16 = lane & 15;
    XG_TRACE(1, 0);
    const bool plain = a.x16 != nullptr;
    NRows nr_;
    if (!plain) stage_norm_load(a, c, t, nr_);
    // S's column scales
    const int srow = 2 * c + t / 192, sfp = 2 * (t % 192);
    float sg[2] = {1.f, 1.f}, su[2] = {1.f, 1.f};
    if (a.s1 && t < 384) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            sg[q] = a.s1[GF * j + sfp + q];
            su[q] = a.s1[FF + GF * j + sfp + q];
        }
    }
    XG_TRACE(1, 1);

    // ================= N =================
    if (!plain) stage_norm_finish(a, rs, ep_xn, j, c, t, nr_, ss_red);

    // G: tile group pg (48 features: gate tiles 0..2, up tiles 3..5), K split s
    const int pg = c & 7, s = c >> 3;
    const int f0 = GF * j + 48 * pg;
    const int gct = wave;   // waves 0..5
    uint4 bg[NKB256];
    if (wave < 6) {
        const int wrow = gct < 3 ? f0 + 16 * gct + c16 : FF + f0 + 16 * (gct - 3) + c16;
        load_b<KIND, NKB256>(bg, a.w1, wrow, D, 256 * s, lane);
    }
    // D: columns 32c.., K = the group's 384 features in three parts; waves 0..5
    const int dct = wave & 1, dkp = wave >> 1;
    uint4 bd[NKB128];
    if (wave < 6) load_b<KIND, NKB128>(bd, a.w2, 32 * c + 16 * dct + c16, FF, GF * j + 128 * dkp, lane);
    XG_TRACE(1, 2);

    // ================= G =================
    if (plain) stage_plain256<PQ>(panel, a.x16, M, 256 * s, t);
    else if (!stage_ll_panel<256, D, PQ>(panel, rs, X_XN, 256 * s, M, ep_xn, dead, lim, t)) { dead = true; timed_out(); }
    __syncthreads();
    XG_TRACE(1, 4);
    float4_t acc[4];
    if (wave < 6) {
        zero_acc(acc);
        wave_mma<KIND, NKB256, PQ>(acc, bg, panel, 0, lane);
        XG_TRACE(1, 5);
        const int fl = 16 * (gct % 3) + c16, gu = gct / 3;
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = 16 * r + 4 * l4 + i;
                if (row < M)
                    xst2(rs, X_GP + (((s * MR + row) * GF + 48 * pg + fl) * 2 + gu) * 2, ll_f32x(acc[r][i], ep_gp));
            }
    }
    XG_TRACE(1, 6);

    // ================= S: rows 2c, 2c + 1 =================
    if (t < 384) {
        const int row = srow, fp = sfp;
        if (row < M) {
            int wd[8];
#pragma unroll
            for (int sp = 0; sp < 4; sp++) {
                wd[2 * sp] = X_GP + ((sp * MR + row) * GF + fp) * 4;
                wd[2 * sp + 1] = wd[2 * sp] + 4;
            }
            u32x4 v[8];
            if (!xwait_probe<8, 7>(rs, wd, v, ep_gp, dead, lim)) { dead = true; timed_out(); }
            XG_TRACE(1, 7);
            float gs[2], us[2];
#pragma unroll
            for (int q = 0; q < 2; q++) {
                float gv = ll_f32(v[q].x, v[q].y), uv = ll_f32(v[q].z, v[q].w);
#pragma unroll
                for (int sp = 1; sp < 4; sp++) {
                    gv = gv + ll_f32(v[2 * sp + q].x, v[2 * sp + q].y);
                    uv = uv + ll_f32(v[2 * sp + q].z, v[2 * sp + q].w);
                }
                gs[q] = a.s1 ? gv * sg[q] : gv;
                us[q] = a.s1 ? uv * su[q] : uv;
            }
            u32x2 o;
            o.x = ll_word(f32_to_f16_bits(silu_mul(gs[0], us[0])), ep_sa);
            o.y = ll_word(f32_to_f16_bits(silu_mul(gs[1], us[1])), ep_sa);
            xst2(rs, X_SA + row * GF + fp, o);
        }
    }
    XG_TRACE(1, 8);

    // ================= D: 32 columns over the group's 384 features =================
    __syncthreads();   // the G panel is no longer read
    if (!stage_ll_panel<GF, GF, PD>(panel, rs, X_SA, 0, M, ep_sa, dead, lim, t)) { dead = true; timed_out(); }
    __syncthreads();
    XG_TRACE(1, 10);
    if (wave < 6) {
        zero_acc(acc);
        wave_mma<KIND, NKB128, PD>(acc, bd, panel, 128 * dkp, lane);
        XG_TRACE(1, 11);
        if (dkp > 0) {
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int i = 0; i < 4; i++) red_d[dkp - 1][dct][16 * r + 4 * l4 + i][c16] = acc[r][i];
        }
    }
    __syncthreads();
    if (wave < 2) {
        const int col = 32 * c + 16 * dct + c16;
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = 16 * r + 4 * l4 + i;
                if (row < M)
                    store_wt(&a.part_out[((size_t)j * MR + row) * D + col],
                             (acc[r][i] + red_d[0][dct][row][c16]) + red_d[1][dct][row][c16]);
            }
    }
    XG_TRACE(1, 12);
}

// End of a fused prefill: the position advances by M and the prefill counter
// (the epoch source) by one.
__global__ void k_prefill_xg_end(mdx_state* st, int advance, unsigned* xbuf) {
    if (threadIdx.x == 0) {
        st->pos = st->pos + advance;
        xbuf[0] = xbuf[0] + 1u;
    }
}

template <int KIND>
int launch_pair(const XgArgs& a, int which, void* stream) {
    if (which == 0)
        hipLaunchKernelGGL(k_prefill_attn<KIND>, dim3(NB), dim3(NT), 0, (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL(k_prefill_mlp<KIND>, dim3(NB), dim3(NT), 0, (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

int launch_kind(int kind, const XgArgs& a, int which, void* stream) {
    switch (kind) {
        case MDX_W_F16: return launch_pair<MDX_W_F16>(a, which, stream);
        case MDX_W_I8: return launch_pair<MDX_W_I8>(a, which, stream);
        case MDX_W_I4: return launch_pair<MDX_W_I4>(a, which, stream);
        default: return -5;
    }
}

}  // namespace

extern "C" {

int mdx_prefill_xg_shape_ok(int d, int nq, int nkv, int hd, int F) {
    return d == D && nq == NQ && nkv == NKV && hd == HD && F == FF;
}

size_t mdx_prefill_xg_buf_bytes(void) { return X_BYTES; }

int mdx_launch_prefill_attn(const mdx_prefill_xg_args* p, const mdx_wdesc* qkv, const mdx_wdesc* o,
                            const float* q_norm, const float* k_norm, const float* cos_t, const float* sin_t,
                            int rope_style, uint16_t* k_cache, uint16_t* v_cache, void* stream) {
    const bool plain = p && p->x16;
    if (!p || p->M <= 0 || p->M > MR || !p->state || !p->part_out || !p->xbuf || !qkv || !o ||
        qkv->kind != o->kind || qkv->K != D || qkv->N != QD + 2 * KVD || o->K != QD || o->N != D || p->layer < 0 ||
        p->layer >= p->n_layers ||
        (!plain && (!p->h_in || !p->h_out || !p->norm_w || p->part_in == p->part_out || p->h_in == p->h_out)))
        return -1;
    XgArgs a = {};
    a.x16 = p->x16;
    a.st = p->state;
    a.M = p->M;
    a.n_layers = p->n_layers;
    a.layer = p->layer;
    a.rope_style = rope_style;
    a.eps = p->eps;
    a.h_in = p->h_in;
    a.h_out = p->h_out;
    a.part_in = p->part_in;
    a.scale_in = p->scale_in;
    a.norm_w = p->norm_w;
    a.w1 = (const uint8_t*)qkv->w;
    a.s1 = qkv->scale;
    a.w2 = (const uint8_t*)o->w;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.cos_t = cos_t;
    a.sin_t = sin_t;
    a.kc = k_cache;
    a.vc = v_cache;
    a.part_out = p->part_out;
    a.xbuf = (unsigned*)p->xbuf;
    a.trace = p->trace;
    return launch_kind(qkv->kind, a, 0, stream);
}

int mdx_launch_prefill_mlp(const mdx_prefill_xg_args* p, const mdx_wdesc* gu, const mdx_wdesc* down,
                           void* stream) {
    const bool plain = p && p->x16;
    if (!p || p->M <= 0 || p->M > MR || !p->state || !p->part_out || !p->xbuf || !gu || !down ||
        gu->kind != down->kind || gu->K != D || gu->N != 2 * FF || down->K != FF || down->N != D || p->layer < 0 ||
        p->layer >= p->n_layers ||
        (!plain && (!p->h_in || !p->h_out || !p->norm_w || !p->part_in || p->part_in == p->part_out ||
                    p->h_in == p->h_out)))
        return -1;
    XgArgs a = {};
    a.x16 = p->x16;
    a.st = p->state;
    a.M = p->M;
    a.n_layers = p->n_layers;
    a.layer = p->layer;
    a.eps = p->eps;
    a.h_in = p->h_in;
    a.h_out = p->h_out;
    a.part_in = p->part_in;
    a.scale_in = p->scale_in;
    a.norm_w = p->norm_w;
    a.w1 = (const uint8_t*)gu->w;
    a.s1 = gu->scale;
    a.w2 = (const uint8_t*)down->w;
    a.part_out = p->part_out;
    a.xbuf = (unsigned*)p->xbuf;
    a.trace = p->trace;
    return launch_kind(gu->kind, a, 1, stream);
}

int mdx_launch_prefill_xg_end(mdx_state* state, int advance, void* xbuf, void* stream) {
    if (!state || !xbuf) return -1;
    hipLaunchKernelGGL(k_prefill_xg_end, dim3(1), dim3(64), 0, (hipStream_t)stream, state, advance,
                       (unsigned*)xbuf);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // extern "C"
