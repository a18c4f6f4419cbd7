// mdx_persist.hip — one decode step of the 0.6B-class decoder (hidden 1024,
// 16 query / 8 KV heads of 128, SwiGLU FFN 3072, INT8 lm_head) as a single
// cooperative launch of 256 workgroups, one per CU.
//
// Reference path replaced: matmul_decoder_step (src/matmul_decoder.c:1430-1634):
// embedding, per layer RMSNorm -> q/k/v -> QK-norm -> RoPE -> KV append ->
// GQA attention -> o -> residual -> RMSNorm -> gate/up -> SwiGLU -> down ->
// residual, then final norm, the INT8 lm_head and argmax_f32.
//
// A step of this model is a chain of six dependent exchanges per layer; each
// one needs every workgroup's output before anyone can go on.  With one
// kernel per stage every exchange costs a kernel boundary and every kernel
// starts with an idle HBM pipe.  Here the workgroups stay resident and
// exchange through "LL" words: 32-bit words holding 16 payload bits and a
// 16-bit epoch, written with agent-coherent stores and polled with
// L2-bypassing (sc1) 16-byte loads.  A reader knows a word is current when
// its epoch matches, so there is no flag, fence or barrier round trip.  The
// weights of later stages are requested ahead, mostly just after a wait, so
// the HBM stream runs while workgroups wait for each other.
//
// Work split (b = workgroup, t = thread):
//   qkv    group j = b % 8 (one KV head), split s = b / 8: the 16 rows
//          s*16.. of [q(2j) | q(2j+1) | k(j) | v(j)];
//   attn   (j, s): positions [s*c, (s+1)*c) of KV head j, c = ceil(L/32),
//          online softmax over the chunk -> partial (m, l, o);
//   merge  (j, s): 8 of the 256 outputs of KV head j from the 32 partials;
//   o      rows 4b..4b+3 (+ residual), gate/up: features 12b..12b+11,
//   down   rows 4b..4b+3 (+ residual), lm_head: rows [bV/256, (b+1)V/256).
// Every wait is bounded: a workgroup that times out records an error in
// state->pad[1] and stops waiting, so the grid always drains.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdlib>

#include "mdx_common.h"
#include "mdx_device.h"

using namespace mdx;

namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int NB = 256;                 // workgroups
constexpr int NT = 256;                 // threads per workgroup
constexpr int D = 1024, NQ = 16, NKV = 8, HD = 128, FF = 3072;
constexpr int QD = NQ * HD, KVD = NKV * HD;
constexpr int GRP = NB / NKV;           // workgroups per KV head
constexpr unsigned kSpinLimit = 1u << 18;   // polling rounds before a wait gives up

// Attention split of a step at position pos: split s (of GRP per KV head)
// covers positions [p0, p0 + n) of the Lk = pos + 1 cached ones.  The cache
// row a K/V load reads for position index pi of the split: the position
// itself while pi < n and it is not the step's own (that row is appended by
// this step and taken from registers), else row 0 as a stand-in for an
// unused slot, so every address lies in rows [0, pos].  Shared by the kernel
// and by mdx_debug_persist_kv_rows, which enumerates it on the host.
struct KvSplit {
    int p0, n;
};
__host__ __device__ inline KvSplit kv_split(int pos, int s) {
    const int Lk = pos + 1;
    const int cks = (Lk + GRP - 1) / GRP;
    const int p0 = s * cks;
    const int p1 = Lk < p0 + cks ? Lk : p0 + cks;
    return KvSplit{p0, p1 > p0 ? p1 - p0 : 0};
}
__host__ __device__ inline int kv_row(const KvSplit& sp, int pi, int pos) {
    const int p = sp.p0 + pi;
    return (pi < sp.n && p != pos) ? p : 0;
}

// exchange buffer layout, in 32-bit words
constexpr int W_CTRL = 0;                          // [0] step counter
constexpr int W_QKV = 16;                          // [NKV][512 values][2]
// Partial attention records of KV head j, laid out for the merge's reads: the
// merging workgroup (j, s) owns 8 output dimensions c = s & 15 of head
// hh = s >> 4 and finds the 32 splits' values for them in one 2 KiB run
// ([hh][c][split][8 values x 2 words]), and the 32 (m, l) pairs in one 512 B
// run after it.  Every exchange region is read with whole-wave 1 KiB loads
// (lane-contiguous 16-byte groups): polls scattered over 64-byte lines cost
// one memory request per lane and were the slowest exchanges (measured:
// 518 -> 475 us/token over the scattered layouts).
constexpr int PART_O = 2 * 16 * GRP * 16;           // [2][16][GRP][16] o values
constexpr int PART_WORDS_J = PART_O + 2 * GRP * 4;  // + [2][GRP][4] (m, l)
constexpr int W_PART = W_QKV + NKV * 1024;          // [NKV][PART_WORDS_J]
// The all-to-all exchanges (attention output, hidden state after o and after
// down, SwiGLU activations) are written in NREP copies; workgroup b reads copy
// b % NREP, which spreads the reads of one exchange over more memory channels
// (2 copies measured best among 1, 2, 4 and 8).
constexpr int NREP = 2;
constexpr int W_ATT = W_PART + NKV * PART_WORDS_J;  // [NREP][QD] fp16
constexpr int W_HO = W_ATT + NREP * QD;            // [NREP][D][2] hidden after o
constexpr int W_ACT = W_HO + NREP * 2 * D;         // [NREP][NB][12] fp16, writer b at 12 b
constexpr int W_HD = W_ACT + NREP * NB * 12;       // [NREP][D][2] hidden after down
constexpr int W_AMAX = W_HD + NREP * 2 * D;        // [NB][4] argmax keys
constexpr int W_TOTAL = W_AMAX + NB * 4;
static_assert(W_PART % 4 == 0 && W_ATT % 4 == 0 && W_HO % 4 == 0 && W_ACT % 4 == 0 &&
              W_HD % 4 == 0 && W_AMAX % 4 == 0, "16-byte aligned regions");

struct PArgs {
    int n_layers, vocab, max_seq, rope_style, head, advance;
    float eps;
    mdx_state* st;
    mdx_persist_layer l0;       // layer 0; layer l is l0 advanced by l * lstride bytes
    long long lstride;          // (KV caches: by l * kvstride elements)
    long long kvstride;
    const float* emb_table;
    const float* emb_in;
    const float* cos_t;
    const float* sin_t;
    const float* final_norm;
    const int8_t* lm_w;
    const float* lm_scale;
    float* logits;
    float* hidden_out;
    unsigned* xbuf;
    int* out_tokens;
    unsigned long long* trace;  // optional [NB][trace_stride] 100 MHz timestamps
    int trace_stride;
    unsigned spin_limit;
    int kv_stream;
    int in_args;                // 1: pos, token, mode from the three fields below, not st
    int in_pos, in_token, in_mode;
    float* logits_host;         // optional mapped host buffer for the logits (instead of logits)
    int* res_host;              // optional mapped host words: [0] the argmax, [1] set on a timeout
    unsigned* xbl;              // optional cacheable words for the per-head exchanges
};

// Rows of the lm_head per workgroup that the host-logits mode stages in LDS
// (vocabularies up to 256 * 1024 rows use it).
constexpr int kLogitsRows = 1024;

// Timestamp of event ev for this workgroup (thread 0), when tracing is on.
#define MDX_TRACE(ev)                                                                      \
    do {                                                                                   \
        if (a.trace && t == 0) a.trace[(size_t)b * a.trace_stride + (ev)] = wall_clock64(); \
    } while (0)

// ---- LL words ---------------------------------------------------------------

// Cache policy sc1: bypass the non-coherent caches.  The buffer-load builtin
// is a plain read to the optimiser, so the polling loop below carries a
// compiler memory barrier to keep the reload inside the loop.
template <int AUX = 16>
__device__ __forceinline__ u32x4 ll_load(__amdgpu_buffer_rsrc_t rs, int word) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, word * 4, 0, AUX);
}
__device__ __forceinline__ bool ll_ok(u32x4 v, unsigned ep) {
    return ((v.x >> 16) == ep) & ((v.y >> 16) == ep) & ((v.z >> 16) == ep) & ((v.w >> 16) == ep);
}
__device__ __forceinline__ float ll_f32(unsigned lo, unsigned hi) {
    return __uint_as_float((lo & 0xffffu) | (hi << 16));
}
__device__ __forceinline__ void ll_put(unsigned* xb, int word, unsigned payload, unsigned ep) {
    __hip_atomic_store(xb + word, (payload & 0xffffu) | (ep << 16), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Four LL words in one 16-byte store (each word still carries its own epoch,
// so a reader never accepts a partly written group).
__device__ __forceinline__ void ll_put4(__amdgpu_buffer_rsrc_t rs, int word, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, rs, word * 4, 0, 16);
}

// The per-head exchanges (qkv rows -> attention, partial records -> merge)
// have their writers and readers among the 32 workgroups of one KV head, and
// workgroups b, b + 8, ... run on one XCD: with a cacheable word buffer those
// exchanges can stay in that XCD's L2.  Plain stores (through to the L2) and
// non-temporal polls (which do not hit a stale line in the CU's L1; polls with
// sc0, or an L1 invalidate before each poll, kept reading stale words).
constexpr int kLocalPoll = 2;   // nt
__device__ __forceinline__ void lx_put4(__amdgpu_buffer_rsrc_t rs, int word, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, rs, word * 4, 0, 0);
}
__device__ __forceinline__ u32x4 ll_pack2(float v0, float v1, unsigned ep) {
    const unsigned x = __float_as_uint(v0), y = __float_as_uint(v1), e = ep << 16;
    u32x4 r;
    r.x = (x & 0xffffu) | e;
    r.y = (x >> 16) | e;
    r.z = (y & 0xffffu) | e;
    r.w = (y >> 16) | e;
    return r;
}

// Wave 0: lanes 0..3 hold the workgroup's 4 hidden values; lanes 0..2*NREP-1
// store them, two per 16-byte group, into every copy of the region at base.
__device__ __forceinline__ void put_hidden4(__amdgpu_buffer_rsrc_t rs, int base, int b, float hv,
                                            unsigned ep, int lane) {
    const float v0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hv), 0));
    const float v1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hv), 1));
    const float v2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hv), 2));
    const float v3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hv), 3));
    if (lane < 2 * NREP) {
        const bool hi = (lane & 1) != 0;
        ll_put4(rs, base + (lane >> 1) * (2 * D) + 8 * b + 4 * (lane & 1),
                ll_pack2(hi ? v2 : v0, hi ? v3 : v1, ep));
    }
}

// Polls N 16-byte groups until every word carries epoch ep.  Returns false
// after `limit` rounds (the data is then stale; the caller stops waiting).
template <int N, int AUX = 16>
__device__ __forceinline__ bool ll_wait(__amdgpu_buffer_rsrc_t rs, const int (&word)[N],
                                        u32x4 (&v)[N], unsigned ep, bool dead, unsigned limit) {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = ll_load<AUX>(rs, word[i]);
    if (dead) return true;
    for (unsigned spin = 0;; spin++) {
        asm volatile("" ::: "memory");
        bool all = true;
#pragma unroll
        for (int i = 0; i < N; i++) {
            if (!ll_ok(v[i], ep)) {
                all = false;
                v[i] = ll_load<AUX>(rs, word[i]);
            }
        }
        if (all) return true;
        if (spin > limit) return false;
    }
}

// Polls the first group alone, then requests the others together.  For an
// exchange whose writers finish over a spread of time this keeps one load per
// thread in flight while waiting, which shortens the exchange (fewer requests
// compete with the writes and with the other readers' polls).
template <int N>
__device__ __forceinline__ bool ll_wait_probe(__amdgpu_buffer_rsrc_t rs, const int (&word)[N],
                                              u32x4 (&v)[N], unsigned ep, bool dead, unsigned limit) {
    int w0[1] = {word[0]};
    u32x4 v0[1];
    bool ok = ll_wait<1>(rs, w0, v0, ep, dead, limit);
    v[0] = v0[0];
    int wr[N - 1];
    u32x4 vr[N - 1];
#pragma unroll
    for (int i = 1; i < N; i++) wr[i - 1] = word[i];
    ok = ll_wait<N - 1>(rs, wr, vr, ep, dead, limit) && ok;
#pragma unroll
    for (int i = 1; i < N; i++) v[i] = vr[i - 1];
    return ok;
}

// Layer pointers are computed, not loaded: a load of them would be a vector
// memory load (the kernel writes global memory, so the compiler cannot use
// scalar loads) and would queue behind the weight stream.
__device__ __forceinline__ mdx_persist_layer layer_at(const PArgs& a, int l) {
    const size_t off = (size_t)l * (size_t)a.lstride;
    auto adv = [off](const void* p) -> const void* {
        return p ? reinterpret_cast<const char*>(p) + off : nullptr;
    };
    mdx_persist_layer r;
    r.wqkv = adv(a.l0.wqkv);
    r.sqkv = reinterpret_cast<const float*>(adv(a.l0.sqkv));
    r.wo = adv(a.l0.wo);
    r.so = reinterpret_cast<const float*>(adv(a.l0.so));
    r.wgu = adv(a.l0.wgu);
    r.sgu = reinterpret_cast<const float*>(adv(a.l0.sgu));
    r.wdown = adv(a.l0.wdown);
    r.sdown = reinterpret_cast<const float*>(adv(a.l0.sdown));
    r.in_norm = reinterpret_cast<const float*>(adv(a.l0.in_norm));
    r.post_norm = reinterpret_cast<const float*>(adv(a.l0.post_norm));
    r.q_norm = reinterpret_cast<const float*>(adv(a.l0.q_norm));
    r.k_norm = reinterpret_cast<const float*>(adv(a.l0.k_norm));
    r.kc = a.l0.kc + (size_t)l * (size_t)a.kvstride;
    r.vc = a.l0.vc + (size_t)l * (size_t)a.kvstride;
    return r;
}

__device__ __forceinline__ unsigned step_epoch(unsigned E, int L, int l) {
    return (unsigned)(((unsigned long long)E * (unsigned)(L + 2) + (unsigned)l) % 65535ull) + 1u;
}

// ---- weights ----------------------------------------------------------------

// The layer weights (and, for long contexts, the K/V rows) are read once per
// step with non-temporal loads (ld_nt), so they do not evict from the
// last-level cache what is read again every step: the lm_head and a short
// context's K/V rows (measured: 480 -> 470 us/token at KV 512 with the layer
// weights non-temporal; at KV 4096 the K/V rows non-temporal too, 569 -> 550).

template <int KIND> struct KT;
template <> struct KT<MDX_W_F16> { static constexpr int E = 8; };
template <> struct KT<MDX_W_I8> { static constexpr int E = 16; };
template <> struct KT<MDX_W_I4> { static constexpr int E = 32; };

// 16-byte weight chunk . activation chunk (E fp16 values = E/8 uint4).
template <int KIND>
__device__ __forceinline__ float wdot(uint4 w, const uint4* x, float acc) {
    if constexpr (KIND == MDX_W_F16) {
        return dot8_f16(w, x[0], acc);
    } else if constexpr (KIND == MDX_W_I8) {
        return dot16_i8(w, x[0], x[1], acc);
    } else {
        acc = dot8_i4(w.x, x[0], acc);
        acc = dot8_i4(w.y, x[1], acc);
        acc = dot8_i4(w.z, x[2], acc);
        return dot8_i4(w.w, x[3], acc);
    }
}

// Row-major slice: R rows of K; thread t owns chunk kc = t % CPR of rows
// RPT*i + t / CPR, i < NW.  One wave load instruction reads 1 KiB of a row
// (CPR >= 64) or two 512-byte halves (CPR == 32).
template <int KIND, int R, int K>
struct RowMajor {
    static constexpr int E = KT<KIND>::E;
    static constexpr int CPR = K / E;
    static constexpr int RPT = NT / CPR;
    static constexpr int NW = R / RPT;
    static constexpr int G = CPR < 64 ? CPR : 64;          // lanes sharing a row set
    static constexpr int NSPLIT = CPR > 64 ? CPR / 64 : 1; // waves sharing a row
    static constexpr int NV = NW <= 1 ? 1 : (NW <= 2 ? 2 : (NW <= 4 ? 4 : (NW <= 8 ? 8 : 16)));
    static_assert(NT % CPR == 0 && R % RPT == 0 && NW <= 16, "row-major slice shape");
};

// Chunk-major slice: R rows (R divides 64); thread t owns row t % R and
// chunks t / R + (NT / R) * i, i < NW (the last ones may fall past the row).
template <int KIND, int R, int K>
struct ChunkMajor {
    static constexpr int E = KT<KIND>::E;
    static constexpr int CPR = K / E;
    static constexpr int STEP = NT / R;
    static constexpr int NW = (CPR + STEP - 1) / STEP;
    static constexpr bool RAGGED = CPR % STEP != 0;
};

// Row-major dot + reduction; red[r * NSPLIT + part] receives the row sums.
template <int KIND, int R, int K, int NWT>
__device__ __forceinline__ void rm_dot(const uint4 (&w)[NWT], const uint4* xs4, float* red, int t) {
    using S = RowMajor<KIND, R, K>;
    static_assert(NWT == S::NW, "weight register count");
    constexpr int XC = S::E / 8;
    const int kc = t % S::CPR, rsub = t / S::CPR, lane = t & 63;
    uint4 xr[XC];
#pragma unroll
    for (int e = 0; e < XC; e++) xr[e] = xs4[kc * XC + e];
    float v[S::NV];
#pragma unroll
    for (int i = 0; i < S::NV; i++) v[i] = i < S::NW ? wdot<KIND>(w[i < S::NW ? i : 0], xr, 0.0f) : 0.0f;
    const float tot = reduce_scatter<S::NV, S::G>(v, lane);
    constexpr int PER = S::G / S::NV;
    const int idx = (lane % S::G) / PER;
    if ((lane % PER) == 0 && idx < S::NW)
        red[(S::RPT * idx + rsub) * S::NSPLIT + (kc / 64)] = tot;
}

template <int KIND, int R, int K, int NWT, typename RowFn>
__device__ __forceinline__ void rm_load(uint4 (&w)[NWT], const void* W, RowFn row_of, int t,
                                        int i0, int i1) {
    using S = RowMajor<KIND, R, K>;
    static_assert(NWT == S::NW, "weight register count");
    const int kc = t % S::CPR, rsub = t / S::CPR;
    const uint8_t* base = reinterpret_cast<const uint8_t*>(W) + kc * 16;
#pragma unroll
    for (int i = 0; i < S::NW; i++) {
        if (i >= i0 && i < i1)
            w[i] = ld_nt(base + (size_t)row_of(S::RPT * i + rsub) * (S::CPR * 16));
    }
}

template <int KIND, int R, int K, int NWT>
__device__ __forceinline__ void cm_load(uint4 (&w)[NWT], const void* W, int row0, int t) {
    using S = ChunkMajor<KIND, R, K>;
    static_assert(NWT == S::NW, "weight register count");
    const int r = t % R;
    const uint8_t* base = reinterpret_cast<const uint8_t*>(W) + (size_t)(row0 + r) * (S::CPR * 16);
#pragma unroll
    for (int i = 0; i < S::NW; i++) {
        // chunks past the row load chunk 0 instead; cm_dot skips them
        int kc = t / R + S::STEP * i;
        if (S::RAGGED && kc >= S::CPR) kc = 0;
        w[i] = ld_nt(base + kc * 16);
    }
}

// Chunk-major dot + reduction over lanes with equal t % R; red[wave * R + r].
template <int KIND, int R, int K, int NWT>
__device__ __forceinline__ void cm_dot(const uint4 (&w)[NWT], const uint4* xs4, float* red, int t) {
    using S = ChunkMajor<KIND, R, K>;
    static_assert(NWT == S::NW, "weight register count");
    constexpr int XC = S::E / 8;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < S::NW; i++) {
        const int kc = t / R + S::STEP * i;
        if (!S::RAGGED || kc < S::CPR) acc = wdot<KIND>(w[i], xs4 + kc * XC, acc);
    }
    static_assert(R == 4, "the row rotations below sum the lanes equal mod 4");
    acc = acc + dpp<0x124>(acc);   // row_ror:4
    acc = acc + dpp<0x128>(acc);   // row_ror:8
    acc = sum_step<16>(acc);
    acc = sum_step<32>(acc);
    const int lane = t & 63;
    if (lane < R) red[(t >> 6) * R + lane] = acc;
}

// ---- small helpers ----------------------------------------------------------

// Publishes this wave's sum of h^2 to ws[wave]; the barrier that follows
// (the wait's __syncthreads_or) makes the four partials visible.
__device__ __forceinline__ void wave_ss(const float (&h)[4], float* ws, int t) {
    const float v = wave_sum_dpp(h[0] * h[0] + h[1] * h[1] + h[2] * h[2] + h[3] * h[3]);
    if ((t & 63) == 0) ws[t >> 6] = v;
}

// fp16 x[4t..4t+4) = fp16((h * rms) * w) into the LDS activation vector.
__device__ __forceinline__ void norm_to_x(const float (&h)[4], float4 w, float rms, uint4* xs4,
                                          int t) {
    uint2 p;
    p.x = (uint32_t)f32_to_f16_bits((h[0] * rms) * w.x) | ((uint32_t)f32_to_f16_bits((h[1] * rms) * w.y) << 16);
    p.y = (uint32_t)f32_to_f16_bits((h[2] * rms) * w.z) | ((uint32_t)f32_to_f16_bits((h[3] * rms) * w.w) << 16);
    reinterpret_cast<uint2*>(xs4)[t] = p;
}

// QK-norm (optional) + RoPE of one 128-wide head held in LDS, one wave.
// With cache != NULL the results are rounded to fp16, stored there, and the
// rounded values kept (the fp16 KV-cache semantic).
// Lane i rotates the pair (i0, i1) of its style; c, s are cos/sin of pair i
// at the step's position and nw0, nw1 the norm weights of i0, i1 (all read
// before the wait that precedes this).
__device__ __forceinline__ void rope_head(const float* src, bool norm, float nw0, float nw1,
                                          float eps, float c, float s, int style, float* dst,
                                          uint16_t* cache, int lane) {
    constexpr int half = HD / 2;
    float rms = 1.0f;
    if (norm) {
        float ss = src[lane] * src[lane] + src[lane + 64] * src[lane + 64];
        ss = wave_sum_dpp(ss);
        rms = 1.0f / sqrtf(ss / (float)HD + eps);
    }
    const int i = lane;
    const int i0 = style == 0 ? 2 * i : i;
    const int i1 = style == 0 ? 2 * i + 1 : i + half;
    float x0 = src[i0], x1 = src[i1];
    if (norm) {
        x0 = (x0 * rms) * nw0;
        x1 = (x1 * rms) * nw1;
    }
    float o0 = x0 * c - x1 * s;
    float o1 = x1 * c + x0 * s;
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

__device__ __forceinline__ void h8_to_f32(uint4 u, float (&f)[8]) {
    const half2_t a = as_h2(u.x), b = as_h2(u.y), c = as_h2(u.z), d = as_h2(u.w);
    f[0] = (float)a.x; f[1] = (float)a.y; f[2] = (float)b.x; f[3] = (float)b.y;
    f[4] = (float)c.x; f[5] = (float)c.y; f[6] = (float)d.x; f[7] = (float)d.y;
}

// 2^x for x <= 0 (one v_exp_f32).  Scores are kept in the log2 domain, so the
// softmax numerators are exp2(s - max).
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- the step kernel --------------------------------------------------------

// PP: 16-position K/V passes per round (a round's rows are requested
// together).  4, or 5 for a context whose splits hold 129..160 positions (a
// little over 4096): two rounds of 80 then replace a third dependent round
// for the last few positions (W4A16 at KV 4096: 576 -> 558 us/token).  At
// short contexts 5 passes cost 10 us (int8 at KV 512), so the host picks per
// launch.
template <int KIND, int PP>
__global__ __launch_bounds__(NT) void k_persist_step(PArgs a) {
    using SA = RowMajor<KIND, 16, D>;       // qkv
    using SE = RowMajor<KIND, 24, D>;       // gate/up
    using SD = ChunkMajor<KIND, 4, QD>;     // o
    using SF = ChunkMajor<KIND, 4, FF>;     // down

    __shared__ uint4 xs4[FF / 8];
    __shared__ float red[64];
    __shared__ float ws[8];
    __shared__ float hres[4];
    __shared__ float qkv_s[512];
    __shared__ float q_s[2 * HD];
    __shared__ float kn_s[HD];
    __shared__ float vn_s[HD];
    __shared__ float att_o[4][2][HD];
    __shared__ float att_m[4][2];
    __shared__ float att_l[4][2];
    __shared__ unsigned long long bkey[4];
    __shared__ float lgs[kLogitsRows];   // this workgroup's logits (host-logits mode)

    const int t = threadIdx.x, b = blockIdx.x, lane = t & 63, wave = t >> 6;
    const int L = a.n_layers;
    unsigned* xb = a.xbuf;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(xb, (short)0, W_TOTAL * 4, 0x00020000);
    // per-head exchanges: in the XCD's L2 when a cacheable buffer is given
    const bool lx = a.xbl != nullptr;
    const __amdgpu_buffer_rsrc_t rsl =
        __builtin_amdgcn_make_buffer_rsrc(lx ? a.xbl : xb, (short)0, W_TOTAL * 4, 0x00020000);

    const unsigned E = __hip_atomic_load(xb + W_CTRL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int pos = a.in_args ? a.in_pos : a.st->pos;
    const int mode = a.in_args ? a.in_mode : a.st->mode;
    int tok = a.in_args ? a.in_token : a.st->token;
    // a timed-out wait: the device state's flag, and the host's when it reads
    // the result words without a copy
    auto flag_timeout = [&]() {
        __hip_atomic_store(&a.st->pad[1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a.res_host) __hip_atomic_store(&a.res_host[1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    };
    bool dead = false;
    const unsigned spin_lim = a.spin_limit;
    const bool kv_nt = a.kv_stream != 0;

    // attention work split of this workgroup
    const int j = b % NKV, s = b / NKV;
    const KvSplit ksp = kv_split(pos, s);
    const int p0 = ksp.p0, n = ksp.n;
    const int p1 = p0 + n;
    const bool has_new = pos >= p0 && pos < p1;
    const int pl = t >> 4, dl = t & 15;

    // qkv row map: 16 consecutive rows of one head
    const int seg = s >> 3, r0 = (s & 7) * 16;
    const int qkv_row0 = seg == 0 ? (2 * j) * HD + r0
                       : seg == 1 ? (2 * j + 1) * HD + r0
                       : seg == 2 ? QD + j * HD + r0
                                  : QD + KVD + j * HD + r0;
    auto rowA = [&](int r) { return qkv_row0 + r; };
    auto rowE = [&](int r) { return r < 12 ? 12 * b + r : FF + 12 * b + (r - 12); };

    uint4 wA[SA::NW];
    rm_load<KIND, 16, D>(wA, a.l0.wqkv, rowA, t, 0, SA::NW);

    // K/V rows of one round (passes q0 .. q0 + PP - 1) of this workgroup's
    // split: unconditional loads (row 0 stands in for unused slots), so the
    // requests are not tied to a branch that waits for them
    uint4 kr[PP], vr[PP];
    auto load_kv_at = [&](const uint16_t* kc, const uint16_t* vc, uint4 (&kk)[PP], uint4 (&vv)[PP], int q0) {
        if (kv_nt) {
#pragma unroll
            for (int qq = 0; qq < PP; qq++) {
                const size_t off = (size_t)kv_row(ksp, 16 * (q0 + qq) + pl, pos) * KVD + j * HD + dl * 8;
                kk[qq] = ld_nt(kc + off);
                vv[qq] = ld_nt(vc + off);
            }
        } else {
#pragma unroll
            for (int qq = 0; qq < PP; qq++) {
                const size_t off = (size_t)kv_row(ksp, 16 * (q0 + qq) + pl, pos) * KVD + j * HD + dl * 8;
                kk[qq] = *reinterpret_cast<const uint4*>(kc + off);
                vv[qq] = *reinterpret_cast<const uint4*>(vc + off);
            }
        }
    };
    // The next layer's first K/V round is requested at the end of the gate|up
    // stage, so it streams during the activation exchange instead of holding
    // up the q wait (loads complete in issue order): fp16 KV 512 414.4 ->
    // 405.5, int8 KV 512 405.3 -> 403.7, W4A16 KV 4096 493.2 -> 481.6
    // us/token. fp16 layers with a streamed cache (long contexts) keep the
    // request in their own qkv stage: KV 4096 +3 us/token with the early one.
    const bool early_kv = KIND != MDX_W_F16 || !kv_nt;

    // layer-0 input: the token's embedding row (or the uploaded embedding)
    float h[4];
    {
        tok = tok < 0 ? 0 : (tok >= a.vocab ? a.vocab - 1 : tok);
        const float* src = mode == 1 ? a.emb_in : a.emb_table + (size_t)tok * D;
        const float4 v = reinterpret_cast<const float4*>(src)[t];
        h[0] = v.x; h[1] = v.y; h[2] = v.z; h[3] = v.w;
    }

    // lm_head rows of this workgroup; the first batch is requested during the
    // last layer's gate/up stage.  Rows per wave batch (power of two, <= 64):
    // the first batch's registers are live through the whole layer loop (it
    // is loaded inside the loop and used after it), and the kernel runs at
    // the register limit, with AGPRs as spill space.  8-row batches free 32 of
    // them: with fp16 layers 473.1 -> 471.3 us/token, int4 at KV 4096 580.1 ->
    // 567.3 (4 is slower for both: the lm_head keeps fewer bytes in flight).
    // With int8 layers the first batch of 16 rows goes straight to LDS instead
    // (global_load_lds, no registers): 460.5 -> 456.4 us/token; the same for
    // fp16 and int4 costs 1.5 and 2.5 us.
    constexpr int U = KIND == MDX_W_I8 ? 16 : 8;
    constexpr bool kLmLds = KIND == MDX_W_I8;
    constexpr int PER = 64 / U;         // lanes holding one row's total
    const int rb = (int)(((long long)b * a.vocab) / NB);
    const int re = (int)(((long long)(b + 1) * a.vocab) / NB);
    auto load_rows = [&](uint4 (&w)[U], float& sc, int base) {
        // rows past the workgroup's range re-read row re-1; consume skips them
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int r = min(base + u, re - 1);
            w[u] = *reinterpret_cast<const uint4*>(a.lm_w + (size_t)r * D + lane * 16);
        }
        sc = a.lm_scale[min(base + lane / PER, re - 1)];
    };
    uint4 w0[U];
    float sc0 = 0.0f;
    __shared__ uint4 lmb[kLmLds ? 4 : 1][kLmLds ? U : 1][64];   // [wave][row][lane]

    for (int l = 0; l < L; l++) {
        const mdx_persist_layer Ly = layer_at(a, l);
        const unsigned ep = step_epoch(E, L, l);
        const unsigned ep_prev = step_epoch(E, L, l - 1 < 0 ? 0 : l - 1);

        // ================= A: RMSNorm + qkv =================
        MDX_TRACE(16 * l + 0);
        const float4 nwA = reinterpret_cast<const float4*>(Ly.in_norm)[t];
        // stage B inputs that do not depend on this step's activations
        const float rc = a.cos_t[(size_t)pos * (HD / 2) + lane];
        const float rsn = a.sin_t[(size_t)pos * (HD / 2) + lane];
        const int ri0 = a.rope_style == 0 ? 2 * lane : lane;
        const int ri1 = a.rope_style == 0 ? 2 * lane + 1 : lane + HD / 2;
        const float* qknw = wave < 2 ? Ly.q_norm : Ly.k_norm;
        const float rn0 = qknw ? qknw[ri0] : 1.0f;
        const float rn1 = qknw ? qknw[ri1] : 1.0f;
        // int4 layers: the column scales are requested by wave 0 alone, which
        // applies them, and the SwiGLU epilogue reads the gate and up sums of
        // its feature straight from the reduction (W4A16 KV 4000 497.7 -> 486.1
        // us/token, tokens unchanged; the same code measured +0.7 us with fp16
        // and +1.8 us with int8 layers at KV 512, so those keep the form below)
        constexpr bool kLean = KIND == MDX_W_I4;
        float sclA = Ly.sqkv && (!kLean || wave == 0) ? Ly.sqkv[qkv_row0 + (t & 15)] : 1.0f;
        // int8/int4 layers: the o column scale is requested here, well ahead of
        // the gate|up and down weight requests. Loads complete in issue order,
        // so a scale read after them made the h-after-o store wait for all of
        // those weights (int8 KV 512 403.1 -> 402.0, W4A16 KV 4096 496.3 ->
        // 491.5 us/token). fp16 layers keep the late read (+1.3 us/token at
        // KV 512 with the early one).
        constexpr bool kEarlyD = KIND != MDX_W_F16;
        float sclD = 1.0f;
        if constexpr (kEarlyD) sclD = Ly.so && (!kLean || wave == 0) ? Ly.so[4 * b + (t & 3)] : 1.0f;
        if (l > 0) {
            const int wb = W_HD + (b % NREP) * (2 * D) + 8 * t;
            int wd[2] = {wb, wb + 4};
            u32x4 v[2];
            const bool ok = ll_wait<2>(rs, wd, v, ep_prev, dead, spin_lim);
            h[0] = ll_f32(v[0].x, v[0].y); h[1] = ll_f32(v[0].z, v[0].w);
            h[2] = ll_f32(v[1].x, v[1].y); h[3] = ll_f32(v[1].z, v[1].w);
            wave_ss(h, ws, t);
            if (__syncthreads_or(!ok)) dead = true;
        } else {
            wave_ss(h, ws, t);
            __syncthreads();
        }
        // weight requests go out after the wait, so they do not queue in front
        // of the exchange's own reads
        auto load_kv = [&](uint4 (&kk)[PP], uint4 (&vv)[PP], int q0) { load_kv_at(Ly.kc, Ly.vc, kk, vv, q0); };
        uint4 wD[SD::NW];
        cm_load<KIND, 4, QD>(wD, Ly.wo, 4 * b, t);
        MDX_TRACE(16 * l + 1);
        if (t == b) { hres[0] = h[0]; hres[1] = h[1]; hres[2] = h[2]; hres[3] = h[3]; }
        {
            const float tot = (ws[0] + ws[1]) + (ws[2] + ws[3]);
            const float rms = 1.0f / sqrtf(tot / (float)D + a.eps);
            norm_to_x(h, nwA, rms, xs4, t);
        }
        __syncthreads();
        rm_dot<KIND, 16, D>(wA, xs4, red, t);
        // Layer 0, and fp16 layers with a streamed cache, request their first
        // K/V round here (the others did at the end of the previous layer's
        // gate|up stage): after the qkv GEMV, which otherwise waits for part
        // of it (fp16 at KV 4096 556.5 -> 550.7, W4A16 at KV 4096 561.5 -> 556
        // us/token). The column scale is forced into a register first: loads
        // complete in issue order, so a wait for it placed after later
        // requests would wait for them too and hold back the qkv store (int8
        // KV 512 407.4 -> 404.5 us/token)
        asm volatile("" : "+v"(sclA));
        if (!early_kv || l == 0) load_kv(kr, vr, 0);
        __syncthreads();
        if (wave == 0) {
            // lanes 0..15 hold rows s*16 + lane; even lanes store two rows in one
            // 16-byte group (eight stores instead of 32 four-byte ones)
            float y = 0.0f;
            if (t < 16) {
                y = red[t * SA::NSPLIT];
                if (SA::NSPLIT == 2) y = y + red[t * SA::NSPLIT + 1];
                y = y * sclA;
            }
            const float y1 = kLean ? dpp<0x101>(y) : __shfl_down(y, 1, 64);   // lane t + 1's y
            if (t < 16 && (t & 1) == 0) {
                const int w = W_QKV + j * 1024 + 2 * (s * 16 + t);
                if (lx) lx_put4(rsl, w, ll_pack2(y, y1, ep));
                else ll_put4(rs, w, ll_pack2(y, y1, ep));
            }
        }
        MDX_TRACE(16 * l + 2);

        // ================= B: QK-norm, RoPE, KV append, partial attention ==========
        uint4 wE[SE::NW];
        {
            // q (values 0..255, threads < 128) is needed by every split; the
            // new k and v only by the split holding position pos, so the
            // others wait for the 16 q writers alone
            const bool need = t < 128 || has_new;
            int wd[1] = {W_QKV + j * 1024 + 4 * t};
            u32x4 v[1];
            const bool ok = lx ? ll_wait<1, kLocalPoll>(rsl, wd, v, ep, dead || !need, spin_lim)
                               : ll_wait<1>(rs, wd, v, ep, dead || !need, spin_lim);
            qkv_s[2 * t] = ll_f32(v[0].x, v[0].y);
            qkv_s[2 * t + 1] = ll_f32(v[0].z, v[0].w);
            if (__syncthreads_or(!ok)) dead = true;
        }
        // the q wait has drained every earlier load: pinning the o scale in a
        // register here costs no wait and keeps any later one off its use
        if constexpr (kEarlyD) asm volatile("" : "+v"(sclD));
        rm_load<KIND, 24, D>(wE, Ly.wgu, rowE, t, 0, SE::NW / 2);
        MDX_TRACE(16 * l + 3);
        if (wave < 2) {
            rope_head(qkv_s + wave * HD, Ly.q_norm != nullptr, rn0, rn1, a.eps, rc, rsn,
                      a.rope_style, q_s + wave * HD, nullptr, lane);
        } else if (has_new && wave == 2) {
            rope_head(qkv_s + 2 * HD, Ly.k_norm != nullptr, rn0, rn1, a.eps, rc, rsn, a.rope_style,
                      kn_s, Ly.kc + (size_t)pos * KVD + j * HD, lane);
        } else if (has_new) {
            for (int e = lane; e < HD; e += 64) {
                const uint16_t hv = f32_to_f16_bits(qkv_s[3 * HD + e]);
                Ly.vc[(size_t)pos * KVD + j * HD + e] = hv;
                vn_s[e] = f16_bits_to_f32(hv);
            }
        }
        __syncthreads();
        MDX_TRACE(16 * l + 12);
        // Online softmax per wave: each wave keeps one running maximum per head
        // (shared by its four 16-lane position rows) and rescales its running
        // sums when a round raises it.  After the last round the four rows are
        // summed on the VALU and the four waves merged through LDS.
        // (runM, runL, runO) of thread t: head t >> 7, dimension t & 127.
        float runM = -INFINITY, runL = 0.0f, runO = 0.0f;
        {
            float q[2][8];
#pragma unroll
            for (int hh = 0; hh < 2; hh++)
#pragma unroll
                for (int e = 0; e < 8; e++) q[hh][e] = q_s[hh * HD + dl * 8 + e];
            float Mw[2] = {-INFINITY, -INFINITY}, ls[2] = {0.0f, 0.0f}, o[2][8];
#pragma unroll
            for (int hh = 0; hh < 2; hh++)
#pragma unroll
                for (int e = 0; e < 8; e++) o[hh][e] = 0.0f;
            auto round = [&](const uint4 (&kk)[PP], const uint4 (&vv)[PP], int q0) {
                float sc[PP][2], vf[PP][8];
#pragma unroll
                for (int qq = 0; qq < PP; qq++) {
                    sc[qq][0] = -INFINITY;
                    sc[qq][1] = -INFINITY;
                    if (16 * (q0 + qq) >= n) continue;   // the whole pass lies past the chunk
                    const int pi = 16 * (q0 + qq) + pl;
                    const bool isnew = pi < n && p0 + pi == pos;
                    float kf[8];
                    if (isnew) {
#pragma unroll
                        for (int e = 0; e < 8; e++) {
                            kf[e] = kn_s[dl * 8 + e];
                            vf[qq][e] = vn_s[dl * 8 + e];
                        }
                    } else {
                        h8_to_f32(kk[qq], kf);
                        h8_to_f32(vv[qq], vf[qq]);
                    }
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) {
                        const float* qh = q[hh];
                        float acc = qh[0] * kf[0];
#pragma unroll
                        for (int e = 1; e < 8; e++) acc = fmaf(qh[e], kf[e], acc);
                        // log2(e) / sqrt(128): scores in the log2 domain
                        const float v = row_sum16(acc) * 0.12751743074924928f;
                        sc[qq][hh] = pi < n ? v : -INFINITY;
                    }
                }
                float mx[2] = {-INFINITY, -INFINITY};
#pragma unroll
                for (int qq = 0; qq < PP; qq++)
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) mx[hh] = fmaxf(mx[hh], sc[qq][hh]);
                if (q0 == 0) MDX_TRACE(16 * l + 14);
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    const float Mn = fmaxf(Mw[hh], rows_max4(mx[hh]));   // uniform over the wave
                    if (Mn != -INFINITY) {
                        const float a = Mw[hh] == -INFINITY ? 0.0f : exp2_fast(Mw[hh] - Mn);
                        ls[hh] = ls[hh] * a;
#pragma unroll
                        for (int e = 0; e < 8; e++) o[hh][e] = o[hh][e] * a;
                        Mw[hh] = Mn;
                    }
                }
#pragma unroll
                for (int qq = 0; qq < PP; qq++) {
                    if (16 * (q0 + qq) >= n) continue;
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) {
                        const float p = sc[qq][hh] == -INFINITY ? 0.0f : exp2_fast(sc[qq][hh] - Mw[hh]);
                        ls[hh] = ls[hh] + p;
#pragma unroll
                        for (int e = 0; e < 8; e++) o[hh][e] = fmaf(p, vf[qq][e], o[hh][e]);
                    }
                }
            };
            // chunks longer than 16*PP positions: with int8/int4 weights the rows
            // of the next round are requested before the current round is
            // computed (two register sets)
            auto load_round = [&](uint4 (&kk)[PP], uint4 (&vv)[PP], int q0) { load_kv(kk, vv, q0); };
            uint4 kx[PP], vx[PP];
            if constexpr (KIND != MDX_W_F16) {
                if (16 * PP < n) load_round(kx, vx, PP);
                round(kr, vr, 0);
                for (int q0 = PP; 16 * q0 < n; q0 += 2 * PP) {
                    if (16 * (q0 + PP) < n) load_round(kr, vr, q0 + PP);
                    round(kx, vx, q0);
                    if (16 * (q0 + PP) >= n) break;
                    if (16 * (q0 + 2 * PP) < n) load_round(kx, vx, q0 + 2 * PP);
                    round(kr, vr, q0 + PP);
                }
            } else {
                // fp16 weights leave no registers for a second set: one round at a time
                round(kr, vr, 0);
                for (int q0 = PP; 16 * q0 < n; q0 += PP) {
                    load_round(kx, vx, q0);
                    round(kx, vx, q0);
                }
            }

            // the four position rows of each wave, then the four waves
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                ls[hh] = rows_sum4(ls[hh]);
#pragma unroll
                for (int e = 0; e < 8; e++) o[hh][e] = rows_sum4(o[hh][e]);
            }
            if (lane < 16) {
#pragma unroll
                for (int hh = 0; hh < 2; hh++)
#pragma unroll
                    for (int e = 0; e < 8; e++) att_o[wave][hh][dl * 8 + e] = o[hh][e];
                if (lane == 0) {
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) {
                        att_m[wave][hh] = Mw[hh];
                        att_l[wave][hh] = ls[hh];
                    }
                }
            }
            __syncthreads();
            const int hh = t >> 7, d = t & 127;
            float Mx = att_m[0][hh];
#pragma unroll
            for (int w = 1; w < 4; w++) Mx = fmaxf(Mx, att_m[w][hh]);
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float mw = att_m[w][hh];
                const float f = mw == -INFINITY ? 0.0f : exp2_fast(mw - Mx);
                runO = runO + att_o[w][hh][d] * f;
                runL = runL + att_l[w][hh] * f;
            }
            runM = Mx;
            __syncthreads();   // att_o is reused for the partial record below
        }
        MDX_TRACE(16 * l + 13);
        {
            // 16-byte stores: thread t < 128 writes values 2t and 2t+1
            const int hh = t >> 7, d = t & 127;
            const int jb = W_PART + j * PART_WORDS_J;
            float* po = &att_o[0][0][0];
            po[t] = runO;
            __syncthreads();
            if (t < 128) {
                // values v, v + 1 of head v >> 7: dimension block dd >> 3, slot dd & 7
                const int v = 2 * t, h2 = v >> 7, dd = v & 127;
                const int w = jb + ((h2 * 16 + (dd >> 3)) * GRP + s) * 16 + 2 * (dd & 7);
                if (lx) lx_put4(rsl, w, ll_pack2(po[v], po[v + 1], ep));
                else ll_put4(rs, w, ll_pack2(po[v], po[v + 1], ep));
            }
            if (d == 0) {
                const int w = jb + PART_O + (hh * GRP + s) * 4;
                if (lx) lx_put4(rsl, w, ll_pack2(runM, runL, ep));
                else ll_put4(rs, w, ll_pack2(runM, runL, ep));
            }
        }
        MDX_TRACE(16 * l + 4);

        uint4 wF[SF::NW];

        // ================= C: merge the 32 partials of KV head j (wave 0) ==========
        // lane i < 32 holds split i's (m, l) (lanes 32..63 the same again); the
        // two 1 KiB loads give lane L the values 2 (L & 3), +1 of splits L >> 2
        // and 16 + (L >> 2)
        if (wave == 0) {
            const int hh = s >> 4, c = s & 15, d0 = c * 8;
            const int jb = W_PART + j * PART_WORDS_J;
            const int ob = jb + (hh * 16 + c) * GRP * 16;
            int wd[3] = {jb + PART_O + (hh * GRP + (lane & 31)) * 4, ob + 4 * lane, ob + 256 + 4 * lane};
            u32x4 v[3];
            if (!(lx ? ll_wait<3, kLocalPoll>(rsl, wd, v, ep, dead, spin_lim)
                     : ll_wait<3>(rs, wd, v, ep, dead, spin_lim)))
                dead = true;
            const float m = ll_f32(v[0].x, v[0].y);
            const float M = half_max_dpp(m);
            const float w = m == -INFINITY ? 0.0f : exp2_fast(m - M);
            const float Ls = half_sum_dpp(ll_f32(v[0].z, v[0].w) * w);
            const float wa = __shfl(w, lane >> 2, 64), wb = __shfl(w, 16 + (lane >> 2), 64);
            float p0 = ll_f32(v[1].x, v[1].y) * wa + ll_f32(v[2].x, v[2].y) * wb;
            float p1 = ll_f32(v[1].z, v[1].w) * wa + ll_f32(v[2].z, v[2].w) * wb;
            // sum over the 16 lanes of each slot pair (lanes equal mod 4): two
            // rotations inside each 16-lane row, then the row swaps across rows
            // (instead of four LDS-routed shuffles: fp16 KV 512 423.1 -> 417.7
            // us/token)
            p0 = p0 + dpp<0x124>(p0);   // row_ror:4
            p1 = p1 + dpp<0x124>(p1);
            p0 = p0 + dpp<0x128>(p0);   // row_ror:8
            p1 = p1 + dpp<0x128>(p1);
            p0 = rows_sum4(p0);
            p1 = rows_sum4(p1);
            float O[8];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                O[2 * k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p0), k));
                O[2 * k + 1] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p1), k));
            }
            if (lane < 2 * NREP) {   // lane: copy lane / 2, half lane % 2
                const unsigned e = ep << 16;
                u32x4 pk;
                const bool hi = (lane & 1) == 1;
                pk.x = f32_to_f16_bits((hi ? O[4] : O[0]) / Ls) | e;
                pk.y = f32_to_f16_bits((hi ? O[5] : O[1]) / Ls) | e;
                pk.z = f32_to_f16_bits((hi ? O[6] : O[2]) / Ls) | e;
                pk.w = f32_to_f16_bits((hi ? O[7] : O[3]) / Ls) | e;
                ll_put4(rs, W_ATT + (lane >> 1) * QD + (2 * j + hh) * HD + d0 + 4 * (lane & 1), pk);
            }
        }
        // The remaining gate/up and the down weights are requested once the
        // merge is done: a burst issued while the partial records are in
        // flight delays them (measured: 522 -> 510 us/token against requesting
        // from waves 1..3 before the merge).  With fp16 weights (the largest
        // burst) waves 1 and 2, which gather the attention output next,
        // request theirs after that gather, so their polls do not wait behind
        // the weights (478.0 -> 475.6 us/token; with int8 or int4 weights the
        // same split costs 6-8 us, so there every wave requests here).
        constexpr bool kSplitReq = KIND == MDX_W_F16;
        __syncthreads();
        if (!kSplitReq || wave == 0 || wave == 3) {
            rm_load<KIND, 24, D>(wE, Ly.wgu, rowE, t, SE::NW / 2, SE::NW);
            cm_load<KIND, 4, FF>(wF, Ly.wdown, 4 * b, t);
        }
        MDX_TRACE(16 * l + 5);

        // ================= D: o projection + residual ==========
        if constexpr (!kEarlyD) sclD = Ly.so ? Ly.so[4 * b + (t & 3)] : 1.0f;
        {
            // waves 1 and 2 gather the attention output: thread u reads the
            // 16-byte groups u + 128 k (4 values each), k < 4
            bool ok = true;
            if (wave == 1 || wave == 2) {
                const int u = t - 64;
                const int wb = W_ATT + (b % NREP) * QD + 4 * u;
                int wd[4] = {wb, wb + 512, wb + 1024, wb + 1536};
                u32x4 v[4];
                ok = ll_wait<4>(rs, wd, v, ep, dead, spin_lim);
                uint4 x0, x1;
                x0.x = (v[0].x & 0xffffu) | (v[0].y << 16);
                x0.y = (v[0].z & 0xffffu) | (v[0].w << 16);
                x0.z = (v[1].x & 0xffffu) | (v[1].y << 16);
                x0.w = (v[1].z & 0xffffu) | (v[1].w << 16);
                x1.x = (v[2].x & 0xffffu) | (v[2].y << 16);
                x1.y = (v[2].z & 0xffffu) | (v[2].w << 16);
                x1.z = (v[3].x & 0xffffu) | (v[3].y << 16);
                x1.w = (v[3].z & 0xffffu) | (v[3].w << 16);
                uint2* x2 = reinterpret_cast<uint2*>(xs4);
                x2[u] = make_uint2(x0.x, x0.y);
                x2[u + 128] = make_uint2(x0.z, x0.w);
                x2[u + 256] = make_uint2(x1.x, x1.y);
                x2[u + 384] = make_uint2(x1.z, x1.w);
                if (kSplitReq) {
                    rm_load<KIND, 24, D>(wE, Ly.wgu, rowE, t, SE::NW / 2, SE::NW);
                    cm_load<KIND, 4, FF>(wF, Ly.wdown, 4 * b, t);
                }
            }
            if (__syncthreads_or(!ok || dead)) dead = true;   // wave 0 may have timed out in C
        }
        MDX_TRACE(16 * l + 6);
        cm_dot<KIND, 4, QD>(wD, xs4, red, t);
        __syncthreads();
        if (wave == 0) {
            const int r = t & 3;
            const float y = ((red[r] + red[4 + r]) + (red[8 + r] + red[12 + r])) * sclD;
            put_hidden4(rs, W_HO, b, hres[r] + y, ep, lane);
        }
        MDX_TRACE(16 * l + 7);

        // ================= E: RMSNorm + gate/up + SwiGLU ==========
        const bool last = l + 1 == L;
        // The next layer's qkv weights. fp16 layers request them in two halves,
        // after the h wait below and after the activation wait, so the h wait
        // does not queue behind 32 KB of requests (KV 512 416.7 -> 415.0
        // us/token); int8 and int4 layers request them here (the split measured
        // +6 us/token for both).
        constexpr bool kSplitA = KIND == MDX_W_F16;
        if (!kSplitA && !last) rm_load<KIND, 16, D>(wA, layer_at(a, l + 1).wqkv, rowA, t, 0, SA::NW);
        else if (last && a.head) {
            if constexpr (kLmLds) {
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const int r = min(rb + wave * U + u, re - 1);
                    __builtin_amdgcn_global_load_lds(a.lm_w + (size_t)r * D + lane * 16,
                                                     (__attribute__((address_space(3))) void*)&lmb[wave][u][0],
                                                     16, 0, 0);
                }
                sc0 = a.lm_scale[min(rb + wave * U + lane / PER, re - 1)];
            } else {
                load_rows(w0, sc0, rb + wave * U);
            }
        }
        const float4 nwE = reinterpret_cast<const float4*>(Ly.post_norm)[t];
        const float sclE = Ly.sgu && (!kLean || wave == 0) ? Ly.sgu[rowE(kLean ? (t < 12 ? t : 0) : (t < 24 ? t : 0))]
                                                           : 1.0f;
        const float sclU = kLean && Ly.sgu && wave == 0 ? Ly.sgu[rowE(t < 12 ? t + 12 : 12)] : 1.0f;
        {
            const int wb = W_HO + (b % NREP) * (2 * D) + 8 * t;
            int wd[2] = {wb, wb + 4};
            u32x4 v[2];
            const bool ok = ll_wait<2>(rs, wd, v, ep, dead, spin_lim);
            h[0] = ll_f32(v[0].x, v[0].y); h[1] = ll_f32(v[0].z, v[0].w);
            h[2] = ll_f32(v[1].x, v[1].y); h[3] = ll_f32(v[1].z, v[1].w);
            wave_ss(h, ws + 4, t);
            if (__syncthreads_or(!ok)) dead = true;
        }
        if (kSplitA && !last) rm_load<KIND, 16, D>(wA, layer_at(a, l + 1).wqkv, rowA, t, 0, SA::NW / 2);
        MDX_TRACE(16 * l + 8);
        if (t == b) { hres[0] = h[0]; hres[1] = h[1]; hres[2] = h[2]; hres[3] = h[3]; }
        {
            const float tot = (ws[4] + ws[5]) + (ws[6] + ws[7]);
            const float rms = 1.0f / sqrtf(tot / (float)D + a.eps);
            norm_to_x(h, nwE, rms, xs4, t);
        }
        __syncthreads();
        rm_dot<KIND, 24, D>(wE, xs4, red, t);
        __syncthreads();
        if (wave == 0) {
            unsigned act;
            if constexpr (kLean) {
                // lane k < 12: feature k, the gate row k and the up row k + 12
                const int r = lane < 12 ? lane : 0;
                float y = red[r * SE::NSPLIT];
                float u = red[(r + 12) * SE::NSPLIT];
                if (SE::NSPLIT == 2) {
                    y = y + red[r * SE::NSPLIT + 1];
                    u = u + red[(r + 12) * SE::NSPLIT + 1];
                }
                act = f32_to_f16_bits(silu_mul(y * sclE, u * sclU));
            } else {
                // lane k < 24: row k (gate k < 12, up k - 12); lane k < 12 then
                // holds feature k's activation
                const int r = lane < 24 ? lane : 0;
                float y = red[r * SE::NSPLIT];
                if (SE::NSPLIT == 2) y = y + red[r * SE::NSPLIT + 1];
                y = y * sclE;
                const float u = __shfl(y, (lane + 12) & 63, 64);
                act = f32_to_f16_bits(silu_mul(y, u));
            }
            // feature k's activation, broadcast with readlane
            unsigned av[12];
#pragma unroll
            for (int k = 0; k < 12; k++) av[k] = __builtin_amdgcn_readlane(act, k);
            if (lane < 3 * NREP) {
                // lane: copy lane / 3, features 4 (lane % 3) .. +3 in one 16-byte store
                const int c = lane % 3;
                const unsigned e = ep << 16;
                u32x4 pk;
                pk.x = (c == 0 ? av[0] : c == 1 ? av[4] : av[8]) | e;
                pk.y = (c == 0 ? av[1] : c == 1 ? av[5] : av[9]) | e;
                pk.z = (c == 0 ? av[2] : c == 1 ? av[6] : av[10]) | e;
                pk.w = (c == 0 ? av[3] : c == 1 ? av[7] : av[11]) | e;
                ll_put4(rs, W_ACT + (lane / 3) * (NB * 12) + 12 * b + 4 * c, pk);
            }
        }
        MDX_TRACE(16 * l + 9);
        if (early_kv && !last) {
            const mdx_persist_layer Ln = layer_at(a, l + 1);
            load_kv_at(Ln.kc, Ln.vc, kr, vr, 0);
        }

        // ================= F: down projection + residual ==========
        const float sclF = Ly.sdown && (!kLean || wave == 0) ? Ly.sdown[4 * b + (t & 3)] : 1.0f;
        MDX_TRACE(16 * l + 15);
        {
            // thread t reads the 16-byte groups t, t + 256, t + 512; group g
            // holds the activations 4 g .. 4 g + 3
            const int wb = W_ACT + (b % NREP) * (NB * 12) + 4 * t;
            int wd[3] = {wb, wb + 1024, wb + 2048};
            u32x4 v[3];
            const bool ok = ll_wait_probe<3>(rs, wd, v, ep, dead, spin_lim);
            uint2* x2 = reinterpret_cast<uint2*>(xs4);
#pragma unroll
            for (int k = 0; k < 3; k++) {
                uint2 p;
                p.x = (v[k].x & 0xffffu) | (v[k].y << 16);
                p.y = (v[k].z & 0xffffu) | (v[k].w << 16);
                x2[t + 256 * k] = p;
            }
            if (__syncthreads_or(!ok)) dead = true;
        }
        MDX_TRACE(16 * l + 10);
        if (kSplitA && !last) rm_load<KIND, 16, D>(wA, layer_at(a, l + 1).wqkv, rowA, t, SA::NW / 2, SA::NW);
        cm_dot<KIND, 4, FF>(wF, xs4, red, t);
        __syncthreads();
        if (wave == 0) {
            const int r = t & 3;
            const float y = ((red[r] + red[4 + r]) + (red[8 + r] + red[12 + r])) * sclF;
            const float hn = hres[r] + y;
            put_hidden4(rs, W_HD, b, hn, ep, lane);
            if (last && t < 4) a.hidden_out[4 * b + t] = hn;
        }
        MDX_TRACE(16 * l + 11);
        __syncthreads();   // hres / red reuse
    }

    const unsigned ep_last = step_epoch(E, L, L - 1);
    const unsigned ep_head = step_epoch(E, L, L);
    if (a.head) {
        // ================= lm_head (INT8 rows, fp16 activations) + argmax ==========
        // three row batches per wave: two in flight while one is multiplied
        uint4 w1[U], w2[U];
        float sc1 = 0.0f, sc2 = 0.0f;
        const float4 nw = reinterpret_cast<const float4*>(a.final_norm)[t];
        // the second batch is requested before the wait (measured: the longer
        // wait costs less than the later start of the stream)
        if (rb + wave * U + 4 * U < re) load_rows(w1, sc1, rb + wave * U + 4 * U);
        {
            const int wb = W_HD + (b % NREP) * (2 * D) + 8 * t;
            int wd[2] = {wb, wb + 4};
            u32x4 v[2];
            const bool ok = ll_wait<2>(rs, wd, v, ep_last, dead, spin_lim);
            h[0] = ll_f32(v[0].x, v[0].y); h[1] = ll_f32(v[0].z, v[0].w);
            h[2] = ll_f32(v[1].x, v[1].y); h[3] = ll_f32(v[1].z, v[1].w);
            wave_ss(h, ws, t);
            if (__syncthreads_or(!ok)) dead = true;
        }
        MDX_TRACE(16 * L + 0);
        if constexpr (kLmLds) {
            // this wave's loads complete in order, so its LDS batch landed
            // before the h words it has just read
#pragma unroll
            for (int u = 0; u < U; u++) w0[u] = lmb[wave][u][lane];
        }
        {
            const float tot = (ws[0] + ws[1]) + (ws[2] + ws[3]);
            const float rms = 1.0f / sqrtf(tot / (float)D + a.eps);
            norm_to_x(h, nw, rms, xs4, t);
        }
        __syncthreads();
        const uint4 x0 = xs4[2 * lane], x1 = xs4[2 * lane + 1];
        unsigned long long best = 0ull;
        auto consume = [&](const uint4 (&w)[U], float sc, int base) {
            float v[U];
#pragma unroll
            for (int u = 0; u < U; u++) v[u] = dot16_i8(w[u], x0, x1, 0.0f);
            const float tot = reduce_scatter<U, 64>(v, lane);
            const int r = base + lane / PER;
            if ((lane % PER) == 0 && r < re) {
                const float y = tot * sc;
                if (a.logits_host) lgs[r - rb] = y;
                else a.logits[r] = y;
                const unsigned long long k = ref_argmax_key(y, r);
                best = k > best ? k : best;
            }
        };
        // this wave's batches start at rb + wave*U, 4U rows apart
        for (int base = rb + wave * U; base < re; base += 12 * U) {
            if (base + 8 * U < re) load_rows(w2, sc2, base + 8 * U);
            consume(w0, sc0, base);
            if (base + 4 * U >= re) break;
            if (base + 12 * U < re) load_rows(w0, sc0, base + 12 * U);
            consume(w1, sc1, base + 4 * U);
            if (base + 8 * U >= re) break;
            if (base + 16 * U < re) load_rows(w1, sc1, base + 16 * U);
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
        if (t == 0) {
            unsigned long long k = bkey[0];
            for (int w = 1; w < 4; w++) k = bkey[w] > k ? bkey[w] : k;
            const unsigned hi = (unsigned)(k >> 32), lo = (unsigned)k;
            const int base = W_AMAX + 4 * b;
            ll_put(xb, base + 0, hi & 0xffffu, ep_head);
            ll_put(xb, base + 1, hi >> 16, ep_head);
            ll_put(xb, base + 2, lo & 0xffffu, ep_head);
            ll_put(xb, base + 3, lo >> 16, ep_head);
        }
        MDX_TRACE(16 * L + 1);
        if (a.trace && t == 0)
            a.trace[(size_t)b * a.trace_stride + 16 * L + 3] = __builtin_amdgcn_s_getreg((3 << 11) | 20);
        // the logits go to the mapped host buffer as whole rows of 256 values
        // per store instruction, after the loads (so no poll waits behind
        // them); workgroup 0 writes its rows after the argmax
        auto logits_out = [&]() {
            for (int i = t; i < re - rb; i += NT) a.logits_host[rb + i] = lgs[i];
        };
        if (b != 0) {
            if (a.logits_host) logits_out();
            if (dead && t == 0) flag_timeout();
            return;
        }
        __syncthreads();   // bkey is reused below
        unsigned long long k = 0ull;
        {
            int wd[1] = {W_AMAX + 4 * t};
            u32x4 v[1];
            const bool ok = ll_wait<1>(rs, wd, v, ep_head, dead, spin_lim);
            const unsigned hi = (v[0].x & 0xffffu) | (v[0].y << 16);
            const unsigned lo = (v[0].z & 0xffffu) | (v[0].w << 16);
            k = ((unsigned long long)hi << 32) | lo;
            if (!ok) dead = true;
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const unsigned lo = __shfl_xor((unsigned)(k & 0xffffffffull), off, 64);
            const unsigned hi = __shfl_xor((unsigned)(k >> 32), off, 64);
            const unsigned long long k2 = ((unsigned long long)hi << 32) | lo;
            k = k2 > k ? k2 : k;
        }
        if (lane == 0) bkey[wave] = k;
        if (__syncthreads_or(dead)) dead = true;
        if (t == 0) {
            unsigned long long kk = bkey[0];
            for (int w = 1; w < 4; w++) kk = bkey[w] > kk ? bkey[w] : kk;
            const int res = ref_argmax_index(kk);
            mdx_state* st = a.st;
            st->argmax = res;
            st->token = res;
            st->mode = 0;
            if (a.out_tokens) {
                a.out_tokens[st->n_out] = res;
                st->n_out = st->n_out + 1;
            }
            st->pos = pos + a.advance;
            if (dead) flag_timeout();
            if (a.res_host) __hip_atomic_store(&a.res_host[0], res, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(xb + W_CTRL, E + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (a.logits_host) logits_out();
        MDX_TRACE(16 * L + 2);
    } else {
        if (dead && t == 0) flag_timeout();
        if (b == 0 && t == 0) {
            a.st->pos = pos + a.advance;
            __hip_atomic_store(xb + W_CTRL, E + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    (void)ep_last;
}

// Test hook: words of the hidden-state region tagged with the epoch that the
// next launch's layer-1 wait accepts (the step counter as it stands now),
// holding 2.0 as payload: what a workgroup of a timed-out launch that started
// late would have left behind.
__global__ __launch_bounds__(256) void k_persist_poison(unsigned* xb, int L) {
    const unsigned E = __hip_atomic_load(xb + W_CTRL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned ep = step_epoch(E, L, 0);
    for (int i = threadIdx.x; i < NREP * 2 * D; i += 256)
        __hip_atomic_store(xb + W_HD + i, 0x4000u | (ep << 16), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

typedef void (*PersistKernel)(PArgs);

// fp16 weights leave no registers for the second K/V register set, so their
// rounds run one at a time and keep 4 passes
PersistKernel pick(int kind, int pass5) {
    switch (kind) {
        case MDX_W_F16: return k_persist_step<MDX_W_F16, 4>;
        case MDX_W_I8: return pass5 ? k_persist_step<MDX_W_I8, 5> : k_persist_step<MDX_W_I8, 4>;
        case MDX_W_I4: return pass5 ? k_persist_step<MDX_W_I4, 5> : k_persist_step<MDX_W_I4, 4>;
        default: return nullptr;
    }
}

// 1 when the device can hold k's whole grid co-resident
int persist_fits(PersistKernel k) {
    if (!k) return 0;
    int dev = 0, coop = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop)
        return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(k), NT, 0) !=
        hipSuccess)
        return 0;
    return (long)per_cu * cus >= NB;
}

}  // namespace

extern "C" {

int mdx_persist_trace_events(int n_layers) { return 16 * n_layers + 4; }

int mdx_persist_shape_ok(int d, int nq, int nkv, int hd, int F) {
    return d == D && nq == NQ && nkv == NKV && hd == HD && F == FF;
}

size_t mdx_persist_xbuf_bytes(void) { return (size_t)W_TOTAL * 4; }

int mdx_persist_usable(int kind) {
    for (int pass5 = 0; pass5 < 2; pass5++)
        if (!persist_fits(pick(kind, pass5))) return 0;
    return 1;
}

int mdx_persist_k_passes(int n_pos) {
    // positions per split, then rounds of 64 against rounds of 80; the first
    // two rounds are requested before any is computed, so only a third or
    // later round costs a dependent round trip
    const int per = (n_pos + GRP - 1) / GRP;
    const int r4 = (per + 63) / 64, r5 = (per + 79) / 80;
    return r4 >= 3 && r5 < r4 ? 5 : 4;
}

long long mdx_debug_persist_kv_rows(int max_seq, int k_passes, long long* n_checked) {
    if (max_seq <= 0 || (k_passes != 4 && k_passes != 5)) return -1;
    const int PP = k_passes;
    long long bad = 0, cnt = 0;
    // every position the step can run at, every split, every 16-position
    // row pl of a pass and every round the kernel requests: the first at
    // q0 = 0, then (fp16 layers) q0 = PP, 2 PP, ... one at a time, or (int8
    // and int4 layers) a second set at q0 = PP before the first is computed
    // and each later one while the previous is computed; all of them are the
    // rounds q0 = r * PP with 16 * q0 < n, and the first even when n is 0
    for (int pos = 0; pos < max_seq; pos++)
        for (int s = 0; s < GRP; s++) {
            const KvSplit sp = kv_split(pos, s);
            if (sp.p0 < 0 || (sp.n > 0 && sp.p0 + sp.n > pos + 1)) bad++;
            for (int q0 = 0; q0 == 0 || 16 * q0 < sp.n; q0 += PP) {
                for (int qq = 0; qq < PP; qq++)
                    for (int pl = 0; pl < 16; pl++) {
                        const int row = kv_row(sp, 16 * (q0 + qq) + pl, pos);
                        if (row < 0 || row > pos || row >= max_seq) bad++;
                        cnt++;
                    }
            }
        }
    if (n_checked) *n_checked = cnt;
    return bad;
}

int mdx_persist_debug_poison(void* xbuf, int n_layers, void* stream) {
    if (!xbuf || n_layers <= 0) return -1;
    hipLaunchKernelGGL(k_persist_poison, dim3(1), dim3(256), 0, (hipStream_t)stream,
                       reinterpret_cast<unsigned*>(xbuf), n_layers);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int mdx_launch_persist_step(const mdx_persist_args* p, void* stream) {
    PersistKernel k = pick(p->kind, p->k_passes == 5);
    if (!k || p->n_layers <= 0 || !p->state || !p->xbuf || !p->l0.wqkv) return -1;
    if (p->head && (!p->lm_w || !p->lm_scale || !p->logits || !p->final_norm)) return -1;
    PArgs a;
    a.n_layers = p->n_layers;
    a.vocab = p->vocab;
    a.max_seq = p->max_seq;
    a.rope_style = p->rope_style;
    a.head = p->head;
    a.advance = p->advance;
    a.eps = p->eps;
    a.st = p->state;
    a.l0 = p->l0;
    a.lstride = p->layer_stride;
    a.kvstride = p->kv_stride;
    a.emb_table = p->emb_table;
    a.emb_in = p->emb_in;
    a.cos_t = p->cos_t;
    a.sin_t = p->sin_t;
    a.final_norm = p->final_norm;
    a.lm_w = p->lm_w;
    a.lm_scale = p->lm_scale;
    a.logits = p->logits;
    a.hidden_out = p->hidden_out;
    a.xbuf = reinterpret_cast<unsigned*>(p->xbuf);
    a.out_tokens = p->out_tokens;
    a.trace = p->trace;
    a.trace_stride = p->trace_stride;
    a.spin_limit = p->spin_limit ? p->spin_limit : kSpinLimit;
    a.kv_stream = p->kv_stream;
    a.in_args = p->in_args;
    a.in_pos = p->in_pos;
    a.in_token = p->in_token;
    a.in_mode = p->in_mode;
    a.logits_host = p->logits_host;
    a.res_host = p->res_host;
    a.xbl = reinterpret_cast<unsigned*>(p->xbl);
    if (a.trace && a.trace_stride < 16 * a.n_layers + 4) return -1;
    // host logits: each workgroup's rows are staged in LDS first
    if (a.logits_host && (!a.head || (long long)a.vocab > (long long)NB * kLogitsRows)) return -1;
    // MDX_COOP=1 / MDX_COOP=0 force the launch kind over the caller's choice
    // (MDX_COOP=0 serves tools that do not follow cooperative launches).  The
    // grid fits the device one workgroup per CU and every wait is bounded, so a
    // workgroup that does not become resident ends the step with an error, not
    // a hang.
    static const int force = [] {
        const char* e = getenv("MDX_COOP");
        return e && e[0] == '0' ? 0 : (e && e[0] == '1' ? 1 : -1);
    }();
    const int coop = force >= 0 ? force : (p->cooperative ? 1 : 0);
    if (!coop) {
        hipLaunchKernelGGL(k, dim3(NB), dim3(NT), 0, (hipStream_t)stream, a);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    void* args[] = {&a};
    hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(k), dim3(NB), dim3(NT),
                                              args, 0, (hipStream_t)stream);
    return e == hipSuccess ? 0 : -1;
}

}  // extern "C"
