// mdx_gemm_tile.h — the MFMA fragment conventions shared by the batch-prefill
// GEMM kernels (v_mfma_f32_16x16x32_f16, gfx950).
//
// K-block layout: a weight load is 16 bytes per lane = EPL consecutive k of
// one weight row (EPL = 8 fp16, 16 int8, 32 int4), lane group g = lane/16
// takes k [g*EPL, (g+1)*EPL) of the block (KB = 4*EPL k), and MFMA step s of
// the block uses k g*EPL + 8s .. +7; the activations (A fragments) are taken
// with the same k mapping.  The D fragment of a 16x16 tile: lane holds
// column lane%16, rows 4*(lane/16) + i, i < 4.
#pragma once

#include "mdx_common.h"
#include "mdx_device.h"

namespace mdx {

template <int KIND> struct GemmKind;
// NKB K-blocks per round; DEPTH rounds are in flight (a round is requested
// DEPTH-1 rounds ahead of the one being multiplied); WAVES waves per block
// share the K range.  Measured on the M=60 prefill: small rounds three deep
// beat larger rounds two deep (fp16 8 K-blocks -> 1: 1.58 -> 1.43 ms; int8
// 4 -> 1: 1.366 -> 1.331 ms; int4 2 -> 1: 1.206 -> 1.190 ms), and 8 waves
// beat 4 (int8: 1.331 -> 1.227 ms; fp16 1.43 -> 1.31 ms; int4, two rounds
// deep to fit 256 registers: 1.188 -> 1.139 ms).
template <> struct GemmKind<MDX_W_F16> { static constexpr int EPL = 8, NKB = 1, DEPTH = 3, WAVES = 8; };
template <> struct GemmKind<MDX_W_I8> { static constexpr int EPL = 16, NKB = 1, DEPTH = 3, WAVES = 8; };
template <> struct GemmKind<MDX_W_I4> { static constexpr int EPL = 32, NKB = 1, DEPTH = 2, WAVES = 8; };



// 16 weight bytes -> the EPL/8 fp16 B fragments of this lane.
template <int KIND>
__device__ __forceinline__ void widen_b(uint4 v, half8_t* out) {
    if constexpr (KIND == MDX_W_F16) {
        out[0] = __builtin_bit_cast(half8_t, v);
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
        out[0] = __builtin_bit_cast(half8_t, make_uint4(o[0], o[1], o[2], o[3]));
        out[1] = __builtin_bit_cast(half8_t, make_uint4(o[4], o[5], o[6], o[7]));
    } else {
        const uint32_t wd[4] = {v.x ^ 0x88888888u, v.y ^ 0x88888888u, v.z ^ 0x88888888u,
                                v.w ^ 0x88888888u};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t o[4];
#pragma unroll
            for (int q = 0; q < 4; q++) o[q] = h2_bits(i4_pair(wd[i], q));
            out[i] = __builtin_bit_cast(half8_t, make_uint4(o[0], o[1], o[2], o[3]));
        }
    }
}

}  // namespace mdx
