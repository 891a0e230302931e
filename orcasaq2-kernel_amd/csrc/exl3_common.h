// Shared device code for the EXL3 trellis kernels (gfx950 / CDNA4, wave64).
//
// Trellis format (the contract the CPU oracle states bit for bit):
//   * trellis (ic/16, oc/16, 16K) int16, K = last_dim / 16 (orcasaq2/ops.py:28-34);
//     tile (ti, tn) covers W_q rows 16ti.. (input features) and columns 16tn.. (outputs).
//   * A tile is 8K little-endian u32 words; stream bit p is bit 31 - p%32 of word p/32.
//   * Position t (0..255) decodes the 16-bit state made of stream bits
//     [(t+1)K - 16, (t+1)K) modulo 256K (tail-biting), earliest bit most significant.
//   * Position t = 8J + i sits at tile row 2(J%4) + {0,1,8,9}[i%4], column J/4 + 8(i/4).
//   * 3INST: x = 89226354 s + 64248484; MCG: x = 0xCBAC1FED s (mod 2^32); then
//     x = (x & 0x8FFF8FFF) ^ 0x3B603B60 and the weight is fp16(lo16) + fp16(hi16), one
//     IEEE round-to-nearest-even (both halves lie in [2^-3, 2), so the sum never is
//     subnormal and an fp16 add is exact-then-rounded).
//
// Work unit used by every kernel: a "chunk" = 32 consecutive positions of one tile =
// K u32 words, handled by one lane.  Chunk c (0..7) of a tile holds positions 32c..32c+31,
// which are exactly tile columns c and c+8 over all 16 rows:
//   q = 8m + i (m = 0..3, i = 0..7) -> row 2m + {0,1,8,9}[i%4], column c + 8(i/4).
// So a lane's chunk yields four 8-row MFMA fragments (column half ch = i/4, row half
// rh = (i%4)/2): fragment (ch, rh) element e (0..7) is position
//   q = 8(e/2) + 4ch + 2rh + (e%2), row 8rh + e.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace exl3 {

enum Codebook : int { CB_3INST = 0, CB_MCG = 1, CB_MUL1 = 2 };

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- codebook

// Masked codebook word: two fp16 halves whose sum is the weight.
template <int CB>
__device__ __forceinline__ uint32_t cb_word(uint32_t s)
{
    uint32_t x;
    if constexpr (CB == CB_MCG) {
        x = s * 0xCBAC1FEDu;
    } else {
        // (a*s + b) mod 2^32 with s < 2^16: a = 1361*2^16 + 31858, b = 64248484.
        // t = 31858*s + b fits a 16x16+32 multiply-add; the high half gets 1361*s.
        uint32_t t = (s & 0xffffu) * 31858u + 64248484u;
        x = t + ((s * 1361u) << 16);
    }
    return (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
}

__device__ __forceinline__ _Float16 half_sum(uint32_t x)
{
    _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(x & 0xffffu));
    _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(x >> 16));
    return lo + hi;
}

template <int CB>
__device__ __forceinline__ _Float16 cb_value(uint32_t s)
{
    return half_sum(cb_word<CB>(s));
}

// ---------------------------------------------------------------- stream access

// w[0] = the u32 word preceding the chunk (wrapping within the tile), w[1..K] = the
// chunk's K words.  State of chunk position q (compile-time): the low 16 bits of the
// 32-bit window ending at bit 32 + (q+1)K of the concatenation w[0]:w[1]:...:w[K].
template <int K, int Q>
__device__ __forceinline__ uint32_t chunk_state(const uint32_t (&w)[K + 1])
{
    constexpr int e = 32 + (Q + 1) * K;   // exclusive end bit
    constexpr int wi = (e - 1) >> 5;      // word holding the last bit
    constexpr int r = e & 31;             // bits of w[wi] that are used
    if constexpr (r == 0) {
        return w[wi] & 0xffffu;
    } else {
        return __builtin_amdgcn_alignbit(w[wi - 1], w[wi], 32 - r) & 0xffffu;
    }
}

// Loads a lane's chunk: words K*c .. K*c+K-1 of the tile and the preceding word.
template <int K>
__device__ __forceinline__ void load_chunk(uint32_t (&w)[K + 1], const uint32_t* __restrict__ tile, int c)
{
#pragma unroll
    for (int i = 0; i < K; i++) w[i + 1] = tile[K * c + i];
    const int prev = (K * c + 8 * K - 1) % (8 * K);
    w[0] = tile[prev];
}

// Fragment (ch, rh) of a chunk: 8 fp16 weights, element e = row 8rh + e of column c + 8ch.
template <int K, int CB, int CH, int RH>
__device__ __forceinline__ f16x8 chunk_fragment(const uint32_t (&w)[K + 1])
{
    f16x8 f;
#define EXL3_FE(E) f[E] = cb_value<CB>(chunk_state<K, 8 * ((E) / 2) + 4 * CH + 2 * RH + ((E) % 2)>(w));
    EXL3_FE(0) EXL3_FE(1) EXL3_FE(2) EXL3_FE(3) EXL3_FE(4) EXL3_FE(5) EXL3_FE(6) EXL3_FE(7)
#undef EXL3_FE
    return f;
}

// ---------------------------------------------------------------- wave helpers

// In-wave normalised Walsh-Hadamard of one 128-vector held as v0 = x[2l], v1 = x[2l+1]
// in lane l (Sylvester order: x'[i] = sum_j (-1)^popcount(i&j) x[j] / sqrt(128)).
__device__ __forceinline__ void wave_fwht128(float& v0, float& v1)
{
    const int lane = threadIdx.x & 63;
    float a = v0 + v1, b = v0 - v1;
    v0 = a;
    v1 = b;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        float p0 = __shfl_xor(v0, d, 64);
        float p1 = __shfl_xor(v1, d, 64);
        const bool upper = (lane & d) != 0;
        v0 = upper ? (p0 - v0) : (v0 + p0);
        v1 = upper ? (p1 - v1) : (v1 + p1);
    }
    const float norm = 0.08838834764831845f;  // 1/sqrt(128)
    v0 *= norm;
    v1 *= norm;
}

__device__ __forceinline__ f32x4 mfma16x16x32(const f16x8& a, const f16x8& b, const f32x4& c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

}  // namespace exl3
