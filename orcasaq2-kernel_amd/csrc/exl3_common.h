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

#include <utility>

namespace exl3 {

enum Codebook : int { CB_3INST = 0, CB_MCG = 1, CB_MUL1 = 2 };

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- stream access

// Loads a lane's chunk: w[1..K] = words K*c .. K*c+K-1 of the tile, w[0] = the word before
// them (wrapping within the tile: the trellis is tail-biting).
template <int K>
__device__ __forceinline__ void load_chunk(uint32_t (&w)[K + 1], const uint32_t* __restrict__ tile, int c)
{
#pragma unroll
    for (int i = 0; i < K; i++) w[i + 1] = tile[K * c + i];
    const int prev = (K * c + 8 * K - 1) % (8 * K);
    w[0] = tile[prev];
}

// 32-bit window of the concatenation w[0]:w[1]:...:w[K] (MSB first) ending at bit E.
template <int K, int E>
__device__ __forceinline__ uint32_t window(const uint32_t (&w)[K + 1])
{
    constexpr int wi = (E - 1) >> 5;
    constexpr int r = E & 31;
    if constexpr (r == 0) return w[wi];
    else return __builtin_amdgcn_alignbit(w[wi - 1], w[wi], 32 - r);
}

// Where the 16-bit state of chunk position Q lives: the low half of the window ending at
// bit 32 + (Q+1)K, or -- when K divides 16 -- the high half of the window ending D = 16/K
// positions later, so that each window feeds two positions (Q and Q + D share one).
template <int K, int Q>
struct StateLoc {
    static constexpr bool pairs = (16 % K) == 0;
    static constexpr int D = pairs ? 16 / K : 1;
    static constexpr bool hi = pairs && ((Q / D) % 2 == 0);
    static constexpr int E = 32 + (Q + 1 + (hi ? D : 0)) * K;
};

// ---------------------------------------------------------------- codebook (VALU form)
//
// x = a*s + b (mod 2^32) for a 16-bit state s held in the low or high half of `src`,
// with a = A1*2^16 + A0:  t = A0*s + b  (v_mad_u32_u16, exact 16x16+32), then
// hi16(x) = hi16(t) + A1*s (mod 2^16)  (v_mad_u16 writing the high half of t only).
// Both are full-rate; the masked word is then one v_bitop3_b32 ((x & m) ^ c = 0x6a).
template <int CB, bool HI>
__device__ __forceinline__ uint32_t cb_masked(uint32_t src)
{
    constexpr uint32_t A0 = CB == CB_MCG ? (0xCBAC1FEDu & 0xffffu) : (89226354u & 0xffffu);
    constexpr uint32_t A1 = CB == CB_MCG ? (0xCBAC1FEDu >> 16) : (89226354u >> 16);
    constexpr uint32_t B = CB == CB_MCG ? 0u : 64248484u;
    uint32_t t;
    if constexpr (HI) {
        asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(t) : "v"(src), "s"(A0), "v"(B));
        asm("v_mad_u16 %0, %1, %2, %0 op_sel:[1,0,1,1]" : "+v"(t) : "v"(src), "s"(A1));
    } else {
        asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(t) : "v"(src), "s"(A0), "v"(B));
        asm("v_mad_u16 %0, %1, %2, %0 op_sel:[0,0,1,1]" : "+v"(t) : "v"(src), "s"(A1));
    }
    asm("v_bitop3_b32 %0, %0, %1, %2 bitop3:0x6a" : "+v"(t) : "s"(0x8FFF8FFFu), "v"(0x3B603B60u));
    return t;
}

// Packed fp16 pair (low = weight of xa, high = weight of xb), each the IEEE fp16 sum of
// the two halves of its masked word (SDWA adds writing one half each).
__device__ __forceinline__ uint32_t pack_sum(uint32_t xa, uint32_t xb)
{
    uint32_t r;
    asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
        : "=v"(r) : "v"(xa));
    asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
        : "+v"(r) : "v"(xb));
    return r;
}

// Masked codebook word of chunk position Q.
template <int K, int CB, int Q>
__device__ __forceinline__ uint32_t chunk_word(const uint32_t (&w)[K + 1])
{
    using L = StateLoc<K, Q>;
    return cb_masked<CB, L::hi>(window<K, L::E>(w));
}

// Two adjacent positions Q, Q+1 as a packed fp16 pair.
template <int K, int CB, int Q>
__device__ __forceinline__ uint32_t chunk_pair(const uint32_t (&w)[K + 1])
{
    return pack_sum(chunk_word<K, CB, Q>(w), chunk_word<K, CB, Q + 1>(w));
}

// Four packed pairs (an 8-element MFMA operand) from eight masked words, in one asm block
// that ends with two wait states: the compiler cannot see that the SDWA adds are VALU
// writes, and an MFMA reading a VGPR needs >= 2 wait states after a VALU wrote it.
__device__ __forceinline__ f16x8 pack_fragment(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3,
                                               uint32_t x4, uint32_t x5, uint32_t x6, uint32_t x7)
{
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    uint32_t r0, r1, r2, r3;
#define EXL3_SDWA_LO(D, S) "v_add_f16_sdwa " D ", " S ", " S " dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
#define EXL3_SDWA_HI(D, S) "v_add_f16_sdwa " D ", " S ", " S " dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
    asm(EXL3_SDWA_LO("%0", "%4") EXL3_SDWA_HI("%0", "%5")
        EXL3_SDWA_LO("%1", "%6") EXL3_SDWA_HI("%1", "%7")
        EXL3_SDWA_LO("%2", "%8") EXL3_SDWA_HI("%2", "%9")
        EXL3_SDWA_LO("%3", "%10") EXL3_SDWA_HI("%3", "%11")
        "s_nop 1"
        : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
        : "v"(x0), "v"(x1), "v"(x2), "v"(x3), "v"(x4), "v"(x5), "v"(x6), "v"(x7));
#undef EXL3_SDWA_LO
#undef EXL3_SDWA_HI
    u32x4 r = {r0, r1, r2, r3};
    return __builtin_bit_cast(f16x8, r);
}

// Fragment (ch, rh) of a chunk: 8 fp16 weights, element e = row 8rh + e of column c + 8ch,
// i.e. position q = 8(e/2) + 4ch + 2rh + e%2.
template <int K, int CB, int CH, int RH>
__device__ __forceinline__ f16x8 chunk_fragment(const uint32_t (&w)[K + 1])
{
    constexpr int q = 4 * CH + 2 * RH;
    return pack_fragment(chunk_word<K, CB, q>(w), chunk_word<K, CB, q + 1>(w),
                         chunk_word<K, CB, q + 8>(w), chunk_word<K, CB, q + 9>(w),
                         chunk_word<K, CB, q + 16>(w), chunk_word<K, CB, q + 17>(w),
                         chunk_word<K, CB, q + 24>(w), chunk_word<K, CB, q + 25>(w));
}

// ---------------------------------------------------------------- codebook (MFMA half-pair form)
//
// The fused GEMV/GEMM never form the fp16 weight: a masked codebook word holds two fp16
// halves whose sum is the weight, and both halves go into the MFMA as two k-slots against
// the same activation, so the sum is formed exactly inside the fp32 accumulation.  Per
// weight this is a clean 16-bit state (one shift or mask), v_mul_lo_u32, an add and one
// v_bitop3_b32 -- all compiler-visible, with the two constants of the bitop3 held in
// VGPRs (on gfx950 a VALU op that reads an SGPR issues at about half the rate of the same
// op on VGPRs/literals).

struct CbConsts {
    uint32_t mask, flip;  // 0x8FFF8FFF, 0x3B603B60 pinned in VGPRs
};

__device__ __forceinline__ CbConsts cb_consts()
{
    CbConsts k;
    asm volatile("v_mov_b32 %0, 0x8fff8fff" : "=v"(k.mask));
    asm volatile("v_mov_b32 %0, 0x3b603b60" : "=v"(k.flip));
    return k;
}

template <int CB>
__device__ __forceinline__ uint32_t cb_masked_clean(uint32_t s, const CbConsts& k)
{
    uint32_t x = CB == CB_MCG ? s * 0xCBAC1FEDu : s * 89226354u + 64248484u;
    return (x & k.mask) ^ k.flip;
}

// Clean 16-bit state of chunk position Q (high half of a shared window when K | 16).
template <int K, int Q>
__device__ __forceinline__ uint32_t chunk_state_clean(const uint32_t (&w)[K + 1])
{
    using L = StateLoc<K, Q>;
    const uint32_t win = window<K, L::E>(w);
    return L::hi ? (win >> 16) : (win & 0xffffu);
}

template <int K, int CB, int Q>
__device__ __forceinline__ uint32_t chunk_hword(const uint32_t (&w)[K + 1], const CbConsts& k)
{
    return cb_masked_clean<CB>(chunk_state_clean<K, Q>(w), k);
}

// Half-pair fragment (ch, m): positions q = 8m + 4ch + {0,1,2,3} -- rows 2m, 2m+1, 2m+8,
// 2m+9 of column c + 8ch -- as 8 fp16 k-slots (lo, hi of each masked word).  The matching
// activation fragment is x(2m), x(2m), x(2m+1), x(2m+1), x(2m+8), x(2m+8), x(2m+9), x(2m+9).
template <int K, int CB, int CH, int M>
__device__ __forceinline__ f16x8 chunk_hfragment(const uint32_t (&w)[K + 1], const CbConsts& k)
{
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    constexpr int q = 8 * M + 4 * CH;
    u32x4 r = {chunk_hword<K, CB, q>(w, k), chunk_hword<K, CB, q + 1>(w, k),
               chunk_hword<K, CB, q + 2>(w, k), chunk_hword<K, CB, q + 3>(w, k)};
    return __builtin_bit_cast(f16x8, r);
}

// ---------------------------------------------------------------- codebook (batch-1 dot2 form)
//
// Three VALU ops per position, whatever K is:
//  * a state on a 16-bit boundary of a word (the low or high half): 3INST in offset form --
//    a = 89226354 and b = 64248484 are both even, so with C = (b/2) * (a/2)^-1 mod 2^31 =
//    0x68b437e2, a*s + b = a*(s + C) (mod 2^32) for every 16-bit state s; one SDWA add takes
//    the half out and adds C, one v_mul_lo_u32 finishes x.  MCG (b = 0): a shift or mask,
//    then the multiply.
//  * any other state: one v_bfe_u32 takes the clean 16-bit field (out of the word, or out of
//    the 32 bits centred on a word boundary when it straddles one -- one v_alignbit per
//    boundary, shared by every state across it), and one v_mad_u64_u32 forms a*s + b (its
//    low half; measured on MI355X at the rate of v_mul_lo_u32).
// Then one v_bitop3_b32 masks the word.
constexpr uint32_t CB3_OFFSET = 0x68b437e2u;
constexpr uint32_t CB3_MUL = 89226354u;
constexpr uint32_t CB3_ADD = 64248484u;
constexpr uint32_t CBMCG_MUL = 0xCBAC1FEDu;

// Where chunk position Q's 16-bit state is taken from.  E = stream end bit (exclusive) of
// the state inside w[0]:w[1]:..:w[K] (MSB first), word wi = (E-1)/32, r = E%32:
//   0: low half of w[wi] (r = 0)            1: high half of w[wi] (r = 16)
//   2: bits [32 - r, 48 - r) of w[wi] (r > 16: inside the word)
//   3: bits [16 - r, 32 - r) of W16, the 32 bits centred on the boundary before w[wi]
//      (0 < r < 16: the state straddles that boundary)
template <int K, int Q>
struct StatePlan {
    static constexpr int E = 32 + (Q + 1) * K;
    static constexpr int wi = (E - 1) >> 5;
    static constexpr int r = E & 31;
    static constexpr int kind = r == 0 ? 0 : r == 16 ? 1 : r > 16 ? 2 : 3;
};

// Clean 16-bit state of a kind-2 or kind-3 position (one v_bfe_u32).
template <int K, int Q>
__device__ __forceinline__ uint32_t state_field(const uint32_t (&w)[K + 1])
{
    using P = StatePlan<K, Q>;
    static_assert(P::kind >= 2, "aligned states are read as halves");
    if constexpr (P::kind == 2) return (w[P::wi] >> (32 - P::r)) & 0xffffu;
    else return (window<K, 32 * P::wi + 16>(w) >> (16 - P::r)) & 0xffffu;
}

__device__ __forceinline__ uint32_t sdwa_add_lo(uint32_t v, uint32_t c)
{
    uint32_t d;
    asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:DWORD"
        : "=v"(d) : "v"(v), "v"(c));
    return d;
}

__device__ __forceinline__ uint32_t sdwa_add_hi(uint32_t v, uint32_t c)
{
    uint32_t d;
    asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:DWORD"
        : "=v"(d) : "v"(v), "v"(c));
    return d;
}

// Low half of s * m + b (one v_mad_u64_u32; the carry-out goes to vcc, declared clobbered).
__device__ __forceinline__ uint32_t mad_lo(uint32_t s, uint32_t m, uint64_t b)
{
    uint64_t d;
    asm("v_mad_u64_u32 %0, vcc, %1, %2, %3" : "=v"(d) : "v"(s), "v"(m), "s"(b) : "vcc");
    return (uint32_t)d;
}

struct Dot2Consts {
    uint32_t mask, flip, off, mul;   // 0x8FFF8FFF, 0x3B603B60, CB3_OFFSET, CB3_MUL pinned in VGPRs
};

__device__ __forceinline__ Dot2Consts dot2_consts()
{
    Dot2Consts k;
    asm volatile("v_mov_b32 %0, 0x8fff8fff" : "=v"(k.mask));
    asm volatile("v_mov_b32 %0, 0x3b603b60" : "=v"(k.flip));
    asm volatile("v_mov_b32 %0, 0x68b437e2" : "=v"(k.off));
    asm volatile("v_mov_b32 %0, %1" : "=v"(k.mul) : "i"(CB3_MUL));
    return k;
}

// Codebook word x = a*s + b (mod 2^32) of chunk position Q, before the mask.
template <int K, int CB, int Q>
__device__ __forceinline__ uint32_t dot2_raw(const uint32_t (&w)[K + 1], const Dot2Consts& k)
{
    using P = StatePlan<K, Q>;
    if constexpr (P::kind <= 1) {
        const uint32_t src = w[P::wi];
        if constexpr (CB == CB_MCG) return (P::kind == 1 ? (src >> 16) : (src & 0xffffu)) * CBMCG_MUL;
        else return (P::kind == 1 ? sdwa_add_hi(src, k.off) : sdwa_add_lo(src, k.off)) * CB3_MUL;
    } else {
        const uint32_t s = state_field<K, Q>(w);
        return CB == CB_MCG ? s * CBMCG_MUL : mad_lo(s, k.mul, CB3_ADD);
    }
}

// Masked codebook word of chunk position Q.
template <int K, int CB, int Q>
__device__ __forceinline__ uint32_t dot2_word(const uint32_t (&w)[K + 1], const Dot2Consts& k)
{
    return (dot2_raw<K, CB, Q>(w, k) & k.mask) ^ k.flip;
}

__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c)
{
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
}

// One tile row's 16 activations, fp16(H128(x * suh)) rows 16a .. 16a+15 of its 128-input
// block, from the block's inputs spread as lane l = x[2l], x[2l+1] (and suh alike).  In
// Sylvester order H128 = H8 (x) H16: row 16a + b, input 16c + d has sign
// H8[a][c] H16[b][d], so the 16 outputs are H16 of the eight inputs rows summed with the
// signs H8[a][c] (c = lane / 8) -- a cross-lane sum over lanes 8 apart, then a 16-point
// butterfly over d = 2(lane % 8) + k.  The result: lane l (in every 16-lane row) holds
// fp16 (v, v) of rows 2(l % 8) (d0) and 2(l % 8) + 1 (d1).
// sign_factor(a, lane) = H8[a][lane / 8] / sqrt(128): the per-lane factor for tile row a.
__device__ __forceinline__ float tile_row_factor(int a, int lane)
{
    return (__builtin_popcount(a & (lane >> 3)) & 1) ? -0.08838834764831845f : 0.08838834764831845f;
}

__device__ __forceinline__ void tile_row_act(uint32_t xw, uint32_t sw, float f, int lane, uint32_t& d0, uint32_t& d1)
{
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    const h2v xh = __builtin_bit_cast(h2v, xw), sh = __builtin_bit_cast(h2v, sw);
    float u0 = (float)xh.x * (float)sh.x * f, u1 = (float)xh.y * (float)sh.y * f;
    u0 += __shfl_xor(u0, 8, 64);
    u1 += __shfl_xor(u1, 8, 64);
    u0 += __shfl_xor(u0, 16, 64);
    u1 += __shfl_xor(u1, 16, 64);
    u0 += __shfl_xor(u0, 32, 64);
    u1 += __shfl_xor(u1, 32, 64);
    float t0 = u0 + u1, t1 = u0 - u1;
#pragma unroll
    for (int bit = 1; bit < 8; bit <<= 1) {
        const float p0 = __shfl_xor(t0, bit, 64), p1 = __shfl_xor(t1, bit, 64);
        const float sg = (lane & bit) ? -1.f : 1.f;
        t0 = p0 + sg * t0;
        t1 = p1 + sg * t1;
    }
    const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16)t0), h1 = __builtin_bit_cast(uint16_t, (_Float16)t1);
    d0 = h0 | (h0 << 16);
    d1 = h1 | (h1 << 16);
}

// One lane's chunk (32 positions) against one tile row of activations (tile_row_act's
// layout): position q = 8m + i sits in tile row r = 2m + {0, 1, 8, 9}[i % 4], whose
// activation DPP broadcasts (row_newbcast) from lane r / 2 of d_{r % 2} straight into
// v_dot2c: both fp16 halves of the masked word are multiplied by the activation and
// summed in fp32, so the weight's fp16 half-sum is never rounded.  acc[2*(i/4) + (m&1)]
// collects column c + 8*(i/4) of the lane's tile.
template <int Q>
struct Dot2Pos {
    static constexpr int m = Q / 8, i = Q % 8;
    static constexpr int slot = 2 * (i / 4) + (m & 1);
    static constexpr int r = 2 * m + ((i & 3) == 0 ? 0 : (i & 3) == 1 ? 1 : (i & 3) == 2 ? 8 : 9);
};

// Positions 4G .. 4G+3 share m and column half (slot); their rows 2m + {0,1,8,9} read lanes
// m, m, m+4, m+4 of d0, d1, d0, d1.  DPP reads of a VGPR need two wait states after a VALU
// write of it and the compiler does not track hazards inside inline asm, so each block of
// four starts with s_nop 1.
template <int K, int CB, int G>
__device__ __forceinline__ void dot2_quad(const uint32_t (&w)[K + 1], uint32_t d0, uint32_t d1, float (&acc)[4],
                                          const Dot2Consts& k)
{
    using P = Dot2Pos<4 * G>;
    static_assert(Dot2Pos<4 * G + 3>::slot == P::slot, "a quad shares one accumulator");
    const uint32_t q0 = dot2_word<K, CB, 4 * G>(w, k), q1 = dot2_word<K, CB, 4 * G + 1>(w, k);
    const uint32_t q2 = dot2_word<K, CB, 4 * G + 2>(w, k), q3 = dot2_word<K, CB, 4 * G + 3>(w, k);
    asm("s_nop 1\n\t"
        "v_dot2c_f32_f16_dpp %0, %1, %3 row_newbcast:%7 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %0, %2, %4 row_newbcast:%7 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %0, %1, %5 row_newbcast:%8 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot2c_f32_f16_dpp %0, %2, %6 row_newbcast:%8 row_mask:0xf bank_mask:0xf"
        : "+v"(acc[P::slot])
        : "v"(d0), "v"(d1), "v"(q0), "v"(q1), "v"(q2), "v"(q3), "i"(P::m), "i"(P::m + 4));
}

template <int K, int CB, int... Gs>
__device__ __forceinline__ void dot2_chunk_seq(const uint32_t (&w)[K + 1], uint32_t d0, uint32_t d1, float (&acc)[4],
                                               const Dot2Consts& k, std::integer_sequence<int, Gs...>)
{
    (dot2_quad<K, CB, Gs>(w, d0, d1, acc, k), ...);
}

// One lane's chunk (32 positions) against one tile row of activations (tile_row_act's
// layout): position q = 8m + i sits in tile row r = 2m + {0, 1, 8, 9}[i % 4], whose
// activation DPP broadcasts (row_newbcast) from lane r / 2 of d_{r % 2} straight into
// v_dot2c: both fp16 halves of the masked word are multiplied by the activation and
// summed in fp32, so the weight's fp16 half-sum is never rounded.  acc[2*(i/4) + (m&1)]
// collects column c + 8*(i/4) of the lane's tile.
template <int K, int CB>
__device__ __forceinline__ void dot2_chunk(const uint32_t (&w)[K + 1], uint32_t d0, uint32_t d1, float (&acc)[4],
                                           const Dot2Consts& k)
{
    dot2_chunk_seq<K, CB>(w, d0, d1, acc, k, std::make_integer_sequence<int, 8>{});
}

// w[0] of a chunk -- the tile's word before the lane's chunk (tail-biting: the tile's last
// word for the tile's first chunk) -- is the last word w[K] of the previous chunk of the
// same tile, held by the previous lane when a tile's 8 chunks sit on 8 consecutive lanes
// (aligned to 8): a rotate by one inside each 8-lane group, made of two 16-lane-row
// rotates (DPP row_ror:1 serves lanes 1..7 of a group, row_ror:9 lane 0).
template <int K>
__device__ __forceinline__ void chunk_prev_dpp(uint32_t (&w)[K + 1], bool first_lane)
{
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w[K], 0x121, 0xf, 0xf, false);
    const uint32_t r9 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w[K], 0x129, 0xf, 0xf, false);
    w[0] = first_lane ? r9 : r1;
}

// ---------------------------------------------------------------- wave helpers

// In-wave normalised Walsh-Hadamard of one 128-vector held as v0 = x[2l], v1 = x[2l+1]
// in lane l (Sylvester order: x'[i] = sum_j (-1)^popcount(i&j) x[j] / sqrt(128)).
// Butterfly partner: lane ^ d (d <= 16 by ds_swizzle's xor mode within 32-lane halves, no
// address arithmetic; d = 32 by ds_bpermute).
template <int D>
__device__ __forceinline__ float fwht_partner(float v)
{
    if constexpr (D < 32)
        return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x1f | (D << 10)));
    else
        return __shfl_xor(v, D, 64);
}

// Per-lane butterfly signs of the six cross-lane rounds (round i pairs lane with lane ^ 2^i):
// +1 in the lower lane of a pair, -1 in the upper.  Two VALU instructions each.
struct FwhtSigns {
    float s[6];
};

__device__ __forceinline__ FwhtSigns fwht_signs(int lane)
{
    FwhtSigns f;
#pragma unroll
    for (int i = 0; i < 6; i++)
        f.s[i] = __builtin_bit_cast(float, 0x3f800000u | (((uint32_t)lane << (31 - i)) & 0x80000000u));
    return f;
}

template <int D>
__device__ __forceinline__ void fwht_round(float& v0, float& v1, float sg)
{
    // lower lane: v + partner, upper lane: partner - v -- one fma with a +-1 factor each
    // (the same single rounding as the add or the subtraction)
    const float p0 = fwht_partner<D>(v0), p1 = fwht_partner<D>(v1);
    v0 = __builtin_fmaf(sg, v0, p0);
    v1 = __builtin_fmaf(sg, v1, p1);
}

// With the signs computed once by the caller: for loops of many transforms whose sign
// registers are dead before any long loop that follows.
__device__ __forceinline__ void wave_fwht128(float& v0, float& v1, const FwhtSigns& f)
{
    float a = v0 + v1, b = v0 - v1;
    v0 = a;
    v1 = b;
    fwht_round<1>(v0, v1, f.s[0]);
    fwht_round<2>(v0, v1, f.s[1]);
    fwht_round<4>(v0, v1, f.s[2]);
    fwht_round<8>(v0, v1, f.s[3]);
    fwht_round<16>(v0, v1, f.s[4]);
    fwht_round<32>(v0, v1, f.s[5]);
    const float norm = 0.08838834764831845f;  // 1/sqrt(128)
    v0 *= norm;
    v1 *= norm;
}

__device__ __forceinline__ void wave_fwht128(float& v0, float& v1)
{
    // The empty asm keeps the per-lane signs from being hoisted out of the caller's loops
    // (six more live registers across a persistent kernel's main loop).
    int lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));
    wave_fwht128(v0, v1, fwht_signs(lane));
}

// N independent transforms round by round: each round's 2N lane exchanges are in flight
// together, where N calls of wave_fwht128 one after another wait out N chains of six
// exchange round trips.
template <int N>
__device__ __forceinline__ void wave_fwht128_n(float (&v0)[N], float (&v1)[N], const FwhtSigns& f)
{
#pragma unroll
    for (int r = 0; r < N; r++) {
        const float a = v0[r] + v1[r], b = v0[r] - v1[r];
        v0[r] = a;
        v1[r] = b;
    }
#pragma unroll
    for (int r = 0; r < N; r++) fwht_round<1>(v0[r], v1[r], f.s[0]);
#pragma unroll
    for (int r = 0; r < N; r++) fwht_round<2>(v0[r], v1[r], f.s[1]);
#pragma unroll
    for (int r = 0; r < N; r++) fwht_round<4>(v0[r], v1[r], f.s[2]);
#pragma unroll
    for (int r = 0; r < N; r++) fwht_round<8>(v0[r], v1[r], f.s[3]);
#pragma unroll
    for (int r = 0; r < N; r++) fwht_round<16>(v0[r], v1[r], f.s[4]);
#pragma unroll
    for (int r = 0; r < N; r++) fwht_round<32>(v0[r], v1[r], f.s[5]);
    const float norm = 0.08838834764831845f;  // 1/sqrt(128)
#pragma unroll
    for (int r = 0; r < N; r++) {
        v0[r] *= norm;
        v1[r] *= norm;
    }
}

__device__ __forceinline__ f32x4 mfma16x16x32(const f16x8& a, const f16x8& b, const f32x4& c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

}  // namespace exl3
