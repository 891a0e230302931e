// Measurement kernels for the batch-1 GEMV's ceilings (libexl3ceiling.so; bench.py
// --workload ceiling).  Not part of the product library or its C ABI: nothing in the op
// path calls them.
//
// The stream kernels walk one shard's trellis exactly as gemv1_kernel<K, CB, true, 1> does
// -- the same units (one tile row of one 128-output column group), the same split into
// G = min(4 CUs, U / 32) contiguous workgroup ranges of 8 waves, the same contiguous wave
// runs and the same D-deep register ring of loads -- and stop short of parts of its work:
//   mode 0  an empty kernel of the same grid (launch and drain alone);
//   mode 1  the loads alone (each word folded into an xor);
//   mode 2  the loads and the three-instruction decode of every position (dot2_raw, the
//           mask folded into an xor accumulator: one v_bitop3 per position, as in the
//           product), no MFMA;
//   mode 3  the loads, the decode and the 16 v_mfma_f32_4x4x4_16b_f16 per unit with the
//           activations read from a constant LDS table (4 ds_read_b128 per unit, as in the
//           product) -- the product's main loop without the activation transform and
//           without the split reduction;
//   mode 4  mode 3 with the unit's products on 8 v_mfma_f32_16x16x32_f16 (group-select A
//           operand, mfma16_group) instead of 16 v_mfma_f32_4x4x4_16b_f16.
// Every accumulator reaches a store that is never taken, so no work is optimised away.
//
// The plain stream (exl3m_plain) reads the same bytes without the GEMV's layout: 16-byte
// pieces at a grid stride, four loads in flight per lane, the same grid of 4 workgroups of
// 8 waves per CU -- what HBM gives a read of this size in its most regular access pattern.
//
// The op kernels time chains of one instruction (8 independent chains per wave, 8 waves
// per SIMD, 4 workgroups of 8 waves per CU) to give the issue cost per wave64 instruction.
#include "../exl3_common.h"

#include <algorithm>

namespace exl3m {

using namespace exl3;

constexpr int NW = 8;

constexpr int depth(int K) { return (24 / (K + 3)) < 2 ? 2 : (24 / (K + 3)) > 6 ? 6 : (24 / (K + 3)); }

template <int K>
__device__ __forceinline__ void ld(uint32_t (&w)[K + 1], const uint32_t* __restrict__ p)
{
    typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    int i = 0;
#pragma unroll
    for (; i + 4 <= K; i += 4) {
        uint4 v;
        __builtin_memcpy(&v, p + i, 16);
        w[i + 1] = v.x; w[i + 2] = v.y; w[i + 3] = v.z; w[i + 4] = v.w;
    }
    if constexpr (K % 4 == 3) {
        u32x3 v;
        __builtin_memcpy(&v, p + i, 12);
        w[i + 1] = v.x; w[i + 2] = v.y; w[i + 3] = v.z;
    } else if constexpr (K % 4 == 2) {
        u32x2 v;
        __builtin_memcpy(&v, p + i, 8);
        w[i + 1] = v.x; w[i + 2] = v.y;
    } else if constexpr (K % 4 == 1) {
        w[i + 1] = p[i];
    }
}

// Position Q's word masked into accumulator Q % 4 with one v_bitop3 ((x & mask) ^ acc, the
// product's masking instruction; four independent chains).
template <int K, int Q>
__device__ __forceinline__ void fold1(const uint32_t (&w)[K + 1], uint32_t (&acc)[4], const Dot2Consts& kc)
{
    asm("v_bitop3_b32 %0, %1, %2, %0 bitop3:0x6a" : "+v"(acc[Q % 4]) : "v"(dot2_raw<K, CB_3INST, Q>(w, kc)), "v"(kc.mask));
}

template <int K, int... Qs>
__device__ __forceinline__ void decode_fold(const uint32_t (&w)[K + 1], uint32_t (&acc)[4], const Dot2Consts& kc,
                                            std::integer_sequence<int, Qs...>)
{
    (fold1<K, Qs>(w, acc, kc), ...);
}

template <int K, int J>
__device__ __forceinline__ void mfma_pair(const uint32_t (&w)[K + 1], const uint32_t (&a16)[16], f32x4 (&acc)[2],
                                          const Dot2Consts& kc)
{
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    constexpr int m = J / 4, p = (J / 2) % 2, h = J % 2;
    constexpr int q0 = 8 * m + 2 * p + 4 * h;
    const u2 bv = {dot2_word<K, CB_3INST, q0>(w, kc), dot2_word<K, CB_3INST, q0 + 1>(w, kc)};
    const u2 av = {a16[2 * m + 8 * p], a16[2 * m + 8 * p + 1]};
    acc[h] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(h4, av), __builtin_bit_cast(h4, bv), acc[h], 0, 0, 0);
}

template <int K, int... Js>
__device__ __forceinline__ void mfma_chunk(const uint32_t (&w)[K + 1], const uint32_t (&a16)[16], f32x4 (&acc)[2],
                                           const Dot2Consts& kc, std::integer_sequence<int, Js...>)
{
    (mfma_pair<K, Js>(w, a16, acc, kc), ...);
}

// The same unit as four groups of two tiles for v_mfma_f32_16x16x32_f16: lane l (column
// l % 16 of tiles 2 (l / 16), 2 (l / 16) + 1) supplies four positions as eight fp16 k-slots
// (each masked word's halves), MFMA (m, h) taking positions 8m + 4h + {0..3}; the A operand
// holds the activations only in rows i with i % 4 == l / 16 (zeros elsewhere), so row j of C
// collects group j alone.
template <int K, int M, int H>
__device__ __forceinline__ void mfma16_group(const uint32_t (&w)[K + 1], const f16x8& a, f32x4 (&acc)[2],
                                             const Dot2Consts& kc)
{
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    constexpr int q = 8 * M + 4 * H;
    const u4 b = {dot2_word<K, CB_3INST, q>(w, kc), dot2_word<K, CB_3INST, q + 1>(w, kc),
                  dot2_word<K, CB_3INST, q + 2>(w, kc), dot2_word<K, CB_3INST, q + 3>(w, kc)};
    acc[H] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(f16x8, b), acc[H], 0, 0, 0);
}

template <int K, int MODE>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(8, 8)))
void stream_kernel(const uint32_t* __restrict__ tr, int ntr, int oc16, int U, uint32_t* sink)
{
    constexpr int D = depth(K);
    __shared__ __attribute__((aligned(16))) uint32_t tab[8 * 32];
    if constexpr (MODE == 0) return;
    const int G = gridDim.x, g = blockIdx.x;
    const int q = U / G, r = U % G;
    const int ub = g * q + min(g, r), L = q + (g < r ? 1 : 0);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int lo = (wave * L) >> 3, n = (((wave + 1) * L) >> 3) - lo;
    const long stride = (long)oc16 * 8 * K;
    // prefetch cursor: column group, tile row, address of the lane's words
    int u0 = ub + lo, cg = u0 / ntr, t = u0 - cg * ntr;
    const uint32_t* p = tr + ((long)t * oc16 + 8 * cg) * 8 * K + lane * K;
    int jpf = 0;
    auto next = [&]() {
        if (jpf + 1 < n) {
            jpf++;
            p += stride;
            if (++t == ntr) {
                t = 0;
                cg++;
                p = tr + (long)8 * cg * 8 * K + lane * K;
            }
        }
    };
    if constexpr (MODE >= 3) {
        // 8 entries of 16 activation words, each followed by 16 zero words (mode 4's zero rows)
        for (int i = threadIdx.x; i < 8 * 32; i += 64 * NW)
            tab[i] = (i & 16) ? 0u : 0x3c003c00u ^ ((i * 2654435761u) & 0x03ff03ffu);
        __syncthreads();
    }
    const uint32_t aoff = ((lane & 15) & 3) == (lane >> 4) ? 0u : 16u;
    struct Slot { uint32_t w[K + 1]; };
    Slot ring[D];
    if (n > 0) {
        ld<K>(ring[0].w, p);
#pragma unroll
        for (int d = 1; d < D; d++) {
            next();
            ld<K>(ring[d].w, p);
        }
    }
    const Dot2Consts kc = dot2_consts();
    uint32_t x = 0, xs[4] = {0, 0, 0, 0};
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    for (int j = 0; j < n; j += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            if (d == 0 || j + d < n) {
                if constexpr (MODE == 1) {
#pragma unroll
                    for (int i = 1; i <= K; i++) x ^= ring[d].w[i];
                } else if constexpr (MODE == 2) {
                    chunk_prev_dpp<K>(ring[d].w, (lane & 7) == 0);
                    decode_fold<K>(ring[d].w, xs, kc, std::make_integer_sequence<int, 32>{});
                } else if constexpr (MODE == 4) {
                    const f16x8* ap = reinterpret_cast<const f16x8*>(tab + ((j + d) & 7) * 32 + aoff);
                    const f16x8 a0 = ap[0], a1 = ap[1], a2 = ap[2], a3 = ap[3];
                    chunk_prev_dpp<K>(ring[d].w, (lane & 7) == 0);
                    mfma16_group<K, 0, 0>(ring[d].w, a0, acc, kc); mfma16_group<K, 0, 1>(ring[d].w, a0, acc, kc);
                    mfma16_group<K, 1, 0>(ring[d].w, a1, acc, kc); mfma16_group<K, 1, 1>(ring[d].w, a1, acc, kc);
                    mfma16_group<K, 2, 0>(ring[d].w, a2, acc, kc); mfma16_group<K, 2, 1>(ring[d].w, a2, acc, kc);
                    mfma16_group<K, 3, 0>(ring[d].w, a3, acc, kc); mfma16_group<K, 3, 1>(ring[d].w, a3, acc, kc);
                } else {
                    const uint4* ap = reinterpret_cast<const uint4*>(tab + ((j + d) & 7) * 32);
                    uint32_t a16[16];
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const uint4 tv = ap[v];
                        a16[4 * v] = tv.x; a16[4 * v + 1] = tv.y; a16[4 * v + 2] = tv.z; a16[4 * v + 3] = tv.w;
                    }
                    chunk_prev_dpp<K>(ring[d].w, (lane & 7) == 0);
                    mfma_chunk<K>(ring[d].w, a16, acc, kc, std::make_integer_sequence<int, 16>{});
                }
            }
            next();
            ld<K>(ring[d].w, p);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) x ^= xs[i];
    if (x == 0x9e3779b9u || acc[0][0] + acc[1][1] == 1234.5f) sink[g * 64 * NW + threadIdx.x] = x;
}

#define EXL3M_R8(X) X(0) X(1) X(2) X(3) X(4) X(5) X(6) X(7)

// Instruction chains: OP selects the instruction; 8 independent chains per wave.
template <int OP>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(8, 8))) void op_kernel(uint32_t* sink, int iters)
{
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t v0 = lane, v1 = lane * 3, v2 = lane * 5, v3 = lane * 7, v4 = lane ^ 9, v5 = lane + 11, v6 = lane * 13,
             v7 = lane + 17;
    uint64_t d0 = lane, d1 = lane, d2 = lane, d3 = lane, d4 = lane, d5 = lane, d6 = lane, d7 = lane;
    const uint32_t c = 0x12345u + lane, m = 0x8fff8fffu;
    f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0, a3 = a0;
    const uint64_t A2 = 0x3c003c013c023c03ull + lane, B2 = 0x3c043c053c063c07ull;
    const u4 A4 = {0x3c003c00u + lane, 0x3c013c01u, 0x3c023c02u, 0x3c033c03u};
    const u4 B4 = {0x3c043c04u, 0x3c053c05u + lane, 0x3c063c06u, 0x3c073c07u};
    const bool mfma_wave = wave & 1;
#define EXL3M_VOP(ID, INS)                                                          \
    if constexpr (OP == ID) {                                                       \
        asm volatile(INS : "+v"(v0) : "v"(c), "v"(m)); asm volatile(INS : "+v"(v1) : "v"(c), "v"(m)); \
        asm volatile(INS : "+v"(v2) : "v"(c), "v"(m)); asm volatile(INS : "+v"(v3) : "v"(c), "v"(m)); \
        asm volatile(INS : "+v"(v4) : "v"(c), "v"(m)); asm volatile(INS : "+v"(v5) : "v"(c), "v"(m)); \
        asm volatile(INS : "+v"(v6) : "v"(c), "v"(m)); asm volatile(INS : "+v"(v7) : "v"(c), "v"(m)); \
    }
#define EXL3M_MAD(i) asm volatile("v_mad_u64_u32 %0, vcc, %1, %2, %0" : "+v"(d##i) : "v"(v##i), "v"(c) : "vcc");
#define EXL3M_MF4(acc) asm volatile("v_mfma_f32_4x4x4_16b_f16 %0, %1, %2, %0" : "+v"(acc) : "v"(A2), "v"(B2));
#define EXL3M_MF16(acc) asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(acc) : "v"(A4), "v"(B4));
#define EXL3M_MUL(i) asm volatile("v_mul_lo_u32 %0, %0, %1" : "+v"(v##i) : "v"(c));
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            EXL3M_VOP(1, "v_add_u32 %0, %0, %1")
            EXL3M_VOP(2, "v_bitop3_b32 %0, %0, %1, %2 bitop3:0x6a")
            EXL3M_VOP(3, "v_lshrrev_b32 %0, 5, %0")
            EXL3M_VOP(4, "v_mul_lo_u32 %0, %0, %1")
            EXL3M_VOP(5, "v_bfe_u32 %0, %0, 5, 16")
            EXL3M_VOP(6, "v_alignbit_b32 %0, %0, %1, 7")
            EXL3M_VOP(7, "v_add_u32_sdwa %0, %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:DWORD")
            EXL3M_VOP(8, "v_perm_b32 %0, %0, %1, %2")
            EXL3M_VOP(9, "v_lshlrev_b32 %0, 5, %0")
            EXL3M_VOP(10, "v_mov_b32_dpp %0, %1 row_ror:1 row_mask:0xf bank_mask:0xf")
            if constexpr (OP == 11) { EXL3M_R8(EXL3M_MAD) }
            if constexpr (OP == 12) { EXL3M_MF4(a0) EXL3M_MF4(a1) EXL3M_MF4(a2) EXL3M_MF4(a3) EXL3M_MF4(a0) EXL3M_MF4(a1) EXL3M_MF4(a2) EXL3M_MF4(a3) }
            if constexpr (OP == 13) { EXL3M_MF16(a0) EXL3M_MF16(a1) EXL3M_MF16(a2) EXL3M_MF16(a3) EXL3M_MF16(a0) EXL3M_MF16(a1) EXL3M_MF16(a2) EXL3M_MF16(a3) }
            if constexpr (OP == 14) {   // odd waves: eight 4x4x4 MFMAs; even waves: eight v_mul_lo_u32
                if (mfma_wave) { EXL3M_MF4(a0) EXL3M_MF4(a1) EXL3M_MF4(a2) EXL3M_MF4(a3) EXL3M_MF4(a0) EXL3M_MF4(a1) EXL3M_MF4(a2) EXL3M_MF4(a3) }
                else { EXL3M_R8(EXL3M_MUL) }
            }
            if constexpr (OP == 15) {   // odd waves: eight 16x16x32 MFMAs; even waves: eight v_mul_lo_u32
                if (mfma_wave) { EXL3M_MF16(a0) EXL3M_MF16(a1) EXL3M_MF16(a2) EXL3M_MF16(a3) EXL3M_MF16(a0) EXL3M_MF16(a1) EXL3M_MF16(a2) EXL3M_MF16(a3) }
                else { EXL3M_R8(EXL3M_MUL) }
            }
        }
    }
#undef EXL3M_VOP
#undef EXL3M_MAD
#undef EXL3M_MF4
#undef EXL3M_MF16
#undef EXL3M_MUL
    const uint32_t s = v0 ^ v1 ^ v2 ^ v3 ^ v4 ^ v5 ^ v6 ^ v7 ^ (uint32_t)(d0 ^ d1 ^ d2 ^ d3 ^ d4 ^ d5 ^ d6 ^ d7);
    const float f = a0[0] + a1[0] + a2[0] + a3[0];
    if (s == 0x9e3779b9u || f == 1234.5f) sink[blockIdx.x * 64 * NW + threadIdx.x] = s;
}

__global__ __launch_bounds__(64 * NW) void plain_kernel(const uint4* __restrict__ p, long n16, uint32_t* sink)
{
    const long tid = (long)blockIdx.x * 64 * NW + threadIdx.x, nt = (long)gridDim.x * 64 * NW;
    uint32_t x = 0;
    long i = tid;
    for (; i + 3 * nt < n16; i += 4 * nt) {
        const uint4 a = p[i], b = p[i + nt], c = p[i + 2 * nt], d = p[i + 3 * nt];
        x ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += nt) {
        const uint4 a = p[i];
        x ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (x == 0x9e3779b9u) sink[tid] = x;
}

static int cus()
{
    int dev = 0, n = 0;
    hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    return n;
}

template <int MODE>
static const void* stream_fn(int K)
{
    switch (K) {
    case 2: return (const void*)&stream_kernel<2, MODE>;
    case 3: return (const void*)&stream_kernel<3, MODE>;
    case 4: return (const void*)&stream_kernel<4, MODE>;
    case 5: return (const void*)&stream_kernel<5, MODE>;
    case 6: return (const void*)&stream_kernel<6, MODE>;
    }
    return nullptr;
}

template <int OP>
static const void* op_fn() { return (const void*)&op_kernel<OP>; }

}  // namespace exl3m

using namespace exl3m;

extern "C" {

// Workgroups of a stream launch for one shard (the product's split): min(4 CUs, U / 32).
int exl3m_stream_workgroups(int ic, int oc)
{
    const long U = (long)(oc / 128) * (ic / 16);
    return (int)std::max<long>(1, std::min<long>(4L * cus(), U / 32));
}

// Bytes the sink must hold for a stream or op launch (one u32 per thread).
long exl3m_sink_bytes(int ic, int oc) { return (long)std::max(exl3m_stream_workgroups(ic, oc), 4 * cus()) * 64 * NW * 4; }

// mode 0..3 as above; K 2..6; ic, oc multiples of 128; returns 0 or a HIP error code.
int exl3m_stream(int mode, const void* trellis, int ic, int oc, int K, void* sink, void* stream)
{
    if (mode < 0 || mode > 4 || K < 2 || K > 6 || ic <= 0 || oc <= 0 || ic % 128 || oc % 128) return -1;
    const int ntr = ic / 16, oc16 = oc / 16, U = (oc / 128) * ntr;
    const int G = exl3m_stream_workgroups(ic, oc);
    if (U / G < NW) return -1;   // every wave walks at least one unit
    const void* fn = mode == 0 ? stream_fn<0>(K) : mode == 1 ? stream_fn<1>(K) : mode == 2 ? stream_fn<2>(K)
                   : mode == 3 ? stream_fn<3>(K) : stream_fn<4>(K);
    void* args[] = {(void*)&trellis, (void*)&ntr, (void*)&oc16, (void*)&U, (void*)&sink};
    hipLaunchKernel(fn, dim3(G), dim3(64 * NW), args, 0, static_cast<hipStream_t>(stream));
    return (int)hipGetLastError();
}

// The plain stream over nbytes (a multiple of 16, 16-byte aligned) at trellis; 4 workgroups per CU.
int exl3m_plain(const void* trellis, long nbytes, void* sink, void* stream)
{
    if (nbytes <= 0 || nbytes % 16 || ((uintptr_t)trellis & 15)) return -1;
    const long n16 = nbytes / 16;
    hipLaunchKernelGGL(plain_kernel, dim3(4 * cus()), dim3(64 * NW), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4*>(trellis), n16, static_cast<uint32_t*>(sink));
    return (int)hipGetLastError();
}

// op 1..15 (see op_kernel); one launch of 4 workgroups per CU running `iters` x 32 instructions per wave.
int exl3m_ops(int op, int iters, void* sink, void* stream)
{
    static const void* fns[16] = {nullptr,      op_fn<1>(),  op_fn<2>(),  op_fn<3>(),  op_fn<4>(),  op_fn<5>(),
                                  op_fn<6>(),   op_fn<7>(),  op_fn<8>(),  op_fn<9>(),  op_fn<10>(), op_fn<11>(),
                                  op_fn<12>(),  op_fn<13>(), op_fn<14>(), op_fn<15>()};
    if (op < 1 || op > 15 || iters < 1) return -1;
    void* args[] = {(void*)&sink, (void*)&iters};
    hipLaunchKernel(fns[op], dim3(4 * cus()), dim3(64 * NW), args, 0, static_cast<hipStream_t>(stream));
    return (int)hipGetLastError();
}

}  // extern "C"
