// Trellis reconstruct: packed tiles -> dense W_q (ic, oc) fp16, row-major, or its transpose
// W_q^T (oc, ic).  Replaces exllamav3_ext.reconstruct as called at orcasaq2/ops.py:56 and
// orcasaq2/__init__.py:57.  The transposed form lets the reconstruct branch's library GEMM
// run y = x W_q as a transposed-B product, the library's faster layout on this part.
// Output-write bound: 2 B/weight out against K/8 B in.
//
// (ic, oc): one wave owns a strip of 8 tiles (tile row ti, tile columns 8g..8g+7): lane =
// 8T + c decodes chunk c of tile T, the decoded 16x128 block is staged in LDS, and the wave
// writes it back as 16-byte stores that cover whole 256-byte row segments.
// (oc, ic): one wave owns 8 tiles down one tile column (tile rows 8g..8g+7, column tn);
// chunk c of tile T holds all 16 inputs of outputs c and c + 8, so each lane stages two
// 32-byte runs per output with 16-byte LDS stores, and the block of 16 output rows x 128
// inputs is written back the same way.
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

constexpr int RC_WAVES = 4;
constexpr int RC_STRIDE = 128 + 8;  // halves per staged row (padding against bank conflicts)

template <int K, int CB>
__global__ __launch_bounds__(64 * RC_WAVES) void reconstruct_kernel(
    uint16_t* __restrict__ W, const uint32_t* __restrict__ trellis, int ic, int oc)
{
    __shared__ uint16_t stage[RC_WAVES][16 * RC_STRIDE];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int tc = oc >> 4;
    const int groups = (tc + 7) >> 3;
    const long task = (long)blockIdx.x * RC_WAVES + wave;
    const bool active = task < (long)(ic >> 4) * groups;
    const int ti = active ? (int)(task / groups) : 0, g = active ? (int)(task % groups) : 0;
    const int T = lane >> 3, c = lane & 7;
    const int tn = g * 8 + T;
    uint16_t* st = stage[wave];

    if (active && tn < tc) {
        const uint32_t* tile = trellis + ((long)ti * tc + tn) * (8 * K);
        uint32_t w[K + 1];
        load_chunk<K>(w, tile, c);
        // positions q0 = 2p and q0 + 1 (p = 0..15): q0 = 8m + i, i in {0, 2, 4, 6} ->
        // rows 2m + {0, 8}[i%4 / 2] and the row below it, column c + 8(i/4)
#define EXL3_RC(P)                                                                         \
    {                                                                                      \
        constexpr int q0 = 2 * (P), m = q0 / 8, i = q0 % 8;                                \
        constexpr int row = 2 * m + ((i & 3) == 0 ? 0 : 8);                                \
        constexpr int col8 = 8 * (i >> 2);                                                 \
        const uint32_t v = chunk_pair<K, CB, q0>(w);                                       \
        st[row * RC_STRIDE + 16 * T + c + col8] = (uint16_t)(v & 0xffffu);                \
        st[(row + 1) * RC_STRIDE + 16 * T + c + col8] = (uint16_t)(v >> 16);              \
    }
        EXL3_RC(0) EXL3_RC(1) EXL3_RC(2) EXL3_RC(3) EXL3_RC(4) EXL3_RC(5) EXL3_RC(6) EXL3_RC(7)
        EXL3_RC(8) EXL3_RC(9) EXL3_RC(10) EXL3_RC(11) EXL3_RC(12) EXL3_RC(13) EXL3_RC(14) EXL3_RC(15)
#undef EXL3_RC
    }
    __syncthreads();

    // 16 rows x 256 bytes: each store instruction covers 4 rows, 16 bytes per lane.
    const int seg = lane & 15;          // 16-byte segment within the row (8 halves)
    const int col0 = g * 128 + seg * 8;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int row = s * 4 + (lane >> 4);
        if (active && col0 < oc) {
            const uint4 v = *reinterpret_cast<const uint4*>(st + row * RC_STRIDE + seg * 8);
            *reinterpret_cast<uint4*>(W + (long)(ti * 16 + row) * oc + col0) = v;
        }
    }
}

template <int K, int CB>
__global__ __launch_bounds__(64 * RC_WAVES) void reconstruct_t_kernel(
    uint16_t* __restrict__ Wt, const uint32_t* __restrict__ trellis, int ic, int oc)
{
    __shared__ uint16_t stage[RC_WAVES][16 * RC_STRIDE];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int tr = ic >> 4, tc = oc >> 4;
    const int groups = (tr + 7) >> 3;
    const long task = (long)blockIdx.x * RC_WAVES + wave;
    const bool active = task < (long)tc * groups;
    // consecutive waves take consecutive tile columns of one band of 8 tile rows
    const int g = active ? (int)(task / tc) : 0, tn = active ? (int)(task % tc) : 0;
    const int T = lane >> 3, c = lane & 7;
    const int ti = g * 8 + T;
    uint16_t* st = stage[wave];

    if (active && ti < tr) {
        const uint32_t* tile = trellis + ((long)ti * tc + tn) * (8 * K);
        uint32_t w[K + 1];
        load_chunk<K>(w, tile, c);
        // positions q0 = 2p and q0 + 1 (p = 0..15), q0 = 8m + i: the pair is inputs
        // (rows) 2m + {0, 8}[i%4 / 2] and the one below it, of output c + 8(i/4) -- word
        // m + 4 (i%4 / 2) of that output's 16-input run
        uint32_t o[2][8];
#define EXL3_RCT(P)                                                                        \
    {                                                                                      \
        constexpr int q0 = 2 * (P), m = q0 / 8, i = q0 % 8;                                \
        o[i >> 2][m + ((i & 3) == 0 ? 0 : 4)] = chunk_pair<K, CB, q0>(w);                  \
    }
        EXL3_RCT(0) EXL3_RCT(1) EXL3_RCT(2) EXL3_RCT(3) EXL3_RCT(4) EXL3_RCT(5) EXL3_RCT(6) EXL3_RCT(7)
        EXL3_RCT(8) EXL3_RCT(9) EXL3_RCT(10) EXL3_RCT(11) EXL3_RCT(12) EXL3_RCT(13) EXL3_RCT(14) EXL3_RCT(15)
#undef EXL3_RCT
        // rows of 136 halves (68 words): the 8 lanes of one tile hit banks 4c .. 4c + 3
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint4* d = reinterpret_cast<uint4*>(st + (c + 8 * h) * RC_STRIDE + 16 * T);
            d[0] = uint4{o[h][0], o[h][1], o[h][2], o[h][3]};
            d[1] = uint4{o[h][4], o[h][5], o[h][6], o[h][7]};
        }
    }
    __syncthreads();

    const int seg = lane & 15;
    const int col0 = g * 128 + seg * 8;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int row = s * 4 + (lane >> 4);
        if (active && col0 < ic) {
            const uint4 v = *reinterpret_cast<const uint4*>(st + row * RC_STRIDE + seg * 8);
            *reinterpret_cast<uint4*>(Wt + (long)(tn * 16 + row) * ic + col0) = v;
        }
    }
}

template <int K, int CB>
static int launch_reconstruct_t(uint16_t* Wt, const uint32_t* trellis, int ic, int oc, hipStream_t stream)
{
    const long tasks = (long)(oc / 16) * ((ic / 16 + 7) / 8);
    const long blocks = (tasks + RC_WAVES - 1) / RC_WAVES;
    hipLaunchKernelGGL((reconstruct_t_kernel<K, CB>), dim3((unsigned)blocks), dim3(64 * RC_WAVES), 0,
                       stream, Wt, trellis, ic, oc);
    return check_launch("exl3_reconstruct_t");
}

template <int K, int CB>
static int launch_reconstruct(uint16_t* W, const uint32_t* trellis, int ic, int oc, hipStream_t stream)
{
    const long tasks = (long)(ic / 16) * ((oc / 16 + 7) / 8);
    const long blocks = (tasks + RC_WAVES - 1) / RC_WAVES;
    hipLaunchKernelGGL((reconstruct_kernel<K, CB>), dim3((unsigned)blocks), dim3(64 * RC_WAVES), 0,
                       stream, W, trellis, ic, oc);
    return check_launch("exl3_reconstruct");
}

int reconstruct_dispatch(uint16_t* W, const uint32_t* trellis, int ic, int oc, int K, int cb, bool transposed,
                         hipStream_t stream)
{
#define EXL3_CASE(KK)                                                                           \
    case KK:                                                                                    \
        if (transposed)                                                                         \
            return cb == CB_MCG ? launch_reconstruct_t<KK, CB_MCG>(W, trellis, ic, oc, stream)  \
                                : launch_reconstruct_t<KK, CB_3INST>(W, trellis, ic, oc, stream); \
        return cb == CB_MCG ? launch_reconstruct<KK, CB_MCG>(W, trellis, ic, oc, stream)        \
                            : launch_reconstruct<KK, CB_3INST>(W, trellis, ic, oc, stream);
    switch (K) {
        EXL3_CASE(1) EXL3_CASE(2) EXL3_CASE(3) EXL3_CASE(4)
        EXL3_CASE(5) EXL3_CASE(6) EXL3_CASE(7) EXL3_CASE(8)
    }
#undef EXL3_CASE
    return set_error(EXL3_ERR_ARG, "%s: K=%d is not in 1..8", transposed ? "exl3_reconstruct_t" : "exl3_reconstruct",
                     K);
}

}  // namespace exl3
