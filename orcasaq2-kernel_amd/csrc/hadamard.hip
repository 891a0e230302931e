// Row-wise block-128 Walsh-Hadamard with optional input/output scale vectors:
//   out[r, 128b + i] = (sum_j H[i, j] (in[r, 128b + j] * pre[128b + j])) * post[128b + i] * scale
// with H the Sylvester matrix / sqrt(128).  Replaces exllamav3_ext.had_r_128 as called at
// orcasaq2/ops.py:54 (pre = suh) and orcasaq2/ops.py:59 (post = svh, in place); the
// normalisation follows orcasaq2/__init__.py:39.  fp16 in/out, fp32 arithmetic.
//
// 16-byte-aligned pointers (the usual case): sixteen lanes per 128-block, four blocks per wave: lane l of a block holds elements
// 8(l % 16) .. 8(l % 16) + 7 (one 16-byte load and store).  Index bits 0..2 of the
// transform are inside a lane (three in-register butterfly stages), bits 3..6 are lane
// bits 0..3 (DPP exchanges inside each 16-lane row: quad_perm for 1 and 2, two banked
// row shifts for 4, row_ror:8 for 8).
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

constexpr int HAD_WAVES = 4;

// v from lane l ^ 4 within each 16-lane row: banks 0 and 2 (lane bit 2 clear) read lane l + 4
// (row_shl:4), banks 1 and 3 read lane l - 4 (row_shr:4).
__device__ __forceinline__ float had_xor4(float v)
{
    const int x = __builtin_bit_cast(int, v);
    int t = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xf, 0x5, false);
    t = __builtin_amdgcn_update_dpp(t, x, 0x114, 0xf, 0xa, false);
    return __builtin_bit_cast(float, t);
}

template <int D>
__device__ __forceinline__ float had_xor(float v)
{
    const int x = __builtin_bit_cast(int, v);
    if constexpr (D == 1) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
    else if constexpr (D == 2) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xf, 0xf, false));  // quad_perm [2,3,0,1]
    else if constexpr (D == 4) return had_xor4(v);
    else return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x128, 0xf, 0xf, false));  // row_ror:8
}

__device__ __forceinline__ void had_unpack(const uint4& q, float (&v)[8])
{
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xffffu));
        v[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
    }
}

template <int D>
__device__ __forceinline__ void had_lane_stage(float (&v)[8], int lane)
{
    const float sg = (lane & D) ? -1.f : 1.f;
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = __builtin_fmaf(v[i], sg, had_xor<D>(v[i]));
}

// Words zero[0 .. nzero) to 0 by workgroup 0 (before any of its lanes leaves).
__device__ __forceinline__ void had_zero(uint32_t* zero, int nzero)
{
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < nzero; i += blockDim.x) zero[i] = 0u;
}

__global__ __launch_bounds__(64 * HAD_WAVES) void had_r_128_kernel(
    const uint4* in, uint4* out, const uint4* __restrict__ pre,  // in == out allowed
    const uint4* __restrict__ post, float scale, long blocks, int blocks_per_row, uint32_t* zero, int nzero)
{
    had_zero(zero, nzero);
    const long blk = ((long)blockIdx.x * HAD_WAVES + (threadIdx.x >> 6)) * 4 + ((threadIdx.x >> 4) & 3);
    if (blk >= blocks) return;  // no barriers or cross-row exchanges leave a 16-lane row
    const int lane = threadIdx.x & 15;
    const int col_blk = (int)(blk % blocks_per_row);
    float v[8];
    had_unpack(in[blk * 16 + lane], v);
    if (pre) {
        float p[8];
        had_unpack(pre[col_blk * 16 + lane], p);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] *= p[i];
    }
#pragma unroll
    for (int d = 1; d < 8; d <<= 1)
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (!(i & d)) {
                const float a = v[i], b = v[i + d];
                v[i] = a + b;
                v[i + d] = a - b;
            }
    had_lane_stage<1>(v, lane);
    had_lane_stage<2>(v, lane);
    had_lane_stage<4>(v, lane);
    had_lane_stage<8>(v, lane);
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; i++) f[i] = 0.08838834764831845f * scale;   // 1/sqrt(128)
    if (post) {
        float p[8];
        had_unpack(post[col_blk * 16 + lane], p);
#pragma unroll
        for (int i = 0; i < 8; i++) f[i] *= p[i];
    }
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint16_t h0 = __builtin_bit_cast(uint16_t, (_Float16)(v[2 * i] * f[2 * i]));
        const uint16_t h1 = __builtin_bit_cast(uint16_t, (_Float16)(v[2 * i + 1] * f[2 * i + 1]));
        o[i] = (uint32_t)h0 | ((uint32_t)h1 << 16);
    }
    out[blk * 16 + lane] = uint4{o[0], o[1], o[2], o[3]};
}

// Pointers only 4-byte aligned: one wave per 128-block, lane l holds elements 2l, 2l + 1.
__global__ __launch_bounds__(64 * HAD_WAVES) void had_r_128_narrow_kernel(
    const uint32_t* in, uint32_t* out, const uint32_t* __restrict__ pre,  // in == out allowed
    const uint32_t* __restrict__ post, float scale, long blocks, int blocks_per_row, uint32_t* zero, int nzero)
{
    had_zero(zero, nzero);
    const long blk = (long)blockIdx.x * HAD_WAVES + (threadIdx.x >> 6);
    if (blk >= blocks) return;  // no barriers in this kernel
    const int lane = threadIdx.x & 63;
    const int col_blk = (int)(blk % blocks_per_row);
    const uint32_t v = in[blk * 64 + lane];
    float v0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
    float v1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
    if (pre) {
        const uint32_t p = pre[col_blk * 64 + lane];
        v0 *= (float)__builtin_bit_cast(_Float16, (uint16_t)(p & 0xffffu));
        v1 *= (float)__builtin_bit_cast(_Float16, (uint16_t)(p >> 16));
    }
    wave_fwht128(v0, v1);
    if (post) {
        const uint32_t p = post[col_blk * 64 + lane];
        v0 *= (float)__builtin_bit_cast(_Float16, (uint16_t)(p & 0xffffu));
        v1 *= (float)__builtin_bit_cast(_Float16, (uint16_t)(p >> 16));
    }
    v0 *= scale;
    v1 *= scale;
    const uint16_t h0 = __builtin_bit_cast(uint16_t, (_Float16)v0);
    const uint16_t h1 = __builtin_bit_cast(uint16_t, (_Float16)v1);
    out[blk * 64 + lane] = (uint32_t)h0 | ((uint32_t)h1 << 16);
}

int had_dispatch(const uint16_t* in, uint16_t* out, const uint16_t* pre, const uint16_t* post,
                 float scale, long rows, int cols, hipStream_t stream, uint32_t* zero, int nzero)
{
    const int bpr = cols / 128;
    const long blocks = rows * bpr;
    if (blocks == 0 && nzero == 0) return EXL3_OK;   // with words to clear: one workgroup, no blocks
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (!a16(in) || !a16(out) || (pre && !a16(pre)) || (post && !a16(post))) {
        const long grid = std::max<long>(1, (blocks + HAD_WAVES - 1) / HAD_WAVES);
        hipLaunchKernelGGL(had_r_128_narrow_kernel, dim3((unsigned)grid), dim3(64 * HAD_WAVES), 0, stream,
                           reinterpret_cast<const uint32_t*>(in), reinterpret_cast<uint32_t*>(out),
                           reinterpret_cast<const uint32_t*>(pre), reinterpret_cast<const uint32_t*>(post),
                           scale, blocks, bpr, zero, nzero);
        return check_launch("exl3_had_r_128");
    }
    const long grid = std::max<long>(1, (blocks + 4 * HAD_WAVES - 1) / (4 * HAD_WAVES));
    hipLaunchKernelGGL(had_r_128_kernel, dim3((unsigned)grid), dim3(64 * HAD_WAVES), 0, stream,
                       reinterpret_cast<const uint4*>(in), reinterpret_cast<uint4*>(out),
                       reinterpret_cast<const uint4*>(pre), reinterpret_cast<const uint4*>(post),
                       scale, blocks, bpr, zero, nzero);
    return check_launch("exl3_had_r_128");
}

}  // namespace exl3
