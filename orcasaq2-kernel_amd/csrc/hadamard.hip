// Row-wise block-128 Walsh-Hadamard with optional input/output scale vectors:
//   out[r, 128b + i] = (sum_j H[i, j] (in[r, 128b + j] * pre[128b + j])) * post[128b + i] * scale
// with H the Sylvester matrix / sqrt(128).  Replaces exllamav3_ext.had_r_128 as called at
// orcasaq2/ops.py:54 (pre = suh) and orcasaq2/ops.py:59 (post = svh, in place); the
// normalisation follows orcasaq2/__init__.py:39.  fp16 in/out, fp32 arithmetic.
//
// One wave per 128-block: lane l holds elements 2l and 2l+1 (one 4-byte load/store),
// the first butterfly stage is in-lane and the other six use cross-lane swizzles.
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

constexpr int HAD_WAVES = 4;

__global__ __launch_bounds__(64 * HAD_WAVES) void had_r_128_kernel(
    const uint32_t* in, uint32_t* out, const uint32_t* __restrict__ pre,  // in == out allowed
    const uint32_t* __restrict__ post, float scale, long blocks, int blocks_per_row)
{
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
                 float scale, long rows, int cols, hipStream_t stream)
{
    const int bpr = cols / 128;
    const long blocks = rows * bpr;
    if (blocks == 0) return EXL3_OK;
    const long grid = (blocks + HAD_WAVES - 1) / HAD_WAVES;
    hipLaunchKernelGGL(had_r_128_kernel, dim3((unsigned)grid), dim3(64 * HAD_WAVES), 0, stream,
                       reinterpret_cast<const uint32_t*>(in), reinterpret_cast<uint32_t*>(out),
                       reinterpret_cast<const uint32_t*>(pre), reinterpret_cast<const uint32_t*>(post),
                       scale, blocks, bpr);
    return check_launch("exl3_had_r_128");
}

}  // namespace exl3
