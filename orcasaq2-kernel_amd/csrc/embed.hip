// int8 embedding gather with a per-row scale applied to the gathered rows:
//   out[n, :] = dtype(table[ids[n], :]) * scales[ids[n]]
// as in orcasaq2/heads.py:61-67 (the table stays int8; only the gathered rows are scaled).
// The product of an int8 and a 16/32-bit float is exact in fp32, so one rounding to the
// scale dtype reproduces torch's `q[ids].to(s.dtype) * s[ids]` bit for bit.
// Ids outside [0, vocab) produce zero rows (no out-of-bounds read).
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

enum ScaleType : int { ST_F16 = 0, ST_BF16 = 1, ST_F32 = 2 };

__device__ __forceinline__ float load_scale(const void* s, long i, int st)
{
    if (st == ST_F32) return static_cast<const float*>(s)[i];
    const uint16_t b = static_cast<const uint16_t*>(s)[i];
    if (st == ST_BF16) return __builtin_bit_cast(float, (uint32_t)b << 16);
    return (float)__builtin_bit_cast(_Float16, b);
}

__device__ __forceinline__ uint16_t round_bf16(float f)
{
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);                                           // nearest even
    return (uint16_t)(u >> 16);
}

// One workgroup per id.  Each lane loads up to EMB_BATCH words (4 int8 each) of the row at
// once and only then scales and stores them, so a row of a few thousand bytes costs one
// memory round trip (one wave looping over a 5120-byte row waited on 20 dependent loads:
// 13.5 us per batch-1 gather).
constexpr int EMB_THREADS = 256;
constexpr int EMB_BATCH = 8;

__global__ __launch_bounds__(EMB_THREADS) void embed_int8_kernel(const int8_t* __restrict__ table, const void* __restrict__ scales,
                                                                 int st, const int64_t* __restrict__ ids, void* __restrict__ out,
                                                                 int vocab, int dim)
{
    const long n = blockIdx.x;
    const int64_t id = ids[n];
    const bool ok = id >= 0 && id < vocab;
    const float sc = ok ? load_scale(scales, id, st) : 0.f;
    const uint32_t* row = reinterpret_cast<const uint32_t*>(table + (ok ? id : 0) * (long)dim);
    const int nw = dim / 4;
    for (int q0 = 0; q0 < nw; q0 += EMB_THREADS * EMB_BATCH) {
        uint32_t v[EMB_BATCH];
#pragma unroll
        for (int b = 0; b < EMB_BATCH; b++) {
            const int q = q0 + threadIdx.x + b * EMB_THREADS;
            v[b] = ok && q < nw ? row[q] : 0u;
        }
#pragma unroll
        for (int b = 0; b < EMB_BATCH; b++) {
            const int q = q0 + threadIdx.x + b * EMB_THREADS;
            if (q >= nw) break;
            float f[4];
#pragma unroll
            for (int i = 0; i < 4; i++) f[i] = (float)(int8_t)(v[b] >> (8 * i)) * sc;
            if (st == ST_F32) {
                float4 o = {f[0], f[1], f[2], f[3]};
                reinterpret_cast<float4*>(static_cast<float*>(out) + n * (long)dim)[q] = o;
            } else {
                uint16_t hb[4];
#pragma unroll
                for (int i = 0; i < 4; i++)
                    hb[i] = st == ST_BF16 ? round_bf16(f[i]) : __builtin_bit_cast(uint16_t, (_Float16)f[i]);
                uint2 o = {(uint32_t)hb[0] | ((uint32_t)hb[1] << 16), (uint32_t)hb[2] | ((uint32_t)hb[3] << 16)};
                reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + n * (long)dim)[q] = o;
            }
        }
    }
}

int embed_dispatch(const int8_t* table, const void* scales, int scale_dtype, const int64_t* ids,
                   void* out, long n_ids, int vocab, int dim, hipStream_t stream)
{
    if (n_ids == 0) return EXL3_OK;
    // one workgroup per id, and a launch holds at most 2^32 - 1 work-items
    const long max_ids = 0xffffffffL / EMB_THREADS;
    if (n_ids > max_ids)
        return set_error(EXL3_ERR_ARG, "exl3_embed_int8_gather: %ld ids (at most %ld)", n_ids, max_ids);
    hipLaunchKernelGGL(embed_int8_kernel, dim3((unsigned)n_ids), dim3(EMB_THREADS), 0, stream, table, scales,
                       scale_dtype, ids, out, vocab, dim);
    return check_launch("exl3_embed_int8_gather");
}

}  // namespace exl3
