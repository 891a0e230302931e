// Fused EXL3 decode-GEMV for 1..16 activation rows:
//   C = fp16( H( fp16(H(A * suh)) . W_q ) * svh )
// with W_q decoded from the packed trellis on the fly and never written anywhere.
// Replaces exllamav3_ext.exl3_gemm as called at orcasaq2/ops.py:46-49 (rows <= 144 there;
// this path takes rows <= 16 and the MFMA GEMM takes the rest).
//
// Two kernels, no inter-workgroup synchronisation inside a kernel (an agent-scope fence
// on this part writes back / invalidates the whole per-XCD L2, which serialises):
//   1. gemv_partial_kernel -- one pass over the packed words.  A workgroup owns one
//      128-output column group cg (8 tile columns = one output Hadamard block) and a
//      split of the input dimension (bps blocks of 128 inputs).  It builds
//      fp16(H(A * suh)) for its input range in LDS (16 rows, zero rows past `rows`), then
//      wave w streams tile columns 8cg + 2w + {0,1}: each step covers 4 tile rows, lane
//      16g + 8h + c holds chunk c of tile (ti0 + g, tn_h) -- K contiguous u32 words,
//      prefetched two steps ahead -- decodes its 32 weights into four 8-element fragments
//      and issues four v_mfma_f32_16x16x32_f16 with the weights as the A operand (rows =
//      outputs) and the activations from LDS as the B operand (columns = batch rows).
//      Partial sums go to workspace[split][row][n] (fp32).
//   2. gemv_reduce_kernel -- per column group: add the splits in a fixed order
//      (deterministic), output Hadamard, * svh, fp16 store into C (row stride ldc).
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

constexpr int GV_WAVES = 4;
constexpr int GV_MAX_ROWS = 16;
constexpr int GV_MAX_BLKS = 8;                          // 128-input blocks per workgroup
constexpr int GV_STRIDE = GV_MAX_BLKS * 128 + 8;        // halves per LDS activation row
constexpr int GV_GROUP = 8;                             // shards per launch
constexpr int GV_TARGET_WGS = 1024;

struct GemvGroup {
    const uint32_t* trellis[GV_GROUP];
    const uint16_t* suh[GV_GROUP];
    const uint16_t* svh[GV_GROUP];
    uint16_t* C[GV_GROUP];
    float* partial[GV_GROUP];           // [splits][rows][oc]
    long ldc[GV_GROUP];
    int oc[GV_GROUP];
    int splits[GV_GROUP];
    int bps[GV_GROUP];
    int wg_begin[GV_GROUP + 1];         // partial kernel: workgroups of shards before s
    int cg_begin[GV_GROUP + 1];         // reduce kernel: column groups of shards before s
    int nshards, ic, rows;
};

static inline int gemv_bps(int ic, int oc)
{
    const int nblk = ic / 128, ncg = oc / 128;
    int bps = (int)(((long)nblk * ncg + GV_TARGET_WGS - 1) / GV_TARGET_WGS);
    if (bps < 1) bps = 1;
    if (bps > GV_MAX_BLKS) bps = GV_MAX_BLKS;
    return bps;
}

static inline int gemv_splits(int ic, int oc)
{
    const int bps = gemv_bps(ic, oc);
    return (ic / 128 + bps - 1) / bps;
}

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t gemv_workspace_bytes(int rows, int ic, int oc)
{
    return align256((size_t)gemv_splits(ic, oc) * rows * oc * sizeof(float));
}

__device__ __forceinline__ float h2f_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float h2f_hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }
__device__ __forceinline__ uint32_t pack_h2(float a, float b)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}

__device__ __forceinline__ int find_shard(const int* begin, int n, int idx)
{
    int s = 0;
    while (s + 1 < n && idx >= begin[s + 1]) s++;
    return s;
}

template <int K, int CB>
__global__ __launch_bounds__(64 * GV_WAVES) void gemv_partial_kernel(const uint16_t* __restrict__ A,
                                                                     const GemvGroup g)
{
    __shared__ __attribute__((aligned(16))) _Float16 xs[GV_MAX_ROWS * GV_STRIDE];

    const int sh = find_shard(g.wg_begin, g.nshards, blockIdx.x);
    const int wg = blockIdx.x - g.wg_begin[sh];
    const int oc = g.oc[sh];
    const int ncg = oc >> 7;
    const int cg = wg % ncg;
    const int split = wg / ncg;
    const int blk0 = split * g.bps[sh];
    const int nblk = min(g.bps[sh], (g.ic >> 7) - blk0);
    const int rows = g.rows;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;

    // ---- activations: fp16(H(A * suh)) for this input range, rows >= `rows` zero
    for (int task = wave; task < GV_MAX_ROWS * nblk; task += GV_WAVES) {
        const int r = task / nblk, b = task % nblk;
        float v0 = 0.f, v1 = 0.f;
        if (r < rows) {
            const uint32_t xv = reinterpret_cast<const uint32_t*>(A + (long)r * g.ic + (blk0 + b) * 128)[lane];
            const uint32_t sv = reinterpret_cast<const uint32_t*>(g.suh[sh] + (blk0 + b) * 128)[lane];
            v0 = h2f_lo(xv) * h2f_lo(sv);
            v1 = h2f_hi(xv) * h2f_hi(sv);
            wave_fwht128(v0, v1);
        }
        reinterpret_cast<uint32_t*>(xs + r * GV_STRIDE + b * 128)[lane] = pack_h2(v0, v1);
    }

    // ---- stream the packed tiles (prefetch issued before the barrier)
    const int tc = oc >> 4;
    const int kg = lane >> 4;           // tile row within the step (MFMA k-group)
    const int h = (lane >> 3) & 1;      // tile column within the wave's pair
    const int c = lane & 7;             // chunk within the tile
    const int j = lane & 15;            // batch row fed as B-operand column
    const int tn = cg * 8 + wave * 2 + h;
    const uint32_t* tp = g.trellis[sh] + ((long)(blk0 * 8 + kg) * tc + tn) * (8 * K);
    const long step = 4L * tc * (8 * K);
    const int nsteps = nblk * 2;        // >= 2

    uint32_t w0[K + 1], w1[K + 1], w2[K + 1];
    load_chunk<K>(w0, tp, c);
    load_chunk<K>(w1, tp + step, c);
    __syncthreads();

    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    const _Float16* xrow = xs + j * GV_STRIDE + kg * 16;
    for (int s = 0; s < nsteps; s++) {
        if (s + 2 < nsteps) load_chunk<K>(w2, tp + (s + 2) * step, c);
        const f16x8 b0 = *reinterpret_cast<const f16x8*>(xrow + s * 64);
        const f16x8 b1 = *reinterpret_cast<const f16x8*>(xrow + s * 64 + 8);
        acc0 = mfma16x16x32(chunk_fragment<K, CB, 0, 0>(w0), b0, acc0);
        acc0 = mfma16x16x32(chunk_fragment<K, CB, 0, 1>(w0), b1, acc0);
        acc1 = mfma16x16x32(chunk_fragment<K, CB, 1, 0>(w0), b0, acc1);
        acc1 = mfma16x16x32(chunk_fragment<K, CB, 1, 1>(w0), b1, acc1);
#pragma unroll
        for (int i = 0; i <= K; i++) {
            w0[i] = w1[i];
            w1[i] = w2[i];
        }
    }

    // ---- partial sums: lane holds D[4G + e][j], output n = 16 tn(G/2) + 4(G%2) + e (+8 for acc1)
    if (j < rows) {
        const int G = lane >> 4;
        const int n = (cg * 8 + wave * 2 + (G >> 1)) * 16 + 4 * (G & 1);
        float* p = g.partial[sh] + ((long)split * rows + j) * oc + n;
        *reinterpret_cast<f32x4*>(p) = acc0;
        *reinterpret_cast<f32x4*>(p + 8) = acc1;
    }
}

// One workgroup per (shard, column group); wave w handles rows w, w+4, ...
__global__ __launch_bounds__(64 * GV_WAVES) void gemv_reduce_kernel(const GemvGroup g)
{
    const int sh = find_shard(g.cg_begin, g.nshards, blockIdx.x);
    const int cg = blockIdx.x - g.cg_begin[sh];
    const int oc = g.oc[sh];
    const int rows = g.rows;
    const int nsplit = g.splits[sh];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t sv = reinterpret_cast<const uint32_t*>(g.svh[sh] + cg * 128)[lane];
    for (int r = wave; r < rows; r += GV_WAVES) {
        float v0 = 0.f, v1 = 0.f;
        const float* p = g.partial[sh] + (long)r * oc + cg * 128 + 2 * lane;
        for (int s = 0; s < nsplit; s++) {
            const float2 q = *reinterpret_cast<const float2*>(p + (long)s * rows * oc);
            v0 += q.x;
            v1 += q.y;
        }
        wave_fwht128(v0, v1);
        v0 *= h2f_lo(sv);
        v1 *= h2f_hi(sv);
        reinterpret_cast<uint32_t*>(g.C[sh] + (long)r * g.ldc[sh] + cg * 128)[lane] = pack_h2(v0, v1);
    }
}

template <int K, int CB>
static void launch_partial(const uint16_t* A, const GemvGroup& args, int wgs, hipStream_t stream)
{
    hipLaunchKernelGGL((gemv_partial_kernel<K, CB>), dim3(wgs), dim3(64 * GV_WAVES), 0, stream, A, args);
}

static int launch_partial_kcb(int K, int cb, const uint16_t* A, const GemvGroup& args, int wgs,
                              hipStream_t stream)
{
#define EXL3_CASE(KK)                                                                   \
    case KK:                                                                            \
        if (cb == CB_MCG) launch_partial<KK, CB_MCG>(A, args, wgs, stream);             \
        else launch_partial<KK, CB_3INST>(A, args, wgs, stream);                        \
        break;
    switch (K) {
        EXL3_CASE(1) EXL3_CASE(2) EXL3_CASE(3) EXL3_CASE(4)
        EXL3_CASE(5) EXL3_CASE(6) EXL3_CASE(7) EXL3_CASE(8)
        default: return set_error(EXL3_ERR_ARG, "exl3_gemv: K=%d is not in 1..8", K);
    }
#undef EXL3_CASE
    return check_launch("exl3_gemv (partial)");
}

// Shards with the same (K, codebook) share one partial launch; the reduce kernel covers a
// whole launch group.  The workspace holds each shard's partial block in shard order.
int gemv_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows,
                  void* workspace, size_t ws_bytes, hipStream_t stream)
{
    if (rows < 1 || rows > GV_MAX_ROWS)
        return set_error(EXL3_ERR_ARG, "exl3_gemv: rows=%d is not in 1..%d", rows, GV_MAX_ROWS);
    size_t offs[EXL3_MAX_SHARDS + 1];
    offs[0] = 0;
    for (int i = 0; i < nshards; i++) offs[i + 1] = offs[i] + gemv_workspace_bytes(rows, shards[i].ic, shards[i].oc);
    if (ws_bytes < offs[nshards])
        return set_error(EXL3_ERR_WORKSPACE, "exl3_gemv: workspace of %zu bytes, %zu needed", ws_bytes,
                         offs[nshards]);

    char* ws = static_cast<char*>(workspace);
    bool done[EXL3_MAX_SHARDS] = {false};
    for (int i = 0; i < nshards; i++) {
        if (done[i]) continue;
        GemvGroup args = {};
        args.ic = shards[i].ic;
        args.rows = rows;
        int wgs = 0, cgs = 0;
        for (int s = i; s < nshards && args.nshards < GV_GROUP; s++) {
            if (done[s] || shards[s].K != shards[i].K || shards[s].cb != shards[i].cb) continue;
            const GemvShard& d = shards[s];
            const int n = args.nshards++;
            args.trellis[n] = d.trellis;
            args.suh[n] = d.suh;
            args.svh[n] = d.svh;
            args.C[n] = d.C;
            args.ldc[n] = d.ldc;
            args.oc[n] = d.oc;
            args.bps[n] = gemv_bps(d.ic, d.oc);
            args.splits[n] = gemv_splits(d.ic, d.oc);
            args.partial[n] = reinterpret_cast<float*>(ws + offs[s]);
            args.wg_begin[n] = wgs;
            args.cg_begin[n] = cgs;
            wgs += (d.oc / 128) * args.splits[n];
            cgs += d.oc / 128;
            done[s] = true;
        }
        args.wg_begin[args.nshards] = wgs;
        args.cg_begin[args.nshards] = cgs;
        int rc = launch_partial_kcb(shards[i].K, shards[i].cb, A, args, wgs, stream);
        if (rc != EXL3_OK) return rc;
        hipLaunchKernelGGL(gemv_reduce_kernel, dim3(cgs), dim3(64 * GV_WAVES), 0, stream, args);
        rc = check_launch("exl3_gemv (reduce)");
        if (rc != EXL3_OK) return rc;
    }
    return EXL3_OK;
}

}  // namespace exl3
