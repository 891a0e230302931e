// Fused EXL3 decode-GEMV for 1..16 activation rows:
//   C = fp16( H( fp16(H(A * suh)) . W_q ) * svh )
// with W_q decoded from the packed trellis on the fly and never written anywhere.
// Replaces exllamav3_ext.exl3_gemm as called at orcasaq2/ops.py:46-49 (rows <= 144 there;
// this path takes rows <= 16 and the MFMA GEMM takes the rest).  Row counts:
//   * 1: gemv1.hip (persistent decode, MFMA multiply-accumulate);
//   * 2..GV_SPLIT_MAX_ROWS: gemv1.hip as well where its launch keeps three workgroups per
//     CU resident (gemv1_rows_fit), else the two kernels below;
//   * above (5..16): gemv16.hip (the batch-1 decode on 4 x 2-tile units, one MFMA serving all
//     16 rows; the cost hardly depends on the row count).
//
// Two kernels, no inter-workgroup synchronisation inside a kernel (an agent-scope fence
// on this part writes back and invalidates the whole per-XCD L2, which serialises):
//   1. gemv_partial_kernel -- one pass over the packed words.  A workgroup owns one
//      128-output column group cg (8 tile columns = one output Hadamard block) and a
//      split of the input dimension (bps blocks of 128 inputs).  It builds
//      fp16(H(A * suh)) for its input range in LDS, then wave w streams tile columns
//      8cg + 2w + {0,1}: each step covers 4 tile rows, lane 16g + 8h + c holding chunk c of
//      tile (ti0 + g, tn_h) -- K contiguous u32 words -- through a 4-deep register ring
//      (loads issued three steps ahead).  Each masked codebook word enters
//      v_mfma_f32_16x16x32_f16 as its two fp16 halves (two k-slots) against a duplicated
//      activation, weights as the A operand (rows = outputs), activations as the B operand
//      (columns = batch rows).  Partial sums go to workspace[split][row][n] (fp32).
//   2. gemv_reduce_kernel -- per column group: add the splits in a fixed order
//      (deterministic), output Hadamard, * svh, fp16 store into C (row stride ldc).
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

constexpr int GV_WAVES = 4;
constexpr int GV_MAX_ROWS = 16;
constexpr int GV_SPLIT_MAX_ROWS = 4;                   // more rows: gemv16.hip
constexpr int GV_MAX_BLKS = 8;                          // 128-input blocks per workgroup (even)
constexpr int GV_HX_ROW = GV_MAX_BLKS * 8 * 16 + 4;     // u32 per LDS activation row (16 B per tile row and m)
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

// 128-input blocks per workgroup: even, at most GV_MAX_BLKS, aiming at GV_TARGET_WGS
// workgroups per shard.
static inline int gemv_bps(int ic, int oc)
{
    const int nblk = ic / 128, ncg = oc / 128;
    int bps = (int)(((long)nblk * ncg + GV_TARGET_WGS - 1) / GV_TARGET_WGS);
    bps = (bps + 1) & ~1;
    if (bps < 2) bps = 2;
    if (bps > GV_MAX_BLKS) bps = GV_MAX_BLKS;
    return bps;
}

static inline int gemv_splits(int ic, int oc)
{
    const int bps = gemv_bps(ic, oc);
    return (ic / 128 + bps - 1) / bps;
}

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Per-shard share of a GEMV workspace (the reserved head area is added once per call).
size_t gemv_workspace_bytes(int rows, int ic, int oc)
{
    if (rows == 1) return align256(gemv1_slot_bytes(ic, oc, 1));
    if (rows <= GV_SPLIT_MAX_ROWS)   // either path: the 1..4-row kernel's slots or the split partials
        return align256(std::max(gemv1_slot_bytes(ic, oc, rows),
                                 (size_t)gemv_splits(ic, oc) * rows * oc * sizeof(float)));
    if (rows > GV_SPLIT_MAX_ROWS) return align256(gemv16_shard_bytes(ic, oc));
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
    // Activations in "half-pair" order: row j (0..rows; row `rows` is zero), tile row t,
    // group m: x(2m), x(2m), x(2m+1), x(2m+1), x(2m+8), x(2m+8), x(2m+9), x(2m+9) -- the B
    // fragment that meets the lo/hi halves of the codebook words of rows 2m, 2m+1, 2m+8, 2m+9.
    extern __shared__ __attribute__((aligned(16))) uint32_t hx[];

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

    // ---- first packed words in flight before the activation prologue
    const int tc = oc >> 4;
    const int kg = lane >> 4;           // tile row within the step (MFMA k-group)
    const int h = (lane >> 3) & 1;      // tile column within the wave's pair
    const int c = lane & 7;             // chunk within the tile
    const int j = lane & 15;            // batch row fed as B-operand column
    const int tn = cg * 8 + wave * 2 + h;
    const uint32_t* tp = g.trellis[sh] + ((long)(blk0 * 8 + kg) * tc + tn) * (8 * K);
    const long step = 4L * tc * (8 * K);
    const int nsteps = nblk * 2;          // real steps (even, >= 2)
    const int last = nsteps - 1;
    // The loop runs a multiple of 4 steps; padding steps (only when nblk is odd) reread
    // the last real step's words and meet zero activations.  Prefetch addresses are
    // clamped rather than branched on, so the loop body is straight-line code and the
    // waits before each step only cover that step's own loads.
    uint32_t wa[K + 1], wb[K + 1], wc[K + 1], wd[K + 1];
    load_chunk<K>(wa, tp, c);
    load_chunk<K>(wb, tp + step, c);
    load_chunk<K>(wc, tp + min(2, last) * step, c);
    load_chunk<K>(wd, tp + min(3, last) * step, c);

    // ---- activations: fp16(H(A * suh)) for this input range; the zero row and the padding
    // block (when nblk is odd) are written as zeros
    const int nblk_pad = (nblk + 1) & ~1;
    for (int task = wave; task < (rows + 1) * nblk_pad; task += GV_WAVES) {
        const int r = task / nblk_pad, b = task % nblk_pad;
        float v0 = 0.f, v1 = 0.f;
        if (r < rows && b < nblk) {
            const uint32_t xv = reinterpret_cast<const uint32_t*>(A + (long)r * g.ic + (blk0 + b) * 128)[lane];
            const uint32_t sv = reinterpret_cast<const uint32_t*>(g.suh[sh] + (blk0 + b) * 128)[lane];
            v0 = h2f_lo(xv) * h2f_lo(sv);
            v1 = h2f_hi(xv) * h2f_hi(sv);
            wave_fwht128(v0, v1);
        }
        // lane holds rows r0 = 2(lane%8), r0+1 of tile row 8b + lane/8
        const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16)v0);
        const uint32_t h1 = __builtin_bit_cast(uint16_t, (_Float16)v1);
        const int t = 8 * b + (lane >> 3), r0 = 2 * (lane & 7);
        const int m = (r0 & 7) >> 1, slot = r0 >> 3;
        uint32_t* dst = hx + r * GV_HX_ROW + (t * 4 + m) * 4 + slot * 2;
        *reinterpret_cast<uint2*>(dst) = uint2{h0 | (h0 << 16), h1 | (h1 << 16)};
    }
    const CbConsts kc = cb_consts();
    __syncthreads();

    f32x4 acc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint32_t* xrow = hx + min(j, rows) * GV_HX_ROW + kg * 16;
    auto mac = [&](const uint32_t (&w)[K + 1], int s) {
        const uint32_t* xb = xrow + s * 64;
        const f16x8 b0 = *reinterpret_cast<const f16x8*>(xb);
        const f16x8 b1 = *reinterpret_cast<const f16x8*>(xb + 4);
        const f16x8 b2 = *reinterpret_cast<const f16x8*>(xb + 8);
        const f16x8 b3 = *reinterpret_cast<const f16x8*>(xb + 12);
        acc[0] = mfma16x16x32(chunk_hfragment<K, CB, 0, 0>(w, kc), b0, acc[0]);
        acc[2] = mfma16x16x32(chunk_hfragment<K, CB, 1, 0>(w, kc), b0, acc[2]);
        acc[1] = mfma16x16x32(chunk_hfragment<K, CB, 0, 1>(w, kc), b1, acc[1]);
        acc[3] = mfma16x16x32(chunk_hfragment<K, CB, 1, 1>(w, kc), b1, acc[3]);
        acc[0] = mfma16x16x32(chunk_hfragment<K, CB, 0, 2>(w, kc), b2, acc[0]);
        acc[2] = mfma16x16x32(chunk_hfragment<K, CB, 1, 2>(w, kc), b2, acc[2]);
        acc[1] = mfma16x16x32(chunk_hfragment<K, CB, 0, 3>(w, kc), b3, acc[1]);
        acc[3] = mfma16x16x32(chunk_hfragment<K, CB, 1, 3>(w, kc), b3, acc[3]);
    };
    for (int s = 0; s < nsteps; s += 4) {
        mac(wa, s);
        load_chunk<K>(wa, tp + min(s + 4, last) * step, c);
        mac(wb, s + 1);
        load_chunk<K>(wb, tp + min(s + 5, last) * step, c);
        mac(wc, s + 2);
        load_chunk<K>(wc, tp + min(s + 6, last) * step, c);
        mac(wd, s + 3);
        load_chunk<K>(wd, tp + min(s + 7, last) * step, c);
    }
    const f32x4 acc0 = acc[0] + acc[1], acc1 = acc[2] + acc[3];

    // ---- partial sums: lane holds D[4G + e][j], output n = 16 tn(G/2) + 4(G%2) + e (+8 for acc1)
    if (j < rows) {
        const int G = lane >> 4;
        const int n = (cg * 8 + wave * 2 + (G >> 1)) * 16 + 4 * (G & 1);
        float* p = g.partial[sh] + ((long)split * rows + j) * oc + n;
        *reinterpret_cast<f32x4*>(p) = acc0;
        *reinterpret_cast<f32x4*>(p + 8) = acc1;
    }
}

// One workgroup per (shard, column group).  Phase 1: task (row r, quarter q) adds the
// splits s = q, q+4, q+8, ... into LDS (loads issued together); phase 2: wave w takes rows
// w, w+4, ..., adds the four quarters in order (fixed summation order: deterministic),
// applies the output Hadamard and svh and stores fp16.
__global__ __launch_bounds__(64 * GV_WAVES) void gemv_reduce_kernel(const GemvGroup g)
{
    __shared__ float red[GV_MAX_ROWS * 4 * 128];
    const int sh = find_shard(g.cg_begin, g.nshards, blockIdx.x);
    const int cg = blockIdx.x - g.cg_begin[sh];
    const int oc = g.oc[sh];
    const int rows = g.rows;
    const int nsplit = g.splits[sh];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const long sstride = (long)rows * oc;
    for (int task = wave; task < rows * 4; task += GV_WAVES) {
        const int r = task >> 2, q = task & 3;
        const float* p = g.partial[sh] + (long)r * oc + cg * 128 + 2 * lane;
        float v0 = 0.f, v1 = 0.f;
        int s = q;
        for (; s + 12 < nsplit; s += 16) {
            const float2 x0 = *reinterpret_cast<const float2*>(p + s * sstride);
            const float2 x1 = *reinterpret_cast<const float2*>(p + (s + 4) * sstride);
            const float2 x2 = *reinterpret_cast<const float2*>(p + (s + 8) * sstride);
            const float2 x3 = *reinterpret_cast<const float2*>(p + (s + 12) * sstride);
            v0 += x0.x; v1 += x0.y;
            v0 += x1.x; v1 += x1.y;
            v0 += x2.x; v1 += x2.y;
            v0 += x3.x; v1 += x3.y;
        }
        for (; s < nsplit; s += 4) {
            const float2 x = *reinterpret_cast<const float2*>(p + s * sstride);
            v0 += x.x;
            v1 += x.y;
        }
        red[(r * 4 + q) * 128 + 2 * lane] = v0;
        red[(r * 4 + q) * 128 + 2 * lane + 1] = v1;
    }
    __syncthreads();
    const uint32_t sv = reinterpret_cast<const uint32_t*>(g.svh[sh] + cg * 128)[lane];
    for (int r = wave; r < rows; r += GV_WAVES) {
        float v0 = 0.f, v1 = 0.f;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            v0 += red[(r * 4 + q) * 128 + 2 * lane];
            v1 += red[(r * 4 + q) * 128 + 2 * lane + 1];
        }
        wave_fwht128(v0, v1);
        v0 *= h2f_lo(sv);
        v1 *= h2f_hi(sv);
        reinterpret_cast<uint32_t*>(g.C[sh] + (long)r * g.ldc[sh] + cg * 128)[lane] = pack_h2(v0, v1);
    }
}

// ---------------------------------------------------------------- host side

template <int K, int CB>
static const void* partial_fn() { return reinterpret_cast<const void*>(&gemv_partial_kernel<K, CB>); }

static const void* partial_fn_kcb(int K, int cb)
{
#define EXL3_CASE(KK) case KK: return cb == CB_MCG ? partial_fn<KK, CB_MCG>() : partial_fn<KK, CB_3INST>();
    switch (K) {
        EXL3_CASE(1) EXL3_CASE(2) EXL3_CASE(3) EXL3_CASE(4)
        EXL3_CASE(5) EXL3_CASE(6) EXL3_CASE(7) EXL3_CASE(8)
    }
#undef EXL3_CASE
    return nullptr;
}

static size_t hx_bytes(int rows) { return (size_t)(rows + 1) * GV_HX_ROW * sizeof(uint32_t); }

// Raises a kernel's dynamic-LDS limit once per device (LDS above 64 KB needs it).
static void allow_lds(const void* fn, size_t lds)
{
    struct Entry { const void* fn; int dev; size_t lds; };
    static thread_local Entry seen[128];
    static thread_local int nseen = 0;
    int dev = 0;
    hipGetDevice(&dev);
    for (int i = 0; i < nseen; i++)
        if (seen[i].fn == fn && seen[i].dev == dev && seen[i].lds >= lds) return;
    hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(hx_bytes(GV_MAX_ROWS)));
    (void)hipGetLastError();
    if (nseen < 128) seen[nseen++] = Entry{fn, dev, hx_bytes(GV_MAX_ROWS)};
}

// Shards with the same (K, codebook) share one partial launch; the reduce kernel covers a
// whole launch group.  The workspace holds each shard's partial block in shard order.
int gemv_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows,
                  void* workspace, size_t ws_bytes, hipStream_t stream)
{
    if (rows < 1 || rows > GV_MAX_ROWS)
        return set_error(EXL3_ERR_ARG, "exl3_gemv: rows=%d is not in 1..%d", rows, GV_MAX_ROWS);
    size_t offs[EXL3_MAX_SHARDS + 1];
    offs[0] = GEMV_COUNTER_BYTES;
    for (int i = 0; i < nshards; i++) offs[i + 1] = offs[i] + gemv_workspace_bytes(rows, shards[i].ic, shards[i].oc);
    if (ws_bytes < offs[nshards])
        return set_error(EXL3_ERR_WORKSPACE, "exl3_gemv: workspace of %zu bytes, %zu needed", ws_bytes,
                         offs[nshards]);

    char* ws = static_cast<char*>(workspace);
    if (rows == 1 || (rows <= GV_SPLIT_MAX_ROWS && gemv1_rows_fit(shards, nshards, rows)))
        return gemv1_dispatch(A, shards, nshards, rows, ws + GEMV_COUNTER_BYTES, offs[nshards] - GEMV_COUNTER_BYTES,
                              stream);
    if (rows > GV_SPLIT_MAX_ROWS)
        return gemv16_dispatch(A, shards, nshards, rows, ws + GEMV_COUNTER_BYTES, offs[nshards] - GEMV_COUNTER_BYTES,
                               stream);
    bool done[EXL3_MAX_SHARDS] = {false};
    const size_t lds = hx_bytes(rows);
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
        const void* fn = partial_fn_kcb(shards[i].K, shards[i].cb);
        if (!fn) return set_error(EXL3_ERR_ARG, "exl3_gemv: K=%d is not in 1..8", shards[i].K);
        allow_lds(fn, lds);
        void* kargs[] = {const_cast<uint16_t**>(&A), &args};
        hipLaunchKernel(fn, dim3(wgs), dim3(64 * GV_WAVES), kargs, lds, stream);
        int rc = check_launch("exl3_gemv (partial)");
        if (rc != EXL3_OK) return rc;
        hipLaunchKernelGGL(gemv_reduce_kernel, dim3(cgs), dim3(64 * GV_WAVES), 0, stream, args);
        rc = check_launch("exl3_gemv (reduce)");
        if (rc != EXL3_OK) return rc;
    }
    return EXL3_OK;
}

}  // namespace exl3
