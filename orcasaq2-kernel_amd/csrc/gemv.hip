// Fused EXL3 decode-GEMV for 1..16 activation rows:
//   C = fp16( H( fp16(H(A * suh)) . W_q ) * svh )
// with W_q decoded from the packed trellis on the fly and never written anywhere.
// Replaces exllamav3_ext.exl3_gemm as called at orcasaq2/ops.py:46-49 (rows <= 144 there;
// this kernel takes rows <= 16 and the MFMA GEMM takes the rest).
//
// Layout of the work (HBM-streaming; one pass over the packed words):
//   * A workgroup owns one 128-output column group cg (8 tile columns = one output
//     Hadamard block) and a split of the input dimension (bps blocks of 128 inputs).
//   * It first builds fp16(H(A * suh)) for its input range in LDS (16 rows, zero rows
//     beyond `rows`), one wave per 128-block.
//   * Wave w streams tile columns 8cg + 2w + {0,1}; each step covers 4 tile rows, so
//     lane 16g + 8h + c holds chunk c of tile (ti0 + g, tn_h) -- K contiguous u32 words.
//     The lane decodes its 32 weights into four 8-element MFMA fragments and the wave
//     issues four v_mfma_f32_16x16x32_f16 with the weights as the A operand (rows =
//     outputs) and the activations from LDS as the B operand (columns = batch rows).
//   * Partial sums go to workspace[split][row][n]; the last workgroup of a column group
//     (atomic ticket) adds the splits in a fixed order (deterministic), applies the
//     output Hadamard and svh, writes fp16 C and re-arms the ticket to zero.
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

constexpr int GV_WAVES = 4;
constexpr int GV_MAX_ROWS = 16;
constexpr int GV_MAX_BLKS = 8;                          // 128-input blocks per workgroup
constexpr int GV_STRIDE = GV_MAX_BLKS * 128 + 8;        // halves per LDS activation row
constexpr int GV_MAX_SHARDS = 4;
constexpr int GV_TARGET_WGS = 1024;

struct GemvArgs {
    const uint32_t* trellis[GV_MAX_SHARDS];
    const uint16_t* suh[GV_MAX_SHARDS];
    const uint16_t* svh[GV_MAX_SHARDS];
    uint16_t* C[GV_MAX_SHARDS];
    float* partial[GV_MAX_SHARDS];      // [splits][rows][oc]
    uint32_t* ticket[GV_MAX_SHARDS];    // [oc / 128]
    long ldc[GV_MAX_SHARDS];
    int oc[GV_MAX_SHARDS];
    int splits[GV_MAX_SHARDS];
    int bps[GV_MAX_SHARDS];
    int wg_begin[GV_MAX_SHARDS + 1];
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
    return align256((size_t)gemv_splits(ic, oc) * rows * oc * sizeof(float)) +
           align256((size_t)(oc / 128) * sizeof(uint32_t));
}

__device__ __forceinline__ float h2f_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float h2f_hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }
__device__ __forceinline__ uint32_t pack_h2(float a, float b)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}

template <int K, int CB>
__global__ __launch_bounds__(64 * GV_WAVES) void gemv_kernel(const uint16_t* __restrict__ A, const GemvArgs g)
{
    __shared__ __attribute__((aligned(16))) _Float16 xs[GV_MAX_ROWS * GV_STRIDE];
    __shared__ int last_flag;

    int wg = blockIdx.x, sh = 0;
    while (sh + 1 < g.nshards && wg >= g.wg_begin[sh + 1]) sh++;
    wg -= g.wg_begin[sh];
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
    __syncthreads();

    // ---- stream the packed tiles
    const int tc = oc >> 4;
    const int kg = lane >> 4;           // tile row within the step (MFMA k-group)
    const int h = (lane >> 3) & 1;      // tile column within the wave's pair
    const int c = lane & 7;             // chunk within the tile
    const int j = lane & 15;            // batch row fed as B-operand column
    const int tn = cg * 8 + wave * 2 + h;
    const uint32_t* tp = g.trellis[sh] + ((long)(blk0 * 8 + kg) * tc + tn) * (8 * K);
    const long step = 4L * tc * (8 * K);
    const int nsteps = nblk * 2;

    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    uint32_t w[K + 1], wn[K + 1];
    load_chunk<K>(w, tp, c);
    for (int s = 0; s < nsteps; s++) {
        if (s + 1 < nsteps) load_chunk<K>(wn, tp + (s + 1) * step, c);
        const _Float16* xb = xs + j * GV_STRIDE + (s * 4 + kg) * 16;
        const f16x8 b0 = *reinterpret_cast<const f16x8*>(xb);
        const f16x8 b1 = *reinterpret_cast<const f16x8*>(xb + 8);
        acc0 = mfma16x16x32(chunk_fragment<K, CB, 0, 0>(w), b0, acc0);
        acc0 = mfma16x16x32(chunk_fragment<K, CB, 0, 1>(w), b1, acc0);
        acc1 = mfma16x16x32(chunk_fragment<K, CB, 1, 0>(w), b0, acc1);
        acc1 = mfma16x16x32(chunk_fragment<K, CB, 1, 1>(w), b1, acc1);
#pragma unroll
        for (int i = 0; i <= K; i++) w[i] = wn[i];
    }

    // ---- partial sums: lane holds D[4G + e][j], output n = 16 tn(G/2) + 4(G%2) + e (+8 for acc1)
    if (j < rows) {
        const int G = lane >> 4;
        const int n = (cg * 8 + wave * 2 + (G >> 1)) * 16 + 4 * (G & 1);
        float* p = g.partial[sh] + ((long)split * rows + j) * oc + n;
        *reinterpret_cast<f32x4*>(p) = acc0;
        *reinterpret_cast<f32x4*>(p + 8) = acc1;
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = atomicAdd(g.ticket[sh] + cg, 1u);
        last_flag = (prev == (uint32_t)g.splits[sh] - 1u);
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();

    // ---- last workgroup of this column group: reduce splits, output Hadamard, svh
    const int nsplit = g.splits[sh];
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
    if (threadIdx.x == 0) __hip_atomic_store(g.ticket[sh] + cg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int K, int CB>
static void launch_gemv(const uint16_t* A, const GemvArgs& args, int wgs, hipStream_t stream)
{
    hipLaunchKernelGGL((gemv_kernel<K, CB>), dim3(wgs), dim3(64 * GV_WAVES), 0, stream, A, args);
}

static int launch_gemv_kcb(int K, int cb, const uint16_t* A, const GemvArgs& args, int wgs, hipStream_t stream)
{
#define EXL3_CASE(KK)                                                                   \
    case KK:                                                                            \
        if (cb == CB_MCG) launch_gemv<KK, CB_MCG>(A, args, wgs, stream);                \
        else launch_gemv<KK, CB_3INST>(A, args, wgs, stream);                           \
        break;
    switch (K) {
        EXL3_CASE(1) EXL3_CASE(2) EXL3_CASE(3) EXL3_CASE(4)
        EXL3_CASE(5) EXL3_CASE(6) EXL3_CASE(7) EXL3_CASE(8)
        default: return set_error(EXL3_ERR_ARG, "exl3_gemv: K=%d is not in 1..8", K);
    }
#undef EXL3_CASE
    return check_launch("exl3_gemv");
}

// Shards are grouped by (K, codebook); each group is one launch.  The workspace holds,
// per shard in order, the partial-sum block and the ticket block.
int gemv_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows,
                  void* workspace, size_t ws_bytes, hipStream_t stream)
{
    if (rows < 1 || rows > GV_MAX_ROWS)
        return set_error(EXL3_ERR_ARG, "exl3_gemv: rows=%d is not in 1..%d", rows, GV_MAX_ROWS);
    size_t need = 0;
    for (int i = 0; i < nshards; i++) need += gemv_workspace_bytes(rows, shards[i].ic, shards[i].oc);
    if (ws_bytes < need)
        return set_error(EXL3_ERR_WORKSPACE, "exl3_gemv: workspace of %zu bytes, %zu needed", ws_bytes, need);

    char* ws = static_cast<char*>(workspace);
    bool done[64] = {false};
    size_t offs[64];
    {
        size_t o = 0;
        for (int i = 0; i < nshards; i++) {
            offs[i] = o;
            o += gemv_workspace_bytes(rows, shards[i].ic, shards[i].oc);
        }
    }
    for (int i = 0; i < nshards; i++) {
        if (done[i]) continue;
        GemvArgs args = {};
        args.ic = shards[i].ic;
        args.rows = rows;
        int wgs = 0;
        for (int s = i; s < nshards && args.nshards < GV_MAX_SHARDS; s++) {
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
            args.ticket[n] = reinterpret_cast<uint32_t*>(
                ws + offs[s] + align256((size_t)args.splits[n] * rows * d.oc * sizeof(float)));
            args.wg_begin[n] = wgs;
            wgs += (d.oc / 128) * args.splits[n];
            done[s] = true;
        }
        args.wg_begin[args.nshards] = wgs;
        const int rc = launch_gemv_kcb(shards[i].K, shards[i].cb, A, args, wgs, stream);
        if (rc != EXL3_OK) return rc;
    }
    return EXL3_OK;
}

}  // namespace exl3
