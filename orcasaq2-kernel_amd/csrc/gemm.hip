// Prefill EXL3 GEMM for 17 to GEMM_SK_MIN_ROWS activation rows (more rows: gemm_sk.hip):
//   C = fp16( H( fp16(H(A * suh)) . W_q ) * svh )
// Replaces the reconstruct branch of orcasaq2/ops.py:50-59 (had_r_128 -> reconstruct ->
// hgemm_recon -> had_r_128) with: one had_r_128 pass over A into the workspace, then one
// kernel that decodes trellis tiles straight into MFMA operand registers -- the dense
// W_q is never written to HBM -- and applies the output Hadamard and svh in its epilogue.
//
// Workgroup tile: BM activation rows x 128 outputs (one output Hadamard block).
// Wave w owns tile columns 8cg + 2w + {0,1} for all BM rows.  Per step of 4 tile rows
// (64 inputs): lane 16g + 8h + c decodes chunk c of tile (ti0 + g, tn_h) into four 8-row
// fragments, which are the B operand (columns = outputs) of v_mfma_f32_16x16x32_f16;
// the A operand comes from the activation tile staged in LDS.
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

constexpr int GM_WAVES = 4;
constexpr int GM_BM = 64;
constexpr int GM_KSTEP = 64;                 // inputs per step (4 tile rows)
constexpr int GM_ASTRIDE = GM_KSTEP + 8;     // halves per staged activation row
constexpr int GM_CSTRIDE = 128 + 4;          // floats per staged output row

// Row counts above this take the stream-K kernel (gemm_sk.hip), which decodes each weight
// once per 256 rows; at or below it, this kernel (one decode per 64 rows, no partial sums).
constexpr int GEMM_SK_MIN_ROWS = 192;

static size_t gemm_ah_bytes(int rows, int ic) { return ((size_t)rows * ic * sizeof(uint16_t) + 255) & ~(size_t)255; }

size_t gemm_workspace_bytes(int rows, int ic, int oc)
{
    const size_t ah = gemm_ah_bytes(rows, ic);
    return rows > GEMM_SK_MIN_ROWS ? ah + gemm_sk_slot_bytes(rows, oc, gemm_sk_cus()) : ah;
}

template <int K, int CB>
__global__ __launch_bounds__(64 * GM_WAVES) void gemm_kernel(
    const uint16_t* __restrict__ Ah, const uint32_t* __restrict__ trellis, uint16_t* __restrict__ C,
    const uint16_t* __restrict__ svh, int rows, int ic, int oc)
{
    __shared__ __attribute__((aligned(16))) _Float16 as[GM_BM * GM_ASTRIDE];
    __shared__ __attribute__((aligned(16))) float cs[GM_BM * GM_CSTRIDE];

    const int ncg = oc >> 7;
    const int cg = blockIdx.x % ncg;
    const int m0 = (blockIdx.x / ncg) * GM_BM;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int tc = oc >> 4;
    const int kg = lane >> 4, h = (lane >> 3) & 1, c = lane & 7, i16 = lane & 15;
    const int tn = cg * 8 + wave * 2 + h;
    const uint32_t* tp = trellis + ((long)kg * tc + tn) * (8 * K);
    const long tstep = 4L * tc * (8 * K);
    const int nsteps = ic / GM_KSTEP;

    f32x4 acc[GM_BM / 16][2];
#pragma unroll
    for (int mb = 0; mb < GM_BM / 16; mb++) acc[mb][0] = acc[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};

    uint32_t w[K + 1];
    for (int s = 0; s < nsteps; s++) {
        // stage A[m0 .. m0+BM, 64 s .. 64 s + 64) (zero rows past `rows`)
        for (int t = threadIdx.x; t < GM_BM * (GM_KSTEP / 8); t += 64 * GM_WAVES) {
            const int r = t / (GM_KSTEP / 8), seg = t % (GM_KSTEP / 8);
            uint4 v = {0u, 0u, 0u, 0u};
            if (m0 + r < rows) v = *reinterpret_cast<const uint4*>(Ah + (long)(m0 + r) * ic + s * GM_KSTEP + seg * 8);
            *reinterpret_cast<uint4*>(as + r * GM_ASTRIDE + seg * 8) = v;
        }
        load_chunk<K>(w, tp + s * tstep, c);
        const f16x8 b00 = chunk_fragment<K, CB, 0, 0>(w);
        const f16x8 b01 = chunk_fragment<K, CB, 0, 1>(w);
        const f16x8 b10 = chunk_fragment<K, CB, 1, 0>(w);
        const f16x8 b11 = chunk_fragment<K, CB, 1, 1>(w);
        __syncthreads();
#pragma unroll
        for (int mb = 0; mb < GM_BM / 16; mb++) {
            const _Float16* ap = as + (mb * 16 + i16) * GM_ASTRIDE + kg * 16;
            const f16x8 a0 = *reinterpret_cast<const f16x8*>(ap);
            const f16x8 a1 = *reinterpret_cast<const f16x8*>(ap + 8);
            acc[mb][0] = mfma16x16x32(a0, b00, acc[mb][0]);
            acc[mb][0] = mfma16x16x32(a1, b01, acc[mb][0]);
            acc[mb][1] = mfma16x16x32(a0, b10, acc[mb][1]);
            acc[mb][1] = mfma16x16x32(a1, b11, acc[mb][1]);
        }
        __syncthreads();
    }

    // ---- epilogue: D[mb][ch] lane holds rows 16mb + 4G + e, column j = lane % 16
    {
        const int G = lane >> 4, jj = lane & 15;
        const int ncol = (wave * 2 + (jj >> 3)) * 16 + (jj & 7);   // column within the group
#pragma unroll
        for (int mb = 0; mb < GM_BM / 16; mb++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int r = mb * 16 + 4 * G + e;
                cs[r * GM_CSTRIDE + ncol] = acc[mb][0][e];
                cs[r * GM_CSTRIDE + ncol + 8] = acc[mb][1][e];
            }
    }
    __syncthreads();
    const uint32_t sv = reinterpret_cast<const uint32_t*>(svh + cg * 128)[lane];
    const float s0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(sv & 0xffffu));
    const float s1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(sv >> 16));
    for (int r = wave; r < GM_BM; r += GM_WAVES) {
        if (m0 + r >= rows) break;
        float v0 = cs[r * GM_CSTRIDE + 2 * lane], v1 = cs[r * GM_CSTRIDE + 2 * lane + 1];
        wave_fwht128(v0, v1);
        v0 *= s0;
        v1 *= s1;
        const uint32_t o = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v0) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v1) << 16);
        reinterpret_cast<uint32_t*>(C + (long)(m0 + r) * oc + cg * 128)[lane] = o;
    }
}

template <int K, int CB>
static void launch_gemm(const uint16_t* Ah, const uint32_t* trellis, uint16_t* C, const uint16_t* svh,
                        int rows, int ic, int oc, hipStream_t stream)
{
    const int grid = ((rows + GM_BM - 1) / GM_BM) * (oc / 128);
    hipLaunchKernelGGL((gemm_kernel<K, CB>), dim3(grid), dim3(64 * GM_WAVES), 0, stream, Ah, trellis, C,
                       svh, rows, ic, oc);
}

int gemm_dispatch(const uint16_t* A, const uint32_t* trellis, uint16_t* C, const uint16_t* suh,
                  const uint16_t* svh, void* workspace, size_t ws_bytes, int rows, int ic, int oc,
                  int K, int cb, hipStream_t stream)
{
    const size_t need = gemm_workspace_bytes(rows, ic, oc);
    if (ws_bytes < need)
        return set_error(EXL3_ERR_WORKSPACE, "exl3_gemm: workspace of %zu bytes, %zu needed", ws_bytes, need);
    uint16_t* Ah = static_cast<uint16_t*>(workspace);
    int rc = had_dispatch(A, Ah, suh, nullptr, 1.0f, rows, ic, stream);
    if (rc != EXL3_OK) return rc;
    if (rows > GEMM_SK_MIN_ROWS) {
        const size_t ah = gemm_ah_bytes(rows, ic);
        return gemm_sk_dispatch(Ah, trellis, C, svh, static_cast<char*>(workspace) + ah, ws_bytes - ah, rows, ic, oc,
                                K, cb, gemm_sk_cus(), stream);
    }
#define EXL3_CASE(KK)                                                                        \
    case KK:                                                                                 \
        if (cb == CB_MCG) launch_gemm<KK, CB_MCG>(Ah, trellis, C, svh, rows, ic, oc, stream); \
        else launch_gemm<KK, CB_3INST>(Ah, trellis, C, svh, rows, ic, oc, stream);           \
        break;
    switch (K) {
        EXL3_CASE(1) EXL3_CASE(2) EXL3_CASE(3) EXL3_CASE(4)
        EXL3_CASE(5) EXL3_CASE(6) EXL3_CASE(7) EXL3_CASE(8)
        default: return set_error(EXL3_ERR_ARG, "exl3_gemm: K=%d is not in 1..8", K);
    }
#undef EXL3_CASE
    return check_launch("exl3_gemm");
}

}  // namespace exl3
