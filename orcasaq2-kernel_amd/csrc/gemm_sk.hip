// Prefill EXL3 GEMM for many activation rows, stream-K over 256 x 256 output tiles:
//   C = fp16( H( Ah . W_q ) * svh ),  Ah = fp16(H(A * suh)) (had_r_128 pass, gemm.hip)
// W_q is decoded from the packed trellis straight into LDS (never written to HBM), once per
// 256-row tile, and multiplied with v_mfma_f32_16x16x32_f16.  Replaces the reconstruct
// branch of orcasaq2/ops.py:50-59 (reconstruct -> hgemm_recon -> had_r_128) for row counts
// where the decode cost spread over 256 rows is small next to the MFMA work.
//
// Work decomposition.  Output tiles are 256 rows x 256 outputs (two output Hadamard blocks);
// a tile is nks = ic / 64 K-steps of 64 inputs.  The tiles' K-steps, numbered tile-major,
// are cut into G nearly equal contiguous ranges, one per workgroup, G = one per CU (all
// resident): every CU does the same number of K-steps whatever the tile count ("stream-K").
// A range covers at most a few tile pieces.  A piece that is a whole tile is finished by
// its workgroup; a partial piece leaves its fp32 accumulators in a slot of the workspace,
// and the last of the tile's workgroups to arrive (an agent-scope counter per tile) adds
// the slots in workgroup order -- deterministic -- and finishes the tile.
//
// Per workgroup (8 waves, two per SIMD; wave w owns rows 128 (w / 4) .., outputs
// 64 (w % 4) .. of the tile: 8 x 4 MFMA blocks, 128 fp32 accumulators per lane) and K-step:
//   * the A tile (256 x 64 fp16) is loaded into registers one K-step ahead, then stored to
//     LDS rows of 72 halves (16-byte reads of 16 consecutive rows hit distinct banks);
//   * the B tile is 4 tile rows x 16 tile columns = 512 chunks of 32 positions, one per
//     lane: its K words are loaded one K-step ahead, the tail-biting word comes by DPP from
//     the neighbouring lane, each masked word's fp16 halves are summed (the reconstruct
//     rounding) and the chunk's two output columns' 16 inputs go to LDS as [output][input];
//   * 2 x 12 LDS reads of 16 bytes feed 64 MFMAs.
// Epilogue per 128-output block (two waves): rows through LDS, FWHT across a wave, * svh,
// fp16 store.
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

constexpr int SK_WAVES = 8;
constexpr int SK_BM = 256;
constexpr int SK_BN = 256;
constexpr int SK_KS = 64;                     // inputs per K-step (4 tile rows)
constexpr int SK_LD = SK_KS + 8;              // halves per LDS row of the A and B tiles
constexpr int SK_ACC = 128;                   // fp32 accumulators per lane
constexpr int SK_LDS = 2 * SK_BM * SK_LD * 2; // A + B tiles, bytes (73728)
constexpr int SK_CLD = 128 + 4;               // floats per epilogue row in LDS

struct SkArgs {
    const uint16_t* Ah;        // (rows, ic) fp16, Hadamard-transformed activations
    const uint32_t* trellis;   // (ic/16, oc/16, 8K) u32
    uint16_t* C;               // (rows, oc) fp16
    const uint16_t* svh;       // (oc)
    uint32_t* counters;        // one per tile, zeroed by sk_clear_kernel before the launch
    float* slots;              // (tiles + G) x SK_WAVES x SK_ACC x 64 fp32
    int rows, ic, oc, ntn, nks, ntiles;
    int q, r;                  // K-steps per workgroup: q + (g < r)
};

__global__ void sk_clear_kernel(uint32_t* counters, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) counters[i] = 0u;
}

// First K-step (global numbering) of workgroup g, and the workgroup holding K-step u.
__device__ __forceinline__ long sk_first(const SkArgs& a, int g) { return (long)g * a.q + min(g, a.r); }
__device__ __forceinline__ int sk_wg_of(const SkArgs& a, long u)
{
    const long big = (long)a.r * (a.q + 1);
    return u < big ? (int)(u / (a.q + 1)) : a.r + (int)((u - big) / a.q);
}

// (w_a, w_b) packed: each weight is the fp16 sum of its masked word's two halves (one RNE
// add, as the reconstruct kernel rounds it).
__device__ __forceinline__ uint32_t sk_pair(uint32_t xa, uint32_t xb)
{
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t lo = __builtin_amdgcn_perm(xb, xa, 0x05040100u);
    const uint32_t hi = __builtin_amdgcn_perm(xb, xa, 0x07060302u);
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, lo) + __builtin_bit_cast(h2, hi));
}

template <int K, int CB, int... Qs>
__device__ __forceinline__ void sk_words(const uint32_t (&w)[K + 1], const Dot2Consts& kc, uint32_t (&x)[32],
                                         std::integer_sequence<int, Qs...>)
{
    ((x[Qs] = dot2_word<K, CB, Qs>(w, kc)), ...);
}

// A chunk (tile columns c and c + 8, all 16 input rows) as fp16 weights in input order:
// o[0], o[1] = column c rows 0..7, 8..15; o[2], o[3] = column c + 8.  Position q = 8m + i
// holds row 2m + {0, 1, 8, 9}[i % 4] of column c + 8 (i / 4).
template <int K, int CB>
__device__ __forceinline__ void sk_decode(const uint32_t (&w)[K + 1], const Dot2Consts& kc, uint4 (&o)[4])
{
    uint32_t x[32];
    sk_words<K, CB>(w, kc, x, std::make_integer_sequence<int, 32>{});
    o[0] = uint4{sk_pair(x[0], x[1]), sk_pair(x[8], x[9]), sk_pair(x[16], x[17]), sk_pair(x[24], x[25])};
    o[1] = uint4{sk_pair(x[2], x[3]), sk_pair(x[10], x[11]), sk_pair(x[18], x[19]), sk_pair(x[26], x[27])};
    o[2] = uint4{sk_pair(x[4], x[5]), sk_pair(x[12], x[13]), sk_pair(x[20], x[21]), sk_pair(x[28], x[29])};
    o[3] = uint4{sk_pair(x[6], x[7]), sk_pair(x[14], x[15]), sk_pair(x[22], x[23]), sk_pair(x[30], x[31])};
}

__device__ __forceinline__ uint64_t sk_pack2(float lo, float hi)
{
    return (uint64_t)__builtin_bit_cast(uint32_t, lo) | ((uint64_t)__builtin_bit_cast(uint32_t, hi) << 32);
}

// The lane's K words of a chunk (4-byte aligned, widest loads).
template <int K>
__device__ __forceinline__ void sk_load(uint32_t (&w)[K + 1], const uint32_t* __restrict__ p, bool ok)
{
    typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    if (!ok) {
#pragma unroll
        for (int i = 1; i <= K; i++) w[i] = 0u;
        return;
    }
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

template <int K, int CB>
__global__ __launch_bounds__(64 * SK_WAVES) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_sk_kernel(const SkArgs a)
{
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    _Float16* As = reinterpret_cast<_Float16*>(lds);
    _Float16* Bs = As + SK_BM * SK_LD;

    const int g = blockIdx.x;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int wm = wave >> 2, wn = wave & 3;
    const int tc = a.oc >> 4;                 // tile columns of W_q
    const Dot2Consts kc = dot2_consts();

    // A-tile loader: thread t moves 16 bytes of rows 64 p + t / 8, p = 0..3, segment t % 8.
    const int arow = tid >> 3, aseg = tid & 7;
    // B chunk of this thread: chunk id tid = 8 * tile + c, tile = 16 ti_l + tn_l (a tile's
    // 8 chunks on 8 consecutive lanes)
    const int c = lane & 7;
    const bool first_lane = c == 0;
    const int btile = tid >> 3;
    const int bn0 = 16 * (btile & 15) + c, bk0 = 16 * (btile >> 4);

    f32x4 acc[8][4];
    uint4 areg[4];
    uint32_t w[K + 1];

    const long u_begin = sk_first(a, g), u_end = sk_first(a, g + 1);
    long u = u_begin;
    while (u < u_end) {
        const int t = (int)(u / a.nks);
        const int s0 = (int)(u - (long)t * a.nks);
        const int s1 = (int)min((long)a.nks, s0 + (u_end - u));
        const int tm = t / a.ntn, tn = t - tm * a.ntn;
        const int m0 = tm * SK_BM;
        const int btn = 16 * tn + (btile & 15);
        const bool bok = btn < tc;

        auto load_step = [&](int s) {
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const int row = m0 + 64 * p + arow;
                areg[p] = row < a.rows
                    ? *reinterpret_cast<const uint4*>(a.Ah + (long)row * a.ic + s * SK_KS + aseg * 8)
                    : uint4{0u, 0u, 0u, 0u};
            }
            const int ti = 4 * s + (btile >> 4);
            sk_load<K>(w, a.trellis + ((long)ti * tc + (bok ? btn : 0)) * (8 * K) + c * K, bok);
        };
        auto store_step = [&]() {
#pragma unroll
            for (int p = 0; p < 4; p++)
                *reinterpret_cast<uint4*>(As + (64 * p + arow) * SK_LD + aseg * 8) = areg[p];
            chunk_prev_dpp<K>(w, first_lane);
            uint4 o[4];
            sk_decode<K, CB>(w, kc, o);
            *reinterpret_cast<uint4*>(Bs + bn0 * SK_LD + bk0) = o[0];
            *reinterpret_cast<uint4*>(Bs + bn0 * SK_LD + bk0 + 8) = o[1];
            *reinterpret_cast<uint4*>(Bs + (bn0 + 8) * SK_LD + bk0) = o[2];
            *reinterpret_cast<uint4*>(Bs + (bn0 + 8) * SK_LD + bk0 + 8) = o[3];
        };

#pragma unroll
        for (int mb = 0; mb < 8; mb++)
#pragma unroll
            for (int nb = 0; nb < 4; nb++) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

        load_step(s0);
        for (int s = s0; s < s1; s++) {
            __syncthreads();                  // the previous step's MFMAs are done with LDS
            store_step();
            __syncthreads();
            if (s + 1 < s1) load_step(s + 1);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                f16x8 bf[4];
#pragma unroll
                for (int nb = 0; nb < 4; nb++)
                    bf[nb] = *reinterpret_cast<const f16x8*>(Bs + (64 * wn + 16 * nb + (lane & 15)) * SK_LD + 32 * h +
                                                             8 * (lane >> 4));
#pragma unroll
                for (int mb = 0; mb < 8; mb++) {
                    const f16x8 af = *reinterpret_cast<const f16x8*>(As + (128 * wm + 16 * mb + (lane & 15)) * SK_LD +
                                                                     32 * h + 8 * (lane >> 4));
#pragma unroll
                    for (int nb = 0; nb < 4; nb++) acc[mb][nb] = mfma16x16x32(af, bf[nb], acc[mb][nb]);
                }
            }
        }
        u += s1 - s0;

        // ---- finish: a whole tile here, a piece through the slots
        bool finish = s0 == 0 && s1 == a.nks;
        if (!finish) {
            const int g_lo = sk_wg_of(a, (long)t * a.nks), g_hi = sk_wg_of(a, (long)(t + 1) * a.nks - 1);
            uint64_t* my = reinterpret_cast<uint64_t*>(a.slots + ((long)(t + g) * SK_WAVES + wave) * SK_ACC * 64) + lane;
#pragma unroll
            for (int mb = 0; mb < 8; mb++)
#pragma unroll
                for (int nb = 0; nb < 4; nb++) {
                    const f32x4 v = acc[mb][nb];
                    __hip_atomic_store(my + (long)((mb * 4 + nb) * 2) * 64, sk_pack2(v.x, v.y), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(my + (long)((mb * 4 + nb) * 2 + 1) * 64, sk_pack2(v.z, v.w), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                }
            __builtin_amdgcn_s_waitcnt(0);   // this wave's slot stores are complete
            __syncthreads();                  // ... and every wave's
            if (tid == 0) {
                const uint32_t old = __hip_atomic_fetch_add(a.counters + t, 1u, __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT);
                lds[0] = old == (uint32_t)(g_hi - g_lo) ? 1u : 0u;
            }
            __syncthreads();
            finish = lds[0] != 0u;
            __syncthreads();                  // lds[0] read by all before LDS is reused
            if (finish) {
                // last to arrive: every contributor's stores completed before its increment
#pragma unroll
                for (int mb = 0; mb < 8; mb++)
#pragma unroll
                    for (int nb = 0; nb < 4; nb++) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
                for (int gg = g_lo; gg <= g_hi; gg++) {
                    const uint64_t* sl =
                        reinterpret_cast<const uint64_t*>(a.slots + ((long)(t + gg) * SK_WAVES + wave) * SK_ACC * 64) + lane;
#pragma unroll
                    for (int mb = 0; mb < 8; mb++)
#pragma unroll
                        for (int nb = 0; nb < 4; nb++) {
                            const uint64_t p = __hip_atomic_load(sl + (long)((mb * 4 + nb) * 2) * 64, __ATOMIC_RELAXED,
                                                                 __HIP_MEMORY_SCOPE_AGENT);
                            const uint64_t q = __hip_atomic_load(sl + (long)((mb * 4 + nb) * 2 + 1) * 64,
                                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            acc[mb][nb] += f32x4{__builtin_bit_cast(float, (uint32_t)p),
                                                 __builtin_bit_cast(float, (uint32_t)(p >> 32)),
                                                 __builtin_bit_cast(float, (uint32_t)q),
                                                 __builtin_bit_cast(float, (uint32_t)(q >> 32))};
                        }
                }
            }
        }
        if (finish) {
            // Output block ob (128 outputs) of rows 128 wm ..: waves wn = 2 ob' and 2 ob' + 1 hold
            // its two 64-column halves.  16 rows at a time through LDS (16 x 132 floats per block
            // and row half), then wave (wn & 1) transforms rows 8 (wn & 1) .. + 7: FWHT, * svh,
            // fp16 store.
            const int blk = wn >> 1, half = wn & 1;
            float* cs = reinterpret_cast<float*>(lds) + (wm * 2 + blk) * 16 * SK_CLD;
            const int ob = 16 * tn + 8 * blk;         // tile column of the block's first output
            const bool col_ok = ob < tc;
            const uint32_t sv = col_ok ? reinterpret_cast<const uint32_t*>(a.svh + ob * 16)[lane] : 0u;
            const float sv0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(sv & 0xffffu));
            const float sv1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(sv >> 16));
            __syncthreads();                  // every wave is done with the A/B tiles
            for (int mb = 0; mb < 8; mb++) {
#pragma unroll
                for (int nb = 0; nb < 4; nb++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        cs[(4 * (lane >> 4) + e) * SK_CLD + 64 * half + 16 * nb + (lane & 15)] = acc[mb][nb][e];
                __syncthreads();
                for (int r = 8 * half; r < 8 * half + 8; r++) {
                    float v0 = cs[r * SK_CLD + 2 * lane], v1 = cs[r * SK_CLD + 2 * lane + 1];
                    wave_fwht128(v0, v1);
                    const int row = m0 + 128 * wm + 16 * mb + r;
                    if (col_ok && row < a.rows) {
                        const uint32_t o = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(v0 * sv0)) |
                                           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(v1 * sv1)) << 16);
                        reinterpret_cast<uint32_t*>(a.C + (long)row * a.oc + ob * 16)[lane] = o;
                    }
                }
                __syncthreads();
            }
        }
        __syncthreads();                      // LDS is free for the next piece
    }
}

// ---------------------------------------------------------------- host side

size_t gemm_sk_slot_bytes(int rows, int oc, int G)
{
    const long tiles = (long)((rows + SK_BM - 1) / SK_BM) * ((oc + SK_BN - 1) / SK_BN);
    return ((size_t)tiles * 4 + 255) / 256 * 256 + (size_t)(tiles + G) * SK_WAVES * SK_ACC * 64 * sizeof(float);
}

int gemm_sk_cus()
{
    int dev = 0, cus = 0;
    hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    return cus;
}

template <int K, int CB>
static const void* sk_fn() { return reinterpret_cast<const void*>(&gemm_sk_kernel<K, CB>); }

int gemm_sk_dispatch(const uint16_t* Ah, const uint32_t* trellis, uint16_t* C, const uint16_t* svh, char* ws,
                     size_t ws_bytes, int rows, int ic, int oc, int K, int cb, int G, hipStream_t stream)
{
    SkArgs a = {};
    a.Ah = Ah;
    a.trellis = trellis;
    a.C = C;
    a.svh = svh;
    a.rows = rows;
    a.ic = ic;
    a.oc = oc;
    a.ntn = (oc + SK_BN - 1) / SK_BN;
    a.nks = ic / SK_KS;
    a.ntiles = ((rows + SK_BM - 1) / SK_BM) * a.ntn;
    const long units = (long)a.ntiles * a.nks;
    // at least 16 K-steps per workgroup: a tile has at most nks / 16 + 2 contributors
    if (G > units / 16) G = (int)std::max<long>(1, units / 16);
    const size_t cbytes = ((size_t)a.ntiles * 4 + 255) / 256 * 256;
    // fewer workgroups when the workspace was sized on a device with fewer CUs
    const size_t slot = (size_t)SK_WAVES * SK_ACC * 64 * sizeof(float);
    const long fit = ws_bytes > cbytes ? (long)((ws_bytes - cbytes) / slot) - a.ntiles : 0;
    if (fit < 1)
        return set_error(EXL3_ERR_WORKSPACE, "exl3_gemm: workspace of %zu bytes, %zu needed", ws_bytes,
                         gemm_sk_slot_bytes(rows, oc, G));
    if (G > fit) G = (int)fit;
    a.q = (int)(units / G);
    a.r = (int)(units % G);
    a.counters = reinterpret_cast<uint32_t*>(ws);
    a.slots = reinterpret_cast<float*>(ws + cbytes);
    hipLaunchKernelGGL(sk_clear_kernel, dim3((a.ntiles + 255) / 256), dim3(256), 0, stream, a.counters, a.ntiles);
    int rc = check_launch("exl3_gemm (counters)");
    if (rc != EXL3_OK) return rc;
    const void* fn = nullptr;
#define EXL3_CASE(KK) case KK: fn = cb == CB_MCG ? sk_fn<KK, CB_MCG>() : sk_fn<KK, CB_3INST>(); break;
    switch (K) {
        EXL3_CASE(1) EXL3_CASE(2) EXL3_CASE(3) EXL3_CASE(4)
        EXL3_CASE(5) EXL3_CASE(6) EXL3_CASE(7) EXL3_CASE(8)
        default: return set_error(EXL3_ERR_ARG, "exl3_gemm: K=%d is not in 1..8", K);
    }
#undef EXL3_CASE
    hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, SK_LDS);
    (void)hipGetLastError();
    void* kargs[] = {&a};
    hipLaunchKernel(fn, dim3(G), dim3(64 * SK_WAVES), kargs, SK_LDS, stream);
    return check_launch("exl3_gemm (stream-K)");
}

}  // namespace exl3
