// EXL3 GEMM, stream-K over BM x 256 output tiles (BM = 32, 48, 64, 96, 128 or 256 by row count):
//   C = fp16( H( Ah . W_q ) * svh ),  Ah = fp16(H(A * suh)) (a had_r_128 pass)
// W_q is decoded from the packed trellis straight into LDS (never written to HBM), once per
// BM-row tile, and multiplied with v_mfma_f32_16x16x32_f16.  Replaces the reconstruct
// branch of orcasaq2/ops.py:50-59 (reconstruct -> hgemm_recon -> had_r_128) for many rows,
// and the fused exl3_gemm of orcasaq2/ops.py:46-49 for 17..GEMM_MAX_ROWS rows.
//
// Work decomposition.  Output tiles are BM rows x 256 outputs (two output Hadamard blocks);
// a tile is nks = ic / 64 K-steps of 64 inputs.  The tiles' K-steps (all shards of a launch,
// shard-major, then tile, then K-step) are cut into G nearly equal contiguous ranges, one
// per workgroup ("stream-K"): every workgroup does the same number of K-steps whatever the
// tile count.  A range covers a few tile pieces.  A piece that is a whole tile is finished
// by its workgroup; a partial piece leaves its fp32 accumulators in a slot of the
// workspace, and the last of the tile's workgroups to arrive (an agent-scope counter per
// tile) adds the slots in workgroup order -- deterministic -- and finishes the tile.
//
// Per workgroup (8 waves; BM = 256: wave w owns rows 128 (w / 4) .., outputs 64 (w % 4) ..,
// 8 x 4 MFMA blocks; BM = 32..128: wave w owns all rows and outputs 32 w .., BM/16 x 2
// blocks) and K-step:
//   * the A tile (BM x 64 fp16) is loaded into registers one K-step ahead, then stored to
//     LDS rows of 72 halves (16-byte reads of 16 consecutive rows hit distinct banks);
//   * the B tile is 4 tile rows x 16 tile columns = 512 chunks of 32 positions, one per
//     lane: its K words are loaded one K-step ahead, the tail-biting word comes by DPP from
//     the neighbouring lane, each masked word's fp16 halves are summed (the reconstruct
//     rounding) and the chunk's two output columns' 16 inputs go to LDS as [output][input];
//   * LDS reads of 16 bytes feed the MFMAs.
// Epilogue per 128-output block: rows through LDS, FWHT across a wave, * svh, fp16 store.
#include "exl3_common.h"
#include "gemm_sk_plan.h"

#include <stdlib.h>

namespace exl3 {

// Set-up of a grouped launch (SkPrepArgs): the tile counters to zero and, for every shard,
// its activations Ah = fp16(H128(A * suh)), one wave per (shard, row, 128-input block).
__global__ __launch_bounds__(256) void sk_prep_kernel(const SkPrepArgs a)
{
    const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (w < a.ntiles && lane == 0) a.counters[w] = 0u;
    if (w >= a.nsh * a.rows * a.nblk) return;   // whole waves only
    int s, r, b;
    sk_prep_wave(a, w, s, r, b);
    const long off = sk_prep_elem(a, r, b);
    const uint32_t xw = reinterpret_cast<const uint32_t*>(a.A + off)[lane];
    const uint32_t sw = reinterpret_cast<const uint32_t*>(a.suh[s] + b * 128)[lane];
    float v0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(xw & 0xffffu)) *
               (float)__builtin_bit_cast(_Float16, (uint16_t)(sw & 0xffffu));
    float v1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(xw >> 16)) *
               (float)__builtin_bit_cast(_Float16, (uint16_t)(sw >> 16));
    wave_fwht128(v0, v1);
    reinterpret_cast<uint32_t*>(a.Ah[s] + off)[lane] =
        (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v0) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v1) << 16);
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

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also waits for this
// wave's global stores to complete (a workgroup-scope release), which in the epilogue's
// store loop put a store round trip into every row block.
__device__ __forceinline__ void sk_lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The end of a tile piece: a whole tile is finished by its workgroup; a partial piece leaves
// its accumulators in the workgroup's slot, and the last of the tile's workgroups to arrive
// (an agent-scope counter per tile) adds the slots in workgroup order -- deterministic --
// and finishes the tile.  Epilogue per 128-output block: rows through LDS, FWHT across a
// wave, * svh, fp16 store.  RBCOL: the accumulators hold the register-B kernel's output
// columns (sk_rb_wcol) instead of 16 consecutive outputs per block.
template <int BM, bool RBCOL>
__device__ __forceinline__ void sk_finish_piece(const SkArgs& a, const SkPiece& pc, const SkShard& S, int g, int wave,
                                                int lane, int tid, int wm, int wn,
                                                f32x4 (&acc)[SkCfg<BM>::MB][SkCfg<BM>::NB], uint32_t* lds)
{
    constexpr int MB = SkCfg<BM>::MB, NB = SkCfg<BM>::NB;
    const int t = pc.t, s0 = pc.s0, s1 = pc.s1, tn = pc.tn, m0 = pc.m0, tc = pc.tc;
    // ---- finish: a whole tile here, a piece through the slots
    bool finish = s0 == 0 && s1 == a.nks;
    if (!finish) {
        const int g_lo = sk_wg_of(a, (long)t * a.nks), g_hi = sk_wg_of(a, (long)(t + 1) * a.nks - 1);
        uint64_t* my = reinterpret_cast<uint64_t*>(a.slots + sk_slot<BM>(t, g, wave)) + lane;
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                const f32x4 v = acc[mb][nb];
                __hip_atomic_store(my + (long)((mb * NB + nb) * 2) * 64, sk_pack2(v.x, v.y), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(my + (long)((mb * NB + nb) * 2 + 1) * 64, sk_pack2(v.z, v.w), __ATOMIC_RELAXED,
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
            for (int mb = 0; mb < MB; mb++)
#pragma unroll
                for (int nb = 0; nb < NB; nb++) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
            // Slots in workgroup order, each read in batches of SK_RB 8-byte loads per lane
            // that are all issued before the first add (atomic loads keep program order,
            // so loads interleaved with the adds would have two in flight at a time).
            constexpr int NP = MB * NB * 2;                   // 8-byte words per lane and slot
            constexpr int RB = NP < 16 ? NP : 16;
            for (int gg = g_lo; gg <= g_hi; gg++) {
                const uint64_t* sl =
                    reinterpret_cast<const uint64_t*>(a.slots + sk_slot<BM>(t, gg, wave)) + lane;
#pragma unroll
                for (int b0 = 0; b0 < NP; b0 += RB) {
                    uint64_t v[RB];
#pragma unroll
                    for (int i = 0; i < RB; i++)
                        v[i] = __hip_atomic_load(sl + (long)(b0 + i) * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                    for (int i = 0; i < RB; i += 2) {
                        const int blk = (b0 + i) >> 1, mb = blk / NB, nb = blk % NB;
                        acc[mb][nb] += f32x4{__builtin_bit_cast(float, (uint32_t)v[i]),
                                             __builtin_bit_cast(float, (uint32_t)(v[i] >> 32)),
                                             __builtin_bit_cast(float, (uint32_t)v[i + 1]),
                                             __builtin_bit_cast(float, (uint32_t)(v[i + 1] >> 32))};
                    }
                }
            }
        }
    }
    if (finish) {
        // in registers: the LDS barriers below clobber memory, which would reload these
        uint16_t* const Cp = S.C;
        const long ldc = S.ldc;
        const int rows = a.rows;
        // svh pair of this lane in the 128-output block starting at tile column ob, read
        // once per block: the fp16 output stores could alias it, so a load inside the
        // row loop would be repeated (a round trip per row)
        auto load_sv = [&](int ob) -> uint32_t {
            return ob < tc ? reinterpret_cast<const uint32_t*>(S.svh + ob * 16)[lane] : 0u;
        };
        int lane_v = lane;
        asm volatile("" : "+v"(lane_v));   // the signs stay out of the main loop
        const FwhtSigns fs = fwht_signs(lane_v);
        // The block's svh pair as floats, converted once: a conversion left inside the store
        // loop waits there for the load, and so for every store issued before it.
        struct Sv {
            float s0, s1;
        };
        auto load_svf = [&](int ob) -> Sv {
            const uint32_t sv = load_sv(ob);
            Sv r{(float)__builtin_bit_cast(_Float16, (uint16_t)(sv & 0xffffu)),
                 (float)__builtin_bit_cast(_Float16, (uint16_t)(sv >> 16))};
            asm volatile("" : "+v"(r.s0), "+v"(r.s1));
            return r;
        };
        auto store_row = [&](int row, int ob, const Sv& sv, float v0, float v1) {
            // ob: tile column of the 128-output block's first output; v0, v1 transformed
            if (ob < tc && row < rows) {
                const float sv0 = sv.s0, sv1 = sv.s1;
                const uint32_t o = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(v0 * sv0)) |
                                   ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(v1 * sv1)) << 16);
                reinterpret_cast<uint32_t*>(Cp + (long)row * ldc + ob * 16)[lane] = o;
            }
        };
        __syncthreads();                  // every wave is done with the A/B tiles
        if constexpr (BM == 256) {
            // Output block of rows 128 wm ..: waves wn = 2 blk and 2 blk + 1 hold its two
            // 64-column halves.  16 rows at a time through LDS (16 x 132 floats per block
            // and row half), then wave (wn & 1) transforms rows 8 (wn & 1) .. + 7.
            const int blk = wn >> 1, half = wn & 1;
            const Sv sv = load_svf(16 * tn + 8 * blk);
            float* cs = reinterpret_cast<float*>(lds) + sk_c256(wm, blk, 0, 0);
#pragma unroll
            for (int mb = 0; mb < MB; mb++) {
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        cs[sk_c256(0, 0, 4 * (lane >> 4) + e, 64 * half + (RBCOL ? sk_rb_wcol(nb, lane) : 16 * nb + (lane & 15)))] =
                                acc[mb][nb][e];
                sk_lds_barrier();
                float v0[8], v1[8];                // eight independent transforms
#pragma unroll
                for (int r = 0; r < 8; r++) {
                    v0[r] = cs[sk_c256(0, 0, 8 * half + r, 2 * lane)];
                    v1[r] = cs[sk_c256(0, 0, 8 * half + r, 2 * lane + 1)];
                }
                wave_fwht128_n<8>(v0, v1, fs);
#pragma unroll
                for (int r = 0; r < 8; r++)
                    store_row(m0 + 128 * wm + 16 * mb + 8 * half + r, 16 * tn + 8 * blk, sv, v0[r], v1[r]);
                sk_lds_barrier();
            }
        } else {
            // 16 rows at a time through LDS (16 rows of 260 floats); wave w transforms the
            // chunk's (row, block) pairs w, w + 8, w + 16, w + 24
            float* cs = reinterpret_cast<float*>(lds);
            const Sv sv[2] = {load_svf(16 * tn), load_svf(16 * tn + 8)};
#pragma unroll
            for (int mb = 0; mb < MB; mb++) {
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        cs[sk_cx(4 * (lane >> 4) + e, NB * 16 * wn + 16 * nb + (lane & 15))] = acc[mb][nb][e];
                sk_lds_barrier();
                float v0[4], v1[4];                // four independent transforms
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const int j = wave + SK_WAVES * jj;
                    const int r = j & 15, blk = j >> 4;
                    v0[jj] = cs[sk_cx(r, 128 * blk + 2 * lane)];
                    v1[jj] = cs[sk_cx(r, 128 * blk + 2 * lane + 1)];
                }
                wave_fwht128_n<4>(v0, v1, fs);
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const int j = wave + SK_WAVES * jj;
                    const int r = j & 15, blk = j >> 4;
                    store_row(m0 + 16 * mb + r, 16 * tn + 8 * blk, sv[blk], v0[jj], v1[jj]);
                }
                if (mb + 1 < MB) sk_lds_barrier();
            }
        }
    }
    sk_lds_barrier();                     // LDS is free for the next piece
}

// K > 0: every shard of the launch has K bits per weight; K = 0: each tile piece takes its
// shard's K (one launch for shards of different bit widths).
template <int K, int CB, int BM>
__global__ __launch_bounds__(64 * SK_WAVES) __attribute__((amdgpu_waves_per_eu(SK_WPE, SK_WPE)))
void gemm_sk_kernel(const SkArgs a)
{
    using Cfg = SkCfg<BM>;
    constexpr int MB = Cfg::MB, NB = Cfg::NB;
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    auto As = [&](int b) { return reinterpret_cast<_Float16*>(lds) + sk_as<BM>(b); };
    auto Bs = [&](int b) { return reinterpret_cast<_Float16*>(lds) + sk_bs<BM>(b); };

    const int g = sk_logical(blockIdx.x, gridDim.x);
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
    const Dot2Consts kc = dot2_consts();

    // A-tile loader: thread t moves 16 bytes of row t / 8 (+ 64 p), segment t % 8.
    const int arow = sk_arow(tid), aseg = sk_aseg(tid);
    constexpr int AP = (BM + 63) / 64;               // passes; pass p moves rows 64 p + arow < BM
    auto aload = [&](int p) { return sk_apass<BM>(p, arow); };
    // B chunk of this thread (sk_b_word): a tile's 8 chunks on 8 consecutive lanes
    const int c = lane & 7;
    const bool first_lane = c == 0;
    const int bn0 = sk_bn0(tid), bk0 = sk_bk0(tid);

    f32x4 acc[MB][NB];
    uint4 areg[AP];

    const long u_begin = sk_first(a, g), u_end = sk_first(a, g + 1);
    long u = u_begin;
    while (u < u_end) {
        const SkPiece pc = sk_piece<BM>(a, u, u_end);
        const int t = pc.t, s0 = pc.s0, s1 = pc.s1;
        const SkShard& S = a.sh[pc.si];
        const int tn = pc.tn, m0 = pc.m0;
        const int tc = pc.tc;                        // tile columns of W_q
        const int btn = sk_btn(tid, tn);
        const bool bok = btn < tc;

#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int nb = 0; nb < NB; nb++) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
        // the piece's K-steps, for KK bits per weight
        auto run_piece = [&](auto kk) {
            constexpr int KK = decltype(kk)::value;
            uint32_t w[KK + 1];
            auto load_step = [&](int s) {
#pragma unroll
                for (int p = 0; p < AP; p++) {
                    const int row = m0 + 64 * p + arow;
                    areg[p] = (aload(p) && row < a.rows)
                        ? *reinterpret_cast<const uint4*>(S.Ah + sk_a_elem(a, row, s, aseg))
                        : uint4{0u, 0u, 0u, 0u};
                }
                sk_load<KK>(w, S.trellis + sk_b_word(sk_bti(tid, s), tc, sk_bcol(btn, tc), c, KK), bok);
            };
            // the registers of a K-step into LDS buffer b: A as loaded, B decoded
            auto store_step = [&](int b) {
                _Float16* as = As(b);
                _Float16* bs = Bs(b);
#pragma unroll
                for (int p = 0; p < AP; p++)
                    if (aload(p)) *reinterpret_cast<uint4*>(as + sk_a_store(p, arow, aseg)) = areg[p];
                chunk_prev_dpp<KK>(w, first_lane);
                uint4 o[4];
                sk_decode<KK, CB>(w, kc, o);
#pragma unroll
                for (int j = 0; j < 4; j++) *reinterpret_cast<uint4*>(bs + sk_b_store(bn0, bk0, j)) = o[j];
            };
            // the MFMAs of one K-step from LDS buffer b
            auto mfma_step = [&](int b) {
                const _Float16* as = As(b);
                const _Float16* bs = Bs(b);
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    f16x8 bf[NB];
#pragma unroll
                    for (int nb = 0; nb < NB; nb++)
                        bf[nb] = *reinterpret_cast<const f16x8*>(bs + sk_b_frag<BM>(wn, nb, lane, h));
#pragma unroll
                    for (int mb = 0; mb < MB; mb++) {
                        const f16x8 af = *reinterpret_cast<const f16x8*>(as + sk_a_frag<BM>(wm, mb, lane, h));
#pragma unroll
                        for (int nb = 0; nb < NB; nb++) acc[mb][nb] = mfma16x16x32(af, bf[nb], acc[mb][nb]);
                    }
                }
            };


            // Software pipeline over two LDS buffers, one barrier per K-step: during step s the
            // MFMAs read buffer (s - s0) % 2 while the step s + 1 tiles (loaded into registers a
            // step earlier) are decoded into the other buffer and step s + 2 is loaded.  The step
            // is one basic block (the last steps re-decode and re-load in-bounds data that is
            // never read), so the scheduler can issue the decode's VALU work between the MFMAs,
            // which run on the matrix pipe meanwhile.
            load_step(s0);
            store_step(0);
            load_step(min(s0 + 1, s1 - 1));
            __syncthreads();
            if (wave < SK_WAVES / 2) {
                for (int s = s0; s < s1; s++) {
                    const int b = (s - s0) & 1;
                    mfma_step(b);
                    store_step(b ^ 1);
                    load_step(min(s + 2, s1 - 1));
                    __syncthreads();          // buffer b ^ 1 is complete; buffer b is free
                }
            } else {
                for (int s = s0; s < s1; s++) {
                    const int b = (s - s0) & 1;
                    store_step(b ^ 1);
                    load_step(min(s + 2, s1 - 1));
                    mfma_step(b);
                    __syncthreads();          // buffer b ^ 1 is complete; buffer b is free
                }
            }
        };
        if constexpr (K > 0) {
            run_piece(std::integral_constant<int, K>{});
        } else {
            switch (S.K) {
            case 1: run_piece(std::integral_constant<int, 1>{}); break;
            case 2: run_piece(std::integral_constant<int, 2>{}); break;
            case 3: run_piece(std::integral_constant<int, 3>{}); break;
            case 4: run_piece(std::integral_constant<int, 4>{}); break;
            case 5: run_piece(std::integral_constant<int, 5>{}); break;
            case 6: run_piece(std::integral_constant<int, 6>{}); break;
            case 7: run_piece(std::integral_constant<int, 7>{}); break;
            default: run_piece(std::integral_constant<int, 8>{}); break;
            }
        }
        u += s1 - s0;

        sk_finish_piece<BM, false>(a, pc, S, g, wave, lane, tid, wm, wn, acc, lds);
    }
}

// ---------------------------------------------------------------- 256-row tiles, B in registers
//
// The same stream-K ranges, pieces, slots and epilogue as gemm_sk_kernel<K, CB, 256>; only the
// K-step differs.  The B tile is never stored whole to LDS: each lane decodes one chunk per
// K-step (sk_rb_*), and the chunk's four 8-row fragments are MFMA B operands straight from
// its registers -- the MFMA's four k-groups take four tile rows, so a lane's chunk lines up
// with its own operand slots.  The two waves that share a wave's outputs (rows 0-127 and
// 128-255 of the same 64 outputs) split the decode: each decodes one of the two chunk groups
// and hands its fragments to the other through a 32 KiB LDS exchange buffer (one 16-byte
// store and one load per fragment), so every weight is decoded once per workgroup.  The
// decode of the next K-step runs between the current step's MFMAs, one weight pair per
// group of four MFMAs.  A reaches LDS by direct-to-LDS loads (no registers, no LDS store
// instructions) two K-steps ahead, in three buffers.

// A masked codebook word with the multiply-add in plain code for states off a half-word
// boundary: the compiler schedules and renames it freely (v_mul_lo_u32 + v_add_u32), where
// the single-instruction v_mad_u64_u32 form -- inline assembly with a 64-bit result -- left
// this kernel's register allocation spilling.
template <int K, int CB, int Q>
__device__ __forceinline__ uint32_t rb_word(const uint32_t (&w)[K + 1], const Dot2Consts& k)
{
    using P = StatePlan<K, Q>;
    uint32_t x;
    if constexpr (P::kind <= 1) {
        x = dot2_raw<K, CB, Q>(w, k);
    } else {
        const uint32_t st = state_field<K, Q>(w);
        x = CB == CB_MCG ? st * CBMCG_MUL : st * k.mul + CB3_ADD;   // k.mul: the multiplier in a VGPR
    }
    return (x & k.mask) ^ k.flip;
}

// One 8-row fragment of a chunk as fp16 weights (the reconstruct rounding) in input order:
// positions q0 + 8m + {0, 1}, m = 0..3 -- q0 = 0: column c rows 0..7, 2: column c rows 8..15,
// 4: column c + 8 rows 0..7, 6: column c + 8 rows 8..15 (sk_decode's o[q0 / 2]).
template <int K, int CB, int Q0>
__device__ __forceinline__ uint4 rb_frag(const uint32_t (&w)[K + 1], const Dot2Consts& kc)
{
    return uint4{sk_pair(rb_word<K, CB, Q0>(w, kc), rb_word<K, CB, Q0 + 1>(w, kc)),
                 sk_pair(rb_word<K, CB, Q0 + 8>(w, kc), rb_word<K, CB, Q0 + 9>(w, kc)),
                 sk_pair(rb_word<K, CB, Q0 + 16>(w, kc), rb_word<K, CB, Q0 + 17>(w, kc)),
                 sk_pair(rb_word<K, CB, Q0 + 24>(w, kc), rb_word<K, CB, Q0 + 25>(w, kc))};
}

// The lane's K words of a chunk, always loaded: every wave issues the same number of loads
// per step, which the step-end waits count on.  A column past the shard reads column 0's
// words (sk_bcol) and is left as loaded -- its 128-output block lies wholly past the shard
// and is never stored -- so nothing consumes the loaded registers before the decode does.
template <int K>
__device__ __forceinline__ void rb_load(uint32_t (&w)[K + 1], const uint32_t* __restrict__ p)
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

// f(integral_constant<int, I>) for I = B .. E - 1, in order.
template <int B, int E, class F>
__device__ __forceinline__ void rb_static_for(F&& f)
{
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        rb_static_for<B + 1, E>(f);
    }
}

// s_waitcnt until at most v vector-memory operations are outstanding (gfx9 encoding; no wait
// on the export and LDS/scalar counters).
constexpr int rb_vmcnt(int v) { return (v & 15) | ((v >> 4) << 14) | (7 << 4) | (15 << 8); }

template <int K, int CB>
__global__ __launch_bounds__(64 * SK_WAVES) __attribute__((amdgpu_waves_per_eu(SK_WPE, SK_WPE)))
void gemm_rb_kernel(const SkArgs a)
{
    constexpr int BM = 256, MB = SkCfg<BM>::MB, NB = SkCfg<BM>::NB;
    static_assert(NB == 4 && MB == 8 && SkCfg<BM>::WN == 4, "two chunk groups x two column halves per wave");
    constexpr int NBL = K / 4 + (K % 4 ? 1 : 0);   // B load instructions per step
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    auto As = [&](int b) { return reinterpret_cast<const _Float16*>(lds) + sk_rb_as(b); };
    uint4* const bx = reinterpret_cast<uint4*>(lds) + sk_rb_bx_base();

    const int g = sk_logical(blockIdx.x, gridDim.x);
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int wm = wave / SkCfg<BM>::WN, wn = wave % SkCfg<BM>::WN;
    const int partner = sk_rb_partner(wave);
    const Dot2Consts kc = dot2_consts();
    const int c = lane & 7;
    const bool first_lane = c == 0;

    // acc[mb][2 h + ch]: h = 0 the wave's own chunk group (g = wm), h = 1 its partner's
    f32x4 acc[MB][NB];

    const uint32_t lds_base = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(void __attribute__((address_space(3)))*)lds);
    const long u_begin = sk_first(a, g), u_end = sk_first(a, g + 1);
    long u = u_begin;
    while (u < u_end) {
        const SkPiece pc = sk_piece<BM>(a, u, u_end);
        const int s0 = pc.s0, s1 = pc.s1;
        const SkShard& S = a.sh[pc.si];
        const int m0 = pc.m0, tc = pc.tc;
        const int bcol = sk_bcol(sk_rb_btn(lane, pc.tn, wn, wm), tc);
        // in registers: the assembly loads below clobber memory, which would reload these
        const uint16_t* const Ah = S.Ah;
        const uint32_t* const Bt = S.trellis;
        const int last_row = a.rows - 1;
        const long ic = a.ic;
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int nb = 0; nb < NB; nb++) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

        // Direct-to-LDS load of A(s) into buffer b: 4 passes, this wave's 8 rows each (rows past
        // the call's read the last row: in bounds, and their outputs are never stored).  Issued
        // as inline assembly, so the compiler's wait insertion does not see these loads: it
        // would otherwise wait for every direct-to-LDS load before any later LDS read (it
        // cannot tell the buffers apart) -- the step-end waits order them instead.
        auto dma_a = [&](int s, int b) {
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const int r = sk_rb_dma_row(p, wave, lane);
                const int row = min(m0 + r, last_row);
                const uint16_t* src = Ah + (long)row * ic + s * SK_KS + 8 * sk_rb_dma_chunk(p, wave, lane);
                const uint32_t dst = lds_base + 2u * (uint32_t)(sk_rb_as(b) + (64 * p + 8 * wave) * SK_KS);
                asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(dst)
                             : "memory", "m0");
            }
        };
        auto run_piece = [&](auto kk) {
            constexpr int KK = decltype(kk)::value;
            uint32_t wc[KK + 1], wx[KK + 1];     // words of the chunk decoded this step, of the next
            uint4 own[4], nown[4], pf[4];        // fragment f = 2 ch + rh
            auto load_b = [&](uint32_t (&w)[KK + 1], int s) {
                rb_load<KK>(w, Bt + sk_b_word(sk_rb_bti(lane, s), tc, bcol, c, KK));
            };
            auto decode_put = [&](uint32_t (&w)[KK + 1], uint4 (&o)[4], int b) {
                chunk_prev_dpp<KK>(w, first_lane);
                o[0] = rb_frag<KK, CB, 0>(w, kc);
                o[1] = rb_frag<KK, CB, 2>(w, kc);
                o[2] = rb_frag<KK, CB, 4>(w, kc);
                o[3] = rb_frag<KK, CB, 6>(w, kc);
#pragma unroll
                for (int f = 0; f < 4; f++) bx[sk_rb_bx(b, wave, f, lane)] = o[f];
            };
            // One K-step's MFMAs on A buffer b3 and fragments own / pf, with the decode of the
            // next step's own fragments (from wc, stored to B buffer bo) spread between them:
            // 16 MFMA groups (row half rh outer, row block mb inner: an accumulator's next
            // MFMA comes 32 MFMAs later), each of 4 MFMAs, one A-fragment read two groups
            // ahead, and one weight pair of the decode; a fragment is stored every 4 groups.
            // The order is fixed by scheduling barriers between groups.
            auto step_body = [&](int b3, int bo) {
                const _Float16* as = As(b3);
                auto frag = [&](int i) {
                    return *reinterpret_cast<const f16x8*>(as + sk_rb_a_frag(wm, i % MB, lane, i / MB));
                };
                f16x8 af[3];
                af[0] = frag(0);
                af[1] = frag(1);
                chunk_prev_dpp<KK>(wc, first_lane);
                uint32_t pr[4];
                rb_static_for<0, 2 * MB>([&](auto ic) {
                    constexpr int I = decltype(ic)::value;
                    constexpr int mb = I % MB, rh = I / MB, f = I / 4, m = I % 4;
                    if constexpr (I + 2 < 2 * MB) af[(I + 2) % 3] = frag(I + 2);
#pragma unroll
                    for (int ch = 0; ch < 2; ch++)
                        acc[mb][ch] = mfma16x16x32(af[I % 3], __builtin_bit_cast(f16x8, own[2 * ch + rh]), acc[mb][ch]);
#pragma unroll
                    for (int ch = 0; ch < 2; ch++)
                        acc[mb][2 + ch] = mfma16x16x32(af[I % 3], __builtin_bit_cast(f16x8, pf[2 * ch + rh]),
                                                       acc[mb][2 + ch]);
                    // two SDWA fp16 adds, each writing one half (the same single rounding as
                    // sk_pair's two byte permutes and packed add, one instruction fewer per pair:
                    // 2-4% per M = 2048 call); the pair is stored to LDS before any MFMA reads it
                    pr[m] = pack_sum(rb_word<KK, CB, 2 * f + 8 * m>(wc, kc), rb_word<KK, CB, 2 * f + 8 * m + 1>(wc, kc));
                    if constexpr (m == 3) {
                        nown[f] = uint4{pr[0], pr[1], pr[2], pr[3]};
                        bx[sk_rb_bx(bo, wave, f, lane)] = nown[f];
                    }
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                });
            };

            // Prologue: A(s0), A(s0 + 1) into A buffers 0, 1; the own fragments of s0 decoded
            // and stored to B buffer 0; the words of s0 + 1 loaded.
            dma_a(s0, 0);
            dma_a(min(s0 + 1, s1 - 1), 1);
            load_b(wx, s0);
            load_b(wc, min(s0 + 1, s1 - 1));
            __builtin_amdgcn_s_waitcnt(rb_vmcnt(0));
            decode_put(wx, own, 0);
            __syncthreads();
            // Step s: A(s + 2) streams into A buffer (s - s0 + 2) % 3 (last read at step s - 1)
            // and the words of s + 2 into wx; the partner's fragments of s come from B buffer
            // (s - s0) % 2, and this wave's fragments of s + 1 are decoded from wc and stored to
            // the other B buffer (last read at step s - 1) while the MFMAs of s run.  Steps past
            // the piece load and decode in-bounds data that is never used.
            for (int s = s0; s < s1; s++) {
                const int b3 = (s - s0) % SK_RB_NBUF, b2 = (s - s0) & 1;
                dma_a(min(s + 2, s1 - 1), (s - s0 + 2) % SK_RB_NBUF);
                load_b(wx, min(s + 2, s1 - 1));
#pragma unroll
                for (int f = 0; f < 4; f++) pf[f] = bx[sk_rb_bx(b2, partner, f, lane)];
                step_body(b3, b2 ^ 1);
                // A(s + 1) landed (only this step's loads may still be in flight)
                __builtin_amdgcn_s_waitcnt(rb_vmcnt(4 + NBL));
                __syncthreads();
#pragma unroll
                for (int f = 0; f < 4; f++) own[f] = nown[f];
#pragma unroll
                for (int i = 0; i <= KK; i++) wc[i] = wx[i];
            }
            __builtin_amdgcn_s_waitcnt(rb_vmcnt(0));       // no load still writing LDS
        };
        run_piece(std::integral_constant<int, K>{});
        u += s1 - s0;
        if (wm) {   // accumulator blocks in chunk-group order for the epilogue
#pragma unroll
            for (int mb = 0; mb < MB; mb++)
#pragma unroll
                for (int ch = 0; ch < 2; ch++) {
                    const f32x4 t = acc[mb][ch];
                    acc[mb][ch] = acc[mb][2 + ch];
                    acc[mb][2 + ch] = t;
                }
        }
        sk_finish_piece<BM, true>(a, pc, S, g, wave, lane, tid, wm, wn, acc, lds);
    }
}

// ---------------------------------------------------------------- host side

int gemm_sk_cus() { return device_cus(); }

size_t gemm_sk_slot_bytes(int rows, int oc) { return sk_single_bytes(rows, oc, gemm_sk_cus()); }


size_t gemm_grouped_shard_bytes(int rows, int ic, int oc)
{
    return sk_grouped_bytes_bm(gemm_sk_bm(rows), rows, ic, oc, gemm_sk_cus());
}

// The 256-row form is the register-B kernel (ORCA_EXL3_SK_RB=0 selects the LDS-B kernel of
// the other tile heights at 256 rows, for comparison).
static bool sk_use_rb()
{
    static const bool rb = [] {
        const char* e = getenv("ORCA_EXL3_SK_RB");
        return !(e && e[0] == '0');
    }();
    return rb;
}

template <int K, int CB, int BM>
static const void* sk_fn()
{
    if constexpr (sk_rb<BM>() && K > 0)
        if (sk_use_rb()) return reinterpret_cast<const void*>(&gemm_rb_kernel<K, CB>);
    return reinterpret_cast<const void*>(&gemm_sk_kernel<K, CB, BM>);
}

template <int BM>
static const void* sk_fn_kcb(int K, int cb)
{
#define EXL3_CASE(KK) case KK: return cb == CB_MCG ? sk_fn<KK, CB_MCG, BM>() : sk_fn<KK, CB_3INST, BM>();
    if constexpr (sk_has_k0<BM>())
        if (K == 0) return cb == CB_MCG ? sk_fn<0, CB_MCG, BM>() : sk_fn<0, CB_3INST, BM>();   // per-shard K
    switch (K) {
        EXL3_CASE(1) EXL3_CASE(2) EXL3_CASE(3) EXL3_CASE(4)
        EXL3_CASE(5) EXL3_CASE(6) EXL3_CASE(7) EXL3_CASE(8)
    }
#undef EXL3_CASE
    return nullptr;
}

static const void* sk_fn_any(int BM, int K, int cb)
{
    switch (BM) {
    case 32: return sk_fn_kcb<32>(K, cb);
    case 48: return sk_fn_kcb<48>(K, cb);
    case 64: return sk_fn_kcb<64>(K, cb);
    case 96: return sk_fn_kcb<96>(K, cb);
    case 128: return sk_fn_kcb<128>(K, cb);
    case 256: return sk_fn_kcb<256>(K, cb);
    }
    return nullptr;
}

static int sk_lds_any(int BM)
{
    switch (BM) {
    case 32: return sk_lds<32>();
    case 48: return sk_lds<48>();
    case 64: return sk_lds<64>();
    case 96: return sk_lds<96>();
    case 128: return sk_lds<128>();
    default: return sk_use_rb() ? sk_rb_lds() : sk_lds<256>();
    }
}

// The kernels of one planned launch: the counter clear or the set-up kernel, then the
// stream-K kernel.
static int sk_emit(const SkLaunch& L, const char* what, hipStream_t stream)
{
    SkArgs a = *L.args;
    if (L.prep) {
        hipLaunchKernelGGL(sk_prep_kernel, dim3((unsigned)((L.prep_waves + 3) / 4)), dim3(256), 0, stream, *L.prep_args);
        const int rc = check_launch(what);
        if (rc != EXL3_OK) return rc;
    }
    const void* fn = sk_fn_any(L.BM, L.K, L.cb);
    if (!fn) return set_error(EXL3_ERR_ARG, "%s: K=%d is not in 1..8", what, L.K);   // K = 0: per shard
    const int lds = sk_lds_any(L.BM);
    if (lds > 64 * 1024) {
        hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        (void)hipGetLastError();
    }
    void* kargs[] = {&a};
    hipLaunchKernel(fn, dim3(L.G), dim3(64 * SK_WAVES), kargs, lds, stream);
    return check_launch(what);
}

int gemm_sk_dispatch(const uint16_t* Ah, const uint32_t* trellis, uint16_t* C, const uint16_t* svh, char* ws,
                     size_t ws_bytes, int rows, int ic, int oc, int K, int cb, hipStream_t stream)
{
    return sk_plan_single(Ah, trellis, C, svh, ws, ws_bytes, rows, ic, oc, K, cb, gemm_sk_cus(),
                          [&](const SkLaunch& L) { return sk_emit(L, "exl3_gemm (stream-K)", stream); });
}

template <int BM>
static int sk_grouped_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* ws,
                               size_t ws_bytes, const char* what, hipStream_t stream)
{
    return sk_plan_grouped<BM>(A, shards, nshards, rows, ws, ws_bytes, what, gemm_sk_cus(),
                               [&](const SkLaunch& L) { return sk_emit(L, what, stream); });
}

// Prefill of several shards (exl3_gemm_grouped; exl3_gemm's one-shard form at few rows):
// tile height by rows, as for one shard.  `what` names the entry point in errors.
int gemm_grouped_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* ws,
                          size_t ws_bytes, hipStream_t stream, const char* what)
{
    switch (gemm_sk_bm(rows)) {
    case 32: return sk_grouped_dispatch<32>(A, shards, nshards, rows, ws, ws_bytes, what, stream);
    case 48: return sk_grouped_dispatch<48>(A, shards, nshards, rows, ws, ws_bytes, what, stream);
    case 96: return sk_grouped_dispatch<96>(A, shards, nshards, rows, ws, ws_bytes, what, stream);
    case 64: return sk_grouped_dispatch<64>(A, shards, nshards, rows, ws, ws_bytes, what, stream);
    case 128: return sk_grouped_dispatch<128>(A, shards, nshards, rows, ws, ws_bytes, what, stream);
    default: return sk_grouped_dispatch<256>(A, shards, nshards, rows, ws, ws_bytes, what, stream);
    }
}

}  // namespace exl3
