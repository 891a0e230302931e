// Fused EXL3 decode-GEMV for 5..16 activation rows:
//   y_r (oc) = fp16( H( fp16(H(x_r * suh)) . W_q ) * svh ),  r < nrows
// with W_q decoded from the packed trellis in registers and never stored.  Replaces
// exllamav3_ext.exl3_gemm as called at orcasaq2/ops.py:46-49 for 5..16 rows.
//
// The decode is the batch-1 kernel's (gemv1.hip): one chunk of 32 positions per lane, three
// VALU instructions per position, the tail-biting word from the neighbouring lane by DPP.
// What changes is the unit: 4 tile rows x 2 tile columns instead of 1 x 8, so that the four
// k-groups of a v_mfma_f32_16x16x32_f16's B operand hold the same 16 output columns at
// different inputs, and all 16 rows of its A operand are activation rows -- one MFMA serves
// 16 rows for the same decode work (the unit layout is in gemv16_plan.h).  A 16-row
// activation table would not fit in LDS, so a set-up kernel writes every shard's transformed
// activations fp16(H128(x_r * suh)) once per call in the A-fragment order, and each lane loads
// its 8-byte fragments of a unit from there (L2-resident: 32 KB per 1024 inputs per shard) and
// duplicates each input into the two k-slots that meet a masked word's halves.
//
// Work decomposition as in gemv1.hip: units numbered shard, strip (32 outputs), then unit
// down the strip; G nearly equal contiguous ranges, one per workgroup of 8 waves (at odd K a
// launch of one group hands the workgroups to its blocks XCD by XCD, g16_block_wg), each wave a
// contiguous run, one unit in flight per wave.  A wave's partials of a strip go to
// red[strip + wave] in LDS; per strip the workgroup adds them in wave order into its slot.
// gemv16_finish_kernel then adds each strip's slots in workgroup order (deterministic) and,
// per 128 outputs (four strips), applies the output Hadamard and svh.
#include "exl3_common.h"
#include "gemv16_plan.h"

namespace exl3 {

template <int K>
__device__ __forceinline__ void g16_load(uint32_t (&w)[K + 1], const uint32_t* __restrict__ p)
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

// MFMA (m, h) of a unit: B = the masked words of positions 8m + 4h + t, A = the unit's step-m
// activation fragment.
template <int K, int CB, int M, int H>
__device__ __forceinline__ void g16_mfma(const uint32_t (&w)[K + 1], const uint4& a, f32x4 (&acc)[2],
                                         const Dot2Consts& kc)
{
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    constexpr int q = 8 * M + 4 * H;
    const u4 b = {dot2_word<K, CB, q>(w, kc), dot2_word<K, CB, q + 1>(w, kc), dot2_word<K, CB, q + 2>(w, kc),
                  dot2_word<K, CB, q + 3>(w, kc)};
    acc[H] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                    acc[H], 0, 0, 0);
}

// A fragment of four fp16 inputs (two words) as the MFMA's eight k-slots: each input in the
// two slots that meet a masked word's two halves.
__device__ __forceinline__ uint4 g16_dup(const uint2 x)
{
    return uint4{__builtin_amdgcn_perm(x.x, x.x, 0x01000100u), __builtin_amdgcn_perm(x.x, x.x, 0x03020302u),
                 __builtin_amdgcn_perm(x.y, x.y, 0x01000100u), __builtin_amdgcn_perm(x.y, x.y, 0x03020302u)};
}

template <int K>
struct G16Unit {
    uint32_t w[K + 1];
    uint2 a[4];   // four fp16 inputs per MFMA step, duplicated when the step runs
};

// Workgroup g of group a (shard table sht) -- the whole decode kernel body.
template <int K, int CB, bool ONE>
__device__ __forceinline__ void g16_body(const G1Group& a, const G16Shard* sht, const int g, float* red)
{
    const G1Range w = g16_range<ONE>(a, sht, g);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    __builtin_amdgcn_s_setprio(3);
    const G1Run run = g1_wave_run(w.L, wave);
    const int n = run.n;
    const bool first_lane = (lane & 7) == 0;

    // the lane's chunk inside a unit depends on the shard's tile-column count
    G16Cursor pf = g16_cursor_at<K, ONE>(a, sht, w.ub + run.lo), cu = pf;
    long lw = g16_lane_word(lane, g16_sh<ONE>(sht, pf.s).oc16, K);
    int lw_s = pf.s;
    int jpf = 0;
    // Lane 16 j + i holds activation row i of the A operand.  Rows past the call's nrows only
    // feed C rows that are never stored, so their lanes read the last live row's fragment:
    // at up to 8 rows a k-group's 16 lanes then touch one 128-byte line instead of two.
    const int lane_a = g16_ah_lane(lane, a.nrows);
    auto load = [&](G16Unit<K>& u, const G16Cursor& c) {
        if (c.s != lw_s) {
            lw_s = c.s;
            lw = g16_lane_word(lane, g16_sh<ONE>(sht, c.s).oc16, K);
        }
        g16_load<K>(u.w, c.p + lw);
#pragma unroll
        for (int m = 0; m < 4; m++) u.a[m] = *reinterpret_cast<const uint2*>(c.ah + g16_ah_word(m, lane_a));
    };
    G16Unit<K> un;
    if (n > 0) load(un, pf);
    const Dot2Consts kc = dot2_consts();

    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    int cur = cu.S - w.S_first;
    const int pq1 = (n + 3) >> 2, pq2 = (n + 1) >> 1, pq3 = (3 * n + 3) >> 2;
    auto flush = [&](int k) {
        float* rr = red + g16_red_row(cur, wave);
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int t = 0; t < 4; t++) rr[g16_acc_index(lane, h, t)] = acc[h][t];
        acc[0] = acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
        cur = k;
    };
    for (int j = 0; j < n; j++) {
        if (cu.S - w.S_first != cur) flush(cu.S - w.S_first);
        chunk_prev_dpp<K>(un.w, first_lane);
        G16Unit<K> u = un;
        if (j + 1 < n) g16_advance<K, ONE>(a, sht, cu);
        g16_next_pf<K, ONE>(a, sht, pf, jpf, n);
        load(un, pf);
        {
            const uint4 a0 = g16_dup(u.a[0]);
            g16_mfma<K, CB, 0, 0>(u.w, a0, acc, kc);
            g16_mfma<K, CB, 0, 1>(u.w, a0, acc, kc);
        }
        {
            const uint4 a1 = g16_dup(u.a[1]);
            g16_mfma<K, CB, 1, 0>(u.w, a1, acc, kc);
            g16_mfma<K, CB, 1, 1>(u.w, a1, acc, kc);
        }
        {
            const uint4 a2 = g16_dup(u.a[2]);
            g16_mfma<K, CB, 2, 0>(u.w, a2, acc, kc);
            g16_mfma<K, CB, 2, 1>(u.w, a2, acc, kc);
        }
        {
            const uint4 a3 = g16_dup(u.a[3]);
            g16_mfma<K, CB, 3, 0>(u.w, a3, acc, kc);
            g16_mfma<K, CB, 3, 1>(u.w, a3, acc, kc);
        }
        const int done = j + 1;
        if (done == pq1) __builtin_amdgcn_s_setprio(2);
        if (done == pq2) __builtin_amdgcn_s_setprio(1);
        if (done == pq3) __builtin_amdgcn_s_setprio(0);
    }
    __builtin_amdgcn_s_setprio(3);
    if (n > 0) flush(cur);
    __syncthreads();

    // per strip: the partials of the waves whose runs meet it, in wave order, into this
    // workgroup's slot (lane l: 8 consecutive of the strip's 16 x 32)
    for (int k = wave; k < w.nseg; k += G1_NW) {
        int ub, ue;
        g1_seg_units(w, a.ntr, k, ub, ue);
        float4 v0 = {0.f, 0.f, 0.f, 0.f}, v1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ww = 0; ww < G1_NW; ww++) {
            if (!g1_run_meets(g1_wave_run(w.L, ww), ub, ue)) continue;
            const float4* p = reinterpret_cast<const float4*>(red + g16_red_row(k, ww) + 8 * lane);
            const float4 x0 = p[0], x1 = p[1];
            v0.x += x0.x; v0.y += x0.y; v0.z += x0.z; v0.w += x0.w;
            v1.x += x1.x; v1.y += x1.y; v1.z += x1.z; v1.w += x1.w;
        }
        float4* sl = reinterpret_cast<float4*>(a.slots + g16_slot(w.S_first + k, g) + 8 * lane);
        sl[0] = v0;
        sl[1] = v1;
    }
}

// 5..16 rows need at most 64 VGPRs for eight waves per SIMD, as the batch-1 kernel.
template <int K, int CB, bool ONE>
__global__ __launch_bounds__(64 * G1_NW) __attribute__((amdgpu_waves_per_eu(8, 8), amdgpu_num_sgpr(74))) void gemv16_kernel(const G16Args a)
{
    extern __shared__ __attribute__((aligned(16))) float g16_red[];
    g16_body<K, CB, ONE>(a.grp, a.sh, g16_block_wg(blockIdx.x, gridDim.x, K), g16_red);
}

template <int CB>
__global__ __launch_bounds__(64 * G1_NW) __attribute__((amdgpu_waves_per_eu(8, 8), amdgpu_num_sgpr(74))) void gemv16_multi_kernel(const G16Multi)
{
    extern __shared__ __attribute__((aligned(16))) float g16_red[];
    const G16Multi& mm = *(const G16Multi*)__builtin_amdgcn_kernarg_segment_ptr();
    const int i = __builtin_amdgcn_readfirstlane(g1_group_of(mm.gbeg, mm.ngrp, (int)blockIdx.x));
    const G1Group& a = mm.grp[i];
    const G16Shard* sht = mm.sh + mm.sh0[i];
    const int g = blockIdx.x - mm.gbeg[i];
    switch (mm.K[i]) {
    case 1: g16_body<1, CB, false>(a, sht, g, g16_red); break;
    case 2: g16_body<2, CB, false>(a, sht, g, g16_red); break;
    case 3: g16_body<3, CB, false>(a, sht, g, g16_red); break;
    case 4: g16_body<4, CB, false>(a, sht, g, g16_red); break;
    case 5: g16_body<5, CB, false>(a, sht, g, g16_red); break;
    case 6: g16_body<6, CB, false>(a, sht, g, g16_red); break;
    case 7: g16_body<7, CB, false>(a, sht, g, g16_red); break;
    case 8: g16_body<8, CB, false>(a, sht, g, g16_red); break;
    }
}

// ---------------------------------------------------------------- finish and set-up

// 128 outputs (column group cg4 = four strips) of group a, activation row r (one wave): lane
// l sums output pair 2l, 2l + 1 (strip l / 16) over that strip's slots in workgroup order,
// then the output Hadamard, * svh, fp16 store.  Up to 8 slots are loaded per batch before the
// adds.
template <bool ONE>
__device__ __forceinline__ void g16_finish_body(const G1Group& a, const G16Shard* sht, int cg4, int r)
{
    if (cg4 * 4 >= a.nsegs || r >= a.nrows) return;
    const int lane = threadIdx.x & 63;
    const int S = 4 * cg4 + (lane >> 4);          // this lane's strip
    const int s = g16_shard_of_seg<ONE>(a, sht, 4 * cg4);
    const G16Shard& e = g16_sh<ONE>(sht, s);
    const int cg = cg4 - e.sbeg / 4;                // 128-output block of the shard
    int g_lo, g_hi;
    g16_contributors<ONE>(a, sht, S, g_lo, g_hi);
    const int nsl = g_hi - g_lo + 1;
    // the most slots any lane of the wave has (strips differ)
    int nmax = nsl;
#pragma unroll
    for (int d = 16; d < 64; d <<= 1) nmax = max(nmax, __shfl_xor(nmax, d, 64));
    nmax = __builtin_amdgcn_readfirstlane(nmax);
    const uint32_t sv = reinterpret_cast<const uint32_t*>(e.svh + cg * 128)[lane];
    const int col = (2 * lane) & 31;
    constexpr int B = 8;
    {
        float v0 = 0.f, v1 = 0.f;
        for (int t0 = 0; t0 < nmax; t0 += B) {
            float2 xv[B];
#pragma unroll
            for (int t = 0; t < B; t++) {
                const int tt = min(t0 + t, nsl - 1);
                xv[t] = *reinterpret_cast<const float2*>(a.slots + g16_slot(S, g_lo + tt) + r * G16_STRIP + col);
            }
#pragma unroll
            for (int t = 0; t < B; t++)
                if (t0 + t < nsl) {
                    v0 += xv[t].x;
                    v1 += xv[t].y;
                }
        }
        wave_fwht128(v0, v1);
        v0 *= (float)__builtin_bit_cast(_Float16, (uint16_t)(sv & 0xffffu));
        v1 *= (float)__builtin_bit_cast(_Float16, (uint16_t)(sv >> 16));
        reinterpret_cast<uint32_t*>(e.C + r * e.ldc + cg * 128)[lane] =
            (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v0) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v1) << 16);
    }
}

// Block (x, y): column group x, rows 4y .. 4y + 3 (one wave each).
template <bool ONE>
__global__ __launch_bounds__(256) void gemv16_finish_kernel(const G16Args a)
{
    g16_finish_body<ONE>(a.grp, a.sh, blockIdx.x, 4 * blockIdx.y + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
}

__global__ __launch_bounds__(256) void gemv16_finish_multi_kernel(const G16Multi)
{
    const G16Multi& mm = *(const G16Multi*)__builtin_amdgcn_kernarg_segment_ptr();
    const int i = __builtin_amdgcn_readfirstlane(g1_group_of(mm.fbeg, mm.ngrp, (int)blockIdx.x));
    g16_finish_body<false>(mm.grp[i], mm.sh + mm.sh0[i], blockIdx.x - mm.fbeg[i],
                           4 * blockIdx.y + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
}

// fp16(H128(A_r * suh_s)) into the shard's fragments.  One workgroup per (shard, 128-input block) (g16_prep_wg): the block's 16 rows transformed
// four per wave (the four transforms' lane exchanges in flight together) into LDS, then the
// block's fragment area written with one 16-byte store per lane, in address order.  (One wave
// per row and block storing 4-byte words at the fragment layout's 512-byte strides took
// 4.1 us per qkv call.)
__global__ __launch_bounds__(G16_PREP_LANES) void gemv16_prep_kernel(const G16Prep p)
{
    __shared__ uint32_t xs[16][65];           // [row][input pair], padded
    int s, b;
    g16_prep_wg(p, blockIdx.x, s, b);
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t sw = reinterpret_cast<const uint32_t*>(p.suh[s] + b * 128)[lane];
    const float s0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(sw & 0xffffu));
    const float s1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(sw >> 16));
    float v0[4], v1[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int r = wv + 4 * j;
        const uint32_t xw = r < p.rows ? reinterpret_cast<const uint32_t*>(p.A + (long)r * p.ic + b * 128)[lane] : 0u;
        v0[j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(xw & 0xffffu)) * s0;
        v1[j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(xw >> 16)) * s1;
    }
    wave_fwht128_n<4>(v0, v1, fwht_signs(lane));
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t h0 = __builtin_bit_cast(uint16_t, (_Float16)v0[j]);
        const uint32_t h1 = __builtin_bit_cast(uint16_t, (_Float16)v1[j]);
        xs[wv + 4 * j][lane] = h0 | (h1 << 16);
    }
    __syncthreads();
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        int i, k;
        g16_prep_src(4 * threadIdx.x + e, i, k);
        o[e] = xs[i][k >> 1];
    }
    reinterpret_cast<uint4*>(p.ah[s] + g16_prep_base(b))[threadIdx.x] = uint4{o[0], o[1], o[2], o[3]};
}

// ---------------------------------------------------------------- host side

template <int K, int CB>
static const void* g16_fn(bool one)
{
    return one ? reinterpret_cast<const void*>(&gemv16_kernel<K, CB, true>)
               : reinterpret_cast<const void*>(&gemv16_kernel<K, CB, false>);
}

static const void* g16_fn_kcb(int K, int cb, bool one)
{
#define EXL3_CASE(KK) case KK: return cb == CB_MCG ? g16_fn<KK, CB_MCG>(one) : g16_fn<KK, CB_3INST>(one);
    switch (K) {
        EXL3_CASE(1) EXL3_CASE(2) EXL3_CASE(3) EXL3_CASE(4)
        EXL3_CASE(5) EXL3_CASE(6) EXL3_CASE(7) EXL3_CASE(8)
    }
#undef EXL3_CASE
    return nullptr;
}


size_t gemv16_shard_bytes(int ic, int oc) { return g16_shard_bytes(ic, oc); }

// A decode launch's dynamic LDS above 64 KiB needs the kernel's opt-in first (the plan allows
// up to a CU's 160 KiB when a launch's ranges are long).
static void g16_lds_optin(const void* fn, size_t lds)
{
    if (lds > 64 * 1024) {
        hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        (void)hipGetLastError();
    }
}

int gemv16_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* ws, size_t ws_bytes,
                    hipStream_t stream)
{
    const char* what = "exl3_gemv (5-16 rows)";
    G16Prep prep;
    bool prepped = false;
    return g16_plan(A, shards, nshards, rows, ws, ws_bytes, device_cus(), prep, [&](const G16Launch& L) {
        if (!prepped) {
            hipLaunchKernelGGL(gemv16_prep_kernel, dim3((unsigned)(prep.nsh * prep.nblk)), dim3(G16_PREP_LANES), 0,
                               stream, prep);
            const int rc = check_launch(what);
            if (rc != EXL3_OK) return rc;
            prepped = true;
        }
        if (!L.multi) {
            G16Args args = *L.args;
            const void* fn = g16_fn_kcb(L.K, L.cb, L.one);
            if (!fn) return set_error(EXL3_ERR_ARG, "%s: K=%d is not in 1..8", what, L.K);
            void* kargs[] = {&args};
            g16_lds_optin(fn, L.lds);
            hipLaunchKernel(fn, dim3(L.G), dim3(64 * G1_NW), kargs, L.lds, stream);
            int rc = check_launch(what);
            if (rc != EXL3_OK) return rc;
            const void* ff = L.one ? reinterpret_cast<const void*>(&gemv16_finish_kernel<true>)
                                   : reinterpret_cast<const void*>(&gemv16_finish_kernel<false>);
            hipLaunchKernel(ff, dim3(L.fblocks, (L.args->grp.nrows + 3) / 4), dim3(256), kargs, 0, stream);
            return check_launch(what);
        }
        G16Multi m = *L.m;
        const void* fn = L.cb == CB_MCG ? reinterpret_cast<const void*>(&gemv16_multi_kernel<CB_MCG>)
                                        : reinterpret_cast<const void*>(&gemv16_multi_kernel<CB_3INST>);
        void* kargs[] = {&m};
        g16_lds_optin(fn, L.lds);
        hipLaunchKernel(fn, dim3(L.G), dim3(64 * G1_NW), kargs, L.lds, stream);
        int rc = check_launch(what);
        if (rc != EXL3_OK) return rc;
        hipLaunchKernel(reinterpret_cast<const void*>(&gemv16_finish_multi_kernel), dim3(L.fblocks, (m.grp[0].nrows + 3) / 4),
                        dim3(256), kargs, 0, stream);
        return check_launch(what);
    });
}

}  // namespace exl3
