// Fused EXL3 decode-GEMV for one activation row (batch-1 decode):
//   y (oc) = fp16( H( fp16(H(x * suh)) . W_q ) * svh )
// with W_q decoded from the packed trellis in registers and never stored.  Replaces
// exllamav3_ext.exl3_gemm as called at orcasaq2/ops.py:46-49 for rows == 1 (the other row
// counts take gemv.hip's MFMA kernels).
//
// Work decomposition.  A *unit* is one tile row of one 128-output column group: 8 tiles
// side by side, 64 chunks of 32 positions -- one chunk per lane of a wave, the 8 tiles'
// words one contiguous run of 64K u32 in HBM.  Units are numbered shard-major, then
// column group, then tile row, and the whole launch's units are cut into G equal
// contiguous ranges, one per workgroup (G = a few workgroups per CU, all resident at
// once: there is no tail wave of workgroups).  A workgroup's range touches a few
// *segments* (shard, column group); its waves take the range's units round-robin.
//
// Per workgroup:
//   1. each wave issues the loads of its first D units (D = 2..6 by K, about 24 VGPRs of
//      words in flight per lane), so HBM is busy from the start;
//   2. main loop over the wave's units: a unit's K words (+ the tail-biting word before
//      them) per lane stream through the D-deep register ring.  The tile row's 16
//      activations fp16(H(x * suh)) are built in registers from the 128-input block (one
//      x and one suh dword per lane; per-lane sign factor, cross-lane shuffles over lane
//      bits 3..5, butterflies over lane bits 0..2), one unit ahead of its use.  Each
//      position is decoded with an SDWA add (or a 16-bit field for MCG), a v_mul_lo_u32 and
//      a v_bitop3; the masked word meets its activation in a v_dot2c_f32_f16 whose second
//      operand is broadcast by DPP from the lane that owns the activation row (both fp16
//      halves times x, summed in fp32);
//   3. per segment, the waves' partial sums are added in a fixed order through LDS.  If the
//      segment lies inside this workgroup's range it is finished here; otherwise the
//      partial goes to this workgroup's slot with agent-coherent stores, and the last of the
//      segment's workgroups to arrive (a relaxed agent-scope counter in the workspace) adds
//      all slots in slot order -- deterministic -- and finishes: output Hadamard, * svh,
//      fp16 store, counter back to 0.  No cache-wide release/acquire is used: the slots
//      are written with agent-scope stores and read with agent-scope loads, and each
//      writer waits for its stores to complete before it increments the counter.
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

constexpr int G1_NW = 8;                 // waves per workgroup
constexpr int G1_MAXSH = 8;              // shards per launch
constexpr int G1_WG_PER_CU = 4;          // target resident workgroups per CU (8 waves / SIMD)
constexpr int G1_GMAX = 2048;            // workgroups per launch (bounds the slot area)

// Prefetch depth in units: about 24 VGPRs of loads in flight per lane whatever K is (a unit
// is K + 1 trellis words plus an x and a suh word per lane), 2..6 units.
template <int K>
struct G1Depth {
    static constexpr int value = (24 / (K + 3)) < 2 ? 2 : (24 / (K + 3)) > 6 ? 6 : (24 / (K + 3));
};

struct G1Shard {
    const uint32_t* trellis;   // (ic/16, oc/16, 8K) u32
    const uint16_t* suh;       // (ic)
    const uint16_t* svh;       // (oc)
    uint16_t* C;               // (oc) fp16 output
    int ubeg;                  // first unit of the shard
    int sbeg;                  // first segment of the shard
    int oc16;                  // tile columns
    int ncg;                   // column groups (oc / 128)
};

struct G1Args {
    const uint16_t* x;         // (ic) fp16
    uint32_t* counters;        // one per segment; zero between calls
    float* slots;              // (G + segments) x 128 fp32
    int U, G, ntr, nshards, nsegs;
    G1Shard sh[G1_MAXSH];
};

// Workgroup whose unit range [floor(g U / G), floor((g+1) U / G)) holds unit u.
__device__ __forceinline__ int g1_wg_of(int u, int U, int G)
{
    return (int)((((long)u + 1) * G - 1) / U);
}

__device__ __forceinline__ int g1_shard_of_seg(const G1Args& a, int S)
{
    int s = 0;
#pragma unroll
    for (int i = 1; i < G1_MAXSH; i++)
        if (i < a.nshards && S >= a.sh[i].sbeg) s = i;
    return s;
}

__device__ __forceinline__ float g1_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float g1_hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }

// A lane's chunk: w[1..K] = its K words, w[0] = the tile's word before them (wrapping).
template <int K>
__device__ __forceinline__ void g1_load(uint32_t (&w)[K + 1], const uint32_t* __restrict__ unit, uint32_t lk,
                                        uint32_t lprev)
{
    const uint32_t* p = unit + lk;
    if constexpr (K == 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        w[1] = v.x; w[2] = v.y; w[3] = v.z; w[4] = v.w;
    } else if constexpr (K == 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        const uint4 u = *reinterpret_cast<const uint4*>(p + 4);
        w[1] = v.x; w[2] = v.y; w[3] = v.z; w[4] = v.w;
        w[5] = u.x; w[6] = u.y; w[7] = u.z; w[8] = u.w;
    } else if constexpr (K == 2 || K == 6) {
#pragma unroll
        for (int i = 0; i < K; i += 2) {
            const uint2 v = *reinterpret_cast<const uint2*>(p + i);
            w[i + 1] = v.x;
            w[i + 2] = v.y;
        }
    } else {
#pragma unroll
        for (int i = 0; i < K; i++) w[i + 1] = p[i];
    }
    w[0] = unit[lprev];
}

// Eight waves per SIMD need at most 64 VGPRs (measured on MI355X: 68 VGPRs leave room for
// only 6); the SGPR cap keeps the count well inside what eight waves per SIMD may hold.
template <int K, int CB>
__global__ __launch_bounds__(64 * G1_NW) __attribute__((amdgpu_waves_per_eu(8, 8), amdgpu_num_sgpr(74))) void gemv1_kernel(const G1Args a)
{
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];

    const int g = blockIdx.x;
    const int U = a.U, G = a.G, ntr = a.ntr, ntrb = ntr >> 3;
    const int ub = (int)((long)g * U / G), ue = (int)((long)(g + 1) * U / G);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;

    // ---- this workgroup's segments: S_first .. S_first + nseg - 1
    const int s_first = [&] {
        int s = 0;
#pragma unroll
        for (int i = 1; i < G1_MAXSH; i++)
            if (i < a.nshards && ub >= a.sh[i].ubeg) s = i;
        return s;
    }();
    const int rel0 = ub - a.sh[s_first].ubeg;
    const int S_first = a.sh[s_first].sbeg + rel0 / ntr;
    const int t_first = rel0 % ntr;
    const int nseg = [&] {
        const int u = ue - 1;
        int s = 0;
#pragma unroll
        for (int i = 1; i < G1_MAXSH; i++)
            if (i < a.nshards && u >= a.sh[i].ubeg) s = i;
        return a.sh[s].sbeg + (u - a.sh[s].ubeg) / ntr - S_first + 1;
    }();
    float* red = reinterpret_cast<float*>(lds);                // [nseg][G1_NW][128]

    // ---- this wave's units: ub + wave + G1_NW * j, j < n
    const int n = (ue - ub > wave) ? (ue - ub - wave + G1_NW - 1) / G1_NW : 0;
    const int c = lane & 7;
    const uint32_t lk = lane * K;
    const uint32_t lprev = c ? lk - 1 : lk + 8 * K - 1;

    // Wave-uniform cursor over the wave's units: shard, column group, tile row, segment
    // index within the workgroup, the first word of the unit's 8 tiles and the shard's
    // suh.  Consecutive units of a wave are G1_NW tile rows apart (ntr >= 8, so a step
    // crosses at most one column-group boundary); only such a crossing reads the shard
    // table again.
    struct Cursor {
        int s, cg, tr, k;
        long stride;   // words between tile rows G1_NW apart
        const uint32_t* p;
        const uint16_t* suh;
    };
    auto seat = [&](Cursor& q) {
        q.stride = (long)G1_NW * a.sh[q.s].oc16 * (8 * K);
        q.p = a.sh[q.s].trellis + ((long)q.tr * a.sh[q.s].oc16 + 8 * q.cg) * (8 * K);
        q.suh = a.sh[q.s].suh;
    };
    auto cursor_at = [&](int u) {
        Cursor q;
        q.s = 0;
#pragma unroll
        for (int i = 1; i < G1_MAXSH; i++)
            if (i < a.nshards && u >= a.sh[i].ubeg) q.s = i;
        const int rel = u - a.sh[q.s].ubeg;
        q.cg = rel / ntr;
        q.tr = rel - q.cg * ntr;
        q.k = a.sh[q.s].sbeg + q.cg - S_first;
        seat(q);
        return q;
    };
    auto advance = [&](Cursor& q) {
        q.tr += G1_NW;
        q.p += q.stride;
        if (q.tr >= ntr) {
            q.tr -= ntr;
            q.k++;
            if (++q.cg == a.sh[q.s].ncg) {
                q.s++;
                q.cg = 0;
            }
            seat(q);
        }
    };

    // A unit's loads: the lane's K words + the tail-biting word, and the 128 inputs (x and
    // suh, one dword each per lane) of the tile row's Hadamard block.
    constexpr int D = G1Depth<K>::value;
    struct Slot {
        uint32_t w[K + 1];
        uint32_t xw, sw;
    };
    auto load = [&](Slot& sl, const Cursor& q) {
        g1_load<K>(sl.w, q.p, lk, lprev);
        const int blk = q.tr >> 3;
        sl.xw = reinterpret_cast<const uint32_t*>(a.x + blk * 128)[lane];
        sl.sw = reinterpret_cast<const uint32_t*>(q.suh + blk * 128)[lane];
    };

    // prefetch cursor (D units ahead; it stops at the wave's last unit, whose data is then
    // loaded again and not used) and processing cursor
    Cursor pf = cursor_at(ub + wave), cu = pf;
    int jpf = 0;
    auto next_pf = [&]() -> const Cursor& {
        if (jpf + 1 < n) {
            jpf++;
            advance(pf);
        }
        return pf;
    };
    Slot ring[D];
    if (n > 0) {
        load(ring[0], pf);
#pragma unroll
        for (int d = 1; d < D; d++) load(ring[d], next_pf());
    }
    for (int k = 0; k < nseg; k++)
        *reinterpret_cast<float2*>(red + (k * G1_NW + wave) * 128 + 2 * lane) = float2{0.f, 0.f};
    const Dot2Consts kc = dot2_consts();
    // A wave's units are G1_NW = 8 tile rows apart and segments start on 128-input block
    // boundaries, so its tile row within the block -- and the activation signs -- never change.
    const float fact = tile_row_factor(cu.tr & 7, lane);

    // ---- main loop.  Scalar bookkeeping (cursor steps, column-group crossings, flushes of a
    // finished segment's sums to the wave's LDS row) sits between units, so each unit's
    // work is one basic block the scheduler can interleave; the loads sit outside every
    // branch, so the wait before a unit covers only that unit's own loads.
    const int o0 = (lane >> 3) * 16 + c;
    float y0 = 0.f, y1 = 0.f;
    int cur = 0;
    auto flush = [&](int k) {
        red[(cur * G1_NW + wave) * 128 + o0] = y0;
        red[(cur * G1_NW + wave) * 128 + o0 + 8] = y1;
        y0 = y1 = 0.f;
        cur = k;
    };
    // The activations of unit j + 1 are built while unit j decodes (their cross-lane
    // shuffles wait on LDS; the decode hides that).
    uint32_t a0 = 0, a1 = 0;
    if (n > 0) tile_row_act(ring[0].xw, ring[0].sw, fact, lane, a0, a1);
    for (int j = 0; j < n; j += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            if (d == 0 || j + d < n) {
                if (cu.k != cur) flush(cu.k);
                uint32_t b0, b1;
                tile_row_act(ring[(d + 1) % D].xw, ring[(d + 1) % D].sw, fact, lane, b0, b1);
                float acc[4] = {0.f, 0.f, 0.f, 0.f};
                dot2_chunk<K, CB>(ring[d].w, a0, a1, acc, kc);
                y0 += acc[0] + acc[1];
                y1 += acc[2] + acc[3];
                a0 = b0;
                a1 = b1;
                if (j + d + 1 < n) advance(cu);
            }
            load(ring[d], next_pf());
        }
    }
    if (n > 0) flush(cur);
    __syncthreads();

    // ---- per segment: fixed-order sum of the waves, then finish here or via the slots
    for (int k = wave; k < nseg; k += G1_NW) {
        float v0 = 0.f, v1 = 0.f;
#pragma unroll
        for (int ww = 0; ww < G1_NW; ww++) {
            const float2 p = *reinterpret_cast<const float2*>(red + (k * G1_NW + ww) * 128 + 2 * lane);
            v0 += p.x;
            v1 += p.y;
        }
        const int S = S_first + k;
        const int s = g1_shard_of_seg(a, S);
        const int cg = S - a.sh[s].sbeg;
        const int segU0 = a.sh[s].ubeg + cg * ntr;
        const int g_lo = g1_wg_of(segU0, U, G), g_hi = g1_wg_of(segU0 + ntr - 1, U, G);
        if (g_hi > g_lo) {
            float* my = a.slots + (long)(S + g) * 128 + 2 * lane;
            __hip_atomic_store(my, v0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(my + 1, v1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);   // this wave's slot stores are complete
            uint32_t old = 0;
            if (lane == 0)
                old = __hip_atomic_fetch_add(a.counters + S, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            old = __shfl(old, 0, 64);
            if (old != (uint32_t)(g_hi - g_lo)) continue;
            // last to arrive: every other contributor's slot stores completed before its
            // counter increment, which precedes ours
            v0 = v1 = 0.f;
            const float* sl = a.slots + (long)(S + g_lo) * 128 + 2 * lane;
            const int nsl = g_hi - g_lo + 1;
            for (int g0 = 0; g0 < nsl; g0 += 16) {
                float x0[16], x1[16];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int gg = min(g0 + i, nsl - 1);
                    x0[i] = __hip_atomic_load(sl + gg * 128, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    x1[i] = __hip_atomic_load(sl + gg * 128 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    if (g0 + i < nsl) {
                        v0 += x0[i];
                        v1 += x1[i];
                    }
                }
            }
            if (lane == 0) __hip_atomic_store(a.counters + S, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        wave_fwht128(v0, v1);
        const uint32_t sv = reinterpret_cast<const uint32_t*>(a.sh[s].svh + cg * 128)[lane];
        v0 *= g1_lo(sv);
        v1 *= g1_hi(sv);
        const uint32_t out = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v0) |
                             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v1) << 16);
        reinterpret_cast<uint32_t*>(a.sh[s].C + cg * 128)[lane] = out;
    }
}

// ---------------------------------------------------------------- host side

template <int K, int CB>
static const void* g1_fn() { return reinterpret_cast<const void*>(&gemv1_kernel<K, CB>); }

static const void* g1_fn_kcb(int K, int cb)
{
#define EXL3_CASE(KK) case KK: return cb == CB_MCG ? g1_fn<KK, CB_MCG>() : g1_fn<KK, CB_3INST>();
    switch (K) {
        EXL3_CASE(1) EXL3_CASE(2) EXL3_CASE(3) EXL3_CASE(4)
        EXL3_CASE(5) EXL3_CASE(6) EXL3_CASE(7) EXL3_CASE(8)
    }
#undef EXL3_CASE
    return nullptr;
}

static int g1_cu_count()
{
    struct Entry { int dev, cus; };
    static thread_local Entry seen[16];
    static thread_local int nseen = 0;
    int dev = 0;
    hipGetDevice(&dev);
    for (int i = 0; i < nseen; i++)
        if (seen[i].dev == dev) return seen[i].cus;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (nseen < 16) seen[nseen++] = Entry{dev, cus};
    return cus;
}

// Dynamic LDS a launch needs: a partial row per wave for the most segments (shard, column
// group) a workgroup range of ceil(U / G) units can touch.
static size_t g1_lds_bytes(int U, int G, int ntr)
{
    const int L = (U + G - 1) / G;
    const int nseg = (L - 1 + ntr - 1) / ntr + 1;
    return (size_t)nseg * G1_NW * 128 * sizeof(float);
}

// Per-shard share of the workspace after the counter area: slot rows for up to G1_GMAX
// workgroups and one per column group.
size_t gemv1_slot_bytes(int ic, int oc)
{
    (void)ic;
    return (size_t)(G1_GMAX + oc / 128) * 128 * sizeof(float);
}

int gemv1_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, uint32_t* counters, int max_counters,
                   char* slots, size_t slot_bytes, hipStream_t stream)
{
    const int ic = shards[0].ic;
    const int ntr = ic / 16;
    bool done[EXL3_MAX_SHARDS] = {false};
    int cbase = 0;
    size_t sbase = 0;
    const int gmax = std::min(G1_GMAX, G1_WG_PER_CU * g1_cu_count());
    for (int i = 0; i < nshards; i++) {
        if (done[i]) continue;
        G1Args args = {};
        args.x = A;
        args.ntr = ntr;
        long U = 0;
        int nsegs = 0;
        for (int s = i; s < nshards && args.nshards < G1_MAXSH; s++) {
            if (done[s] || shards[s].K != shards[i].K || shards[s].cb != shards[i].cb) continue;
            const GemvShard& d = shards[s];
            G1Shard& e = args.sh[args.nshards++];
            e.trellis = d.trellis;
            e.suh = d.suh;
            e.svh = d.svh;
            e.C = d.C;
            e.ubeg = (int)U;
            e.sbeg = nsegs;
            e.oc16 = d.oc / 16;
            e.ncg = d.oc / 128;
            U += (long)(d.oc / 128) * ntr;
            nsegs += d.oc / 128;
            done[s] = true;
        }
        if (U > (1L << 30))
            return set_error(EXL3_ERR_ARG, "exl3_gemv: %ld tile-row units in one launch (limit 2^30)", U);
        if (cbase + nsegs > max_counters)
            return set_error(EXL3_ERR_ARG, "exl3_gemv: %d column groups exceed the %d segment counters",
                             cbase + nsegs, max_counters);
        int G = (int)std::min<long>(gmax, std::max<long>(1, U / G1_NW));
        const size_t lds = g1_lds_bytes((int)U, G, ntr);
        const size_t need = (size_t)(G + nsegs) * 128 * sizeof(float);
        if (sbase + need > slot_bytes)
            return set_error(EXL3_ERR_WORKSPACE, "exl3_gemv: slot area of %zu bytes, %zu needed", slot_bytes,
                             sbase + need);
        args.U = (int)U;
        args.G = G;
        args.nsegs = nsegs;
        args.counters = counters + cbase;
        args.slots = reinterpret_cast<float*>(slots + sbase);
        cbase += nsegs;
        sbase += need;
        const void* fn = g1_fn_kcb(shards[i].K, shards[i].cb);
        if (!fn) return set_error(EXL3_ERR_ARG, "exl3_gemv: K=%d is not in 1..8", shards[i].K);
        if (lds > 64 * 1024) {
            hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            (void)hipGetLastError();
        }
        void* kargs[] = {&args};
        hipLaunchKernel(fn, dim3(G), dim3(64 * G1_NW), kargs, lds, stream);
        const int rc = check_launch("exl3_gemv (batch 1)");
        if (rc != EXL3_OK) return rc;
    }
    return EXL3_OK;
}

}  // namespace exl3
