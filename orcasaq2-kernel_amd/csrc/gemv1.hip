// Fused EXL3 decode-GEMV for one activation row (batch-1 decode):
//   y (oc) = fp16( H( fp16(H(x * suh)) . W_q ) * svh )
// with W_q decoded from the packed trellis in registers and never stored.  Replaces
// exllamav3_ext.exl3_gemm as called at orcasaq2/ops.py:46-49 for rows == 1 (the other row
// counts take gemv.hip's MFMA kernels).
//
// Work decomposition.  A *unit* is one tile row of one 128-output column group: 8 tiles
// side by side, 64 chunks of 32 positions -- one chunk per lane of a wave, the 8 tiles'
// words one contiguous run of 64K u32 in HBM.  Units are numbered shard-major, then
// column group, then tile row, and the whole launch's units are cut into G nearly equal
// contiguous ranges, one per workgroup (G = a few workgroups per CU, all resident at
// once: there is no tail wave of workgroups).  A workgroup's range touches a few
// *segments* (shard, column group); its eight waves take eight contiguous runs of it.
//
// Per wave:
//   1. issue the loads of its first D units (D = 2..6 by K): the lane's K trellis words and
//      its x and suh dwords of the unit's 128-input block, so HBM is busy from the start;
//   2. main loop over the run: a unit's data streams through the D-deep register ring.
//      Entering a new 128-input block (every 8 units), the wave transforms it,
//      fp16(H128(x * suh)), and keeps the 128 results as one fp16 pair per lane; a unit of
//      tile row t fetches lane 8t + l % 8's pair (one ds_bpermute) and duplicates each half.
//      The tail-biting word before a lane's chunk is the previous lane's last word (DPP
//      rotate within the tile's 8 lanes).  Each position is decoded with an SDWA add (or a
//      16-bit field for MCG), a v_mul_lo_u32 and a v_bitop3; the masked word meets its
//      activation in a v_dot2c_f32_f16 whose second operand is broadcast by DPP from the lane
//      that holds that activation row (both fp16 halves times x, summed in fp32);
//   3. per segment, the waves' partial sums are added in a fixed order through LDS.  If the
//      segment lies inside this workgroup's range it is finished here; otherwise the
//      partial goes to this workgroup's slot with agent-coherent stores, and the last of the
//      segment's workgroups to arrive (a relaxed agent-scope counter in the workspace) has
//      its eight waves add all slots (a fixed partition and order: deterministic) and
//      finishes: output Hadamard, * svh, fp16 store, counter back to 0.  No cache-wide
//      release/acquire is used: the slots are written with agent-scope stores and read
//      with agent-scope loads, and each writer waits for its stores to complete before it
//      increments the counter.
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

constexpr int G1_NW = 8;                 // waves per workgroup
constexpr int G1_MAXSH = 8;              // shards per launch
constexpr int G1_WG_PER_CU = 4;          // target resident workgroups per CU (8 waves / SIMD)
constexpr int G1_GMAX = 2048;            // workgroups per launch (bounds the slot area)

// Prefetch depth in units: about 24 VGPRs of loads in flight per lane whatever K is (a unit
// is K trellis words and an activation pair per lane), 2..6 units.
constexpr int g1_depth(int K) { return (24 / (K + 3)) < 2 ? 2 : (24 / (K + 3)) > 6 ? 6 : (24 / (K + 3)); }

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

// Division by a launch constant d >= 2 of any x < 2^31 without a division routine (the
// scalar unit is shared by every wave of a CU, and a 64-bit division is ~130 of its
// instructions): floor(x / d) = floor(x * m / 2^(31 + l)), l = ceil(log2 d),
// m = floor(2^(31 + l) / d) + 1 < 2^32 (Granlund and Montgomery, PLDI 1994, Thm 4.2 with
// N = 31).
struct G1Div {
    uint32_t m;
    int sh;                    // l - 1
};

__device__ __forceinline__ int g1_div(int x, G1Div d)
{
    return (int)(__umulhi((uint32_t)x, d.m) >> d.sh);
}

struct G1Args {
    const uint16_t* x;         // (ic) fp16
    uint32_t* counters;        // one per segment; zero between calls
    float* slots;              // (G + segments) x 128 fp32
    int U, G, ntr, nshards, nsegs;
    int q, r;                  // U = q G + r: workgroup g owns q + (g < r) units
    G1Div dntr, dq, dq1;       // division by ntr, q, q + 1
    G1Shard sh[G1_MAXSH];
};

// First unit of workgroup g: the first r workgroups own q + 1 units, the others q.
__device__ __forceinline__ int g1_first_unit(const G1Args& a, int g)
{
    return g * a.q + min(g, a.r);
}

// Workgroup whose unit range holds unit u.
__device__ __forceinline__ int g1_wg_of(const G1Args& a, int u)
{
    const int big = a.r * (a.q + 1);
    return u < big ? g1_div(u, a.dq1) : a.r + g1_div(u - big, a.dq);
}

// Shard holding segment S / unit u.  Every table entry is read at a constant offset, so the
// scalar loads of the whole table issue together instead of as a chain of dependent loads
// (each a few hundred cycles); a single-shard launch (ONE) reads nothing.
template <bool ONE>
__device__ __forceinline__ int g1_shard_of_seg(const G1Args& a, int S)
{
    int s = 0;
    if constexpr (!ONE) {
#pragma unroll
        for (int i = 1; i < G1_MAXSH; i++)
            if (i < a.nshards && S >= a.sh[i].sbeg) s = i;
    }
    return s;
}

template <bool ONE>
__device__ __forceinline__ int g1_shard_of_unit(const G1Args& a, int u)
{
    int s = 0;
    if constexpr (!ONE) {
#pragma unroll
        for (int i = 1; i < G1_MAXSH; i++)
            if (i < a.nshards && u >= a.sh[i].ubeg) s = i;
    }
    return s;
}

__device__ __forceinline__ float g1_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float g1_hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }

// A lane's K words w[1..K] of a unit (lane l's chunk starts at word lk = K l), in the
// widest loads their 4-byte alignment allows (dwordx4/x3/x2).
template <int K>
__device__ __forceinline__ void g1_load(uint32_t (&w)[K + 1], const uint32_t* __restrict__ unit, uint32_t lk)
{
    typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const uint32_t* p = unit + lk;
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

__device__ __forceinline__ uint32_t g1_dup(float v)
{
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)v);
    return h | (h << 16);
}

// ---------------------------------------------------------------- decode kernel

// Eight waves per SIMD need at most 64 VGPRs (measured on MI355X: 68 VGPRs leave room for
// only 6); the SGPR cap keeps the count well inside what eight waves per SIMD may hold.
template <int K, int CB, bool ONE>
__global__ __launch_bounds__(64 * G1_NW) __attribute__((amdgpu_waves_per_eu(8, 8), amdgpu_num_sgpr(74))) void gemv1_kernel(const G1Args a)
{
    // shard table entry; a single-shard launch (ONE) only ever reads entry 0 (constant offsets)
    auto sh = [&](int s) -> const G1Shard& { return a.sh[ONE ? 0 : s]; };
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    constexpr int D = g1_depth(K);

    const int g = blockIdx.x;
    const int ntr = a.ntr;
    const int ub = g1_first_unit(a, g), L = a.q + (g < a.r ? 1 : 0);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;

    // ---- this wave's units: the contiguous run ub + lo .. ub + lo + n - 1 of the range
    const int lo = (wave * L) >> 3;
    const int n = (((wave + 1) * L) >> 3) - lo;
    const uint32_t lk = lane * K;
    const bool first_lane = (lane & 7) == 0;

    // Wave-uniform cursor over the wave's units: shard, column group, tile row, segment and
    // the first word of the unit's 8 tiles.  Consecutive units are consecutive tile rows
    // (ntr >= 8); only a column-group crossing reads the shard table again.
    struct Cursor {
        int s, cg, tr, S;
        long stride;   // words between consecutive tile rows
        const uint32_t* p;
    };
    auto seat = [&](Cursor& q) {
        q.stride = (long)sh(q.s).oc16 * (8 * K);
        q.p = sh(q.s).trellis + ((long)q.tr * sh(q.s).oc16 + 8 * q.cg) * (8 * K);
    };
    auto cursor_at = [&](int u) {
        Cursor q;
        q.s = g1_shard_of_unit<ONE>(a, u);
        const int rel = u - sh(q.s).ubeg;
        q.cg = g1_div(rel, a.dntr);
        q.tr = rel - q.cg * ntr;
        q.S = sh(q.s).sbeg + q.cg;
        seat(q);
        return q;
    };
    auto advance = [&](Cursor& q) {
        q.tr++;
        q.p += q.stride;
        if (q.tr == ntr) {
            q.tr = 0;
            q.S++;
            if (++q.cg == sh(q.s).ncg) {
                q.s++;
                q.cg = 0;
            }
            seat(q);
        }
    };

    // A unit's loads: the lane's K words, and the lane's x and suh dword of the unit's
    // 128-input block (used when the unit starts a new block).  Prefetch cursor (D units
    // ahead; it stops at the wave's last unit, whose data is then loaded again and not used)
    // and processing cursor.
    struct Slot {
        uint32_t w[K + 1];
        uint32_t xw, sw;
    };
    auto load = [&](Slot& sl, const Cursor& q) {
        g1_load<K>(sl.w, q.p, lk);
        const int blk = q.tr >> 3;
        sl.xw = reinterpret_cast<const uint32_t*>(a.x + blk * 128)[lane];
        sl.sw = reinterpret_cast<const uint32_t*>(sh(q.s).suh + blk * 128)[lane];
    };
    Cursor pf = cursor_at(ub + lo), cu = pf;
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

    // ---- this workgroup's segments: S_first .. S_first + nseg - 1
    const int s_first = g1_shard_of_unit<ONE>(a, ub);
    const int S_first = sh(s_first).sbeg + g1_div(ub - sh(s_first).ubeg, a.dntr);
    const int nseg = [&] {
        const int u = ub + L - 1;
        const int s = g1_shard_of_unit<ONE>(a, u);
        return sh(s).sbeg + g1_div(u - sh(s).ubeg, a.dntr) - S_first + 1;
    }();
    // LDS: red[nseg][G1_NW][128] fp32 partial rows | last[nseg] flags
    float* red = reinterpret_cast<float*>(lds);
    int* last = reinterpret_cast<int*>(red + nseg * G1_NW * 128);
    for (int k = 0; k < nseg; k++)
        *reinterpret_cast<float2*>(red + (k * G1_NW + wave) * 128 + 2 * lane) = float2{0.f, 0.f};
    const Dot2Consts kc = dot2_consts();

    // ---- main loop.  Scalar bookkeeping (cursor steps, column-group crossings, flushes of a
    // finished segment's sums to the wave's LDS row) sits between units, so each unit's work
    // is one basic block the scheduler can interleave; the loads sit outside every branch,
    // so the wait before a unit covers only that unit's own loads.
    //
    // Activations: when a unit enters a new 128-input block (every 8 units, or at a shard or
    // column-group change) the wave transforms the block, fp16(H128(x * suh)) across the wave
    // (lane l: outputs 2l, 2l + 1 = rows 2(l % 8), 2(l % 8) + 1 of tile row l / 8, kept as an
    // fp16 pair); a unit of tile row t then reads lane 8t + l % 8's pair and duplicates each
    // half for the v_dot2c broadcasts.
    const int o0 = (lane >> 3) * 16 + (lane & 7);
    float y0 = 0.f, y1 = 0.f;
    int cur = cu.S - S_first;
    auto flush = [&](int k) {
        red[(cur * G1_NW + wave) * 128 + o0] = y0;
        red[(cur * G1_NW + wave) * 128 + o0 + 8] = y1;
        y0 = y1 = 0.f;
        cur = k;
    };
    uint32_t bact = 0;
    int bkey = -1;                            // (shard, block) of bact
    for (int j = 0; j < n; j += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            if (d == 0 || j + d < n) {
                if (cu.S - S_first != cur) flush(cu.S - S_first);
                const int key = (cu.s << 24) | (cu.tr >> 3);
                if (key != bkey) {
                    bkey = key;
                    float v0 = g1_lo(ring[d].xw) * g1_lo(ring[d].sw), v1 = g1_hi(ring[d].xw) * g1_hi(ring[d].sw);
                    wave_fwht128(v0, v1);
                    bact = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v0) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v1) << 16);
                }
                const uint32_t pr = (uint32_t)__builtin_amdgcn_ds_bpermute(((cu.tr & 7) * 8 + (lane & 7)) * 4, (int)bact);
                const uint32_t a0 = __builtin_amdgcn_perm(pr, pr, 0x01000100u);
                const uint32_t a1 = __builtin_amdgcn_perm(pr, pr, 0x03020302u);
                chunk_prev_dpp<K>(ring[d].w, first_lane);
                float acc[4] = {0.f, 0.f, 0.f, 0.f};
                dot2_chunk<K, CB>(ring[d].w, a0, a1, acc, kc);
                y0 += acc[0] + acc[1];
                y1 += acc[2] + acc[3];
                if (j + d + 1 < n) advance(cu);
            }
            load(ring[d], next_pf());
        }
    }
    if (n > 0) flush(cur);
    __syncthreads();

    // ---- per segment: fixed-order sum of the waves; finish here, or via the slots
    auto finish = [&](int k, float v0, float v1) {
        const int S = S_first + k;
        const int s = g1_shard_of_seg<ONE>(a, S);
        const int cg = S - sh(s).sbeg;
        wave_fwht128(v0, v1);
        const uint32_t sv = reinterpret_cast<const uint32_t*>(sh(s).svh + cg * 128)[lane];
        v0 *= g1_lo(sv);
        v1 *= g1_hi(sv);
        const uint32_t out = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v0) |
                             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v1) << 16);
        reinterpret_cast<uint32_t*>(sh(s).C + cg * 128)[lane] = out;
    };
    auto contributors = [&](int k, int& g_lo, int& g_hi) {
        const int S = S_first + k;
        const int s = g1_shard_of_seg<ONE>(a, S);
        const int segU0 = sh(s).ubeg + (S - sh(s).sbeg) * ntr;
        g_lo = g1_wg_of(a, segU0);
        g_hi = g1_wg_of(a, segU0 + ntr - 1);
    };
    bool any_last = false;
    for (int k = wave; k < nseg; k += G1_NW) {
        float v0 = 0.f, v1 = 0.f;
#pragma unroll
        for (int ww = 0; ww < G1_NW; ww++) {
            const float2 p = *reinterpret_cast<const float2*>(red + (k * G1_NW + ww) * 128 + 2 * lane);
            v0 += p.x;
            v1 += p.y;
        }
        int g_lo, g_hi;
        contributors(k, g_lo, g_hi);
        int is_last = 0;
        if (g_hi > g_lo) {
            uint64_t* my = reinterpret_cast<uint64_t*>(a.slots + (long)(S_first + k + g) * 128) + lane;
            const uint64_t pv = (uint64_t)__builtin_bit_cast(uint32_t, v0) |
                                ((uint64_t)__builtin_bit_cast(uint32_t, v1) << 32);
            __hip_atomic_store(my, pv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);   // this wave's slot stores are complete
            uint32_t old = 0;
            if (lane == 0)
                old = __hip_atomic_fetch_add(a.counters + S_first + k, 1u, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
            old = __shfl(old, 0, 64);
            // last to arrive: every other contributor's slot stores completed before its
            // counter increment, which precedes ours
            is_last = old == (uint32_t)(g_hi - g_lo);
            if (is_last && lane == 0)
                __hip_atomic_store(a.counters + S_first + k, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            finish(k, v0, v1);
        }
        if (lane == 0) last[k] = is_last;
        any_last |= is_last != 0;
    }
    // Segments this workgroup completes for everyone: the eight waves add the slots (wave w
    // takes slots g_lo + w, g_lo + w + 8, ... in order), then wave k adds the eight sums.
    if (__syncthreads_or(any_last)) {
        for (int k = 0; k < nseg; k++) {
            if (!last[k]) continue;
            int g_lo, g_hi;
            contributors(k, g_lo, g_hi);
            const int nsl = g_hi - g_lo + 1;
            const uint64_t* sl = reinterpret_cast<const uint64_t*>(a.slots + (long)(S_first + k + g_lo) * 128) + lane;
            float v0 = 0.f, v1 = 0.f;
            for (int t0 = wave; t0 < nsl; t0 += 8 * G1_NW) {
                uint64_t xv[8];
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const int gg = min(t0 + t * G1_NW, nsl - 1);
                    xv[t] = __hip_atomic_load(sl + (long)gg * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    if (t0 + t * G1_NW < nsl) {
                        v0 += __builtin_bit_cast(float, (uint32_t)xv[t]);
                        v1 += __builtin_bit_cast(float, (uint32_t)(xv[t] >> 32));
                    }
                }
            }
            *reinterpret_cast<float2*>(red + (k * G1_NW + wave) * 128 + 2 * lane) = float2{v0, v1};
        }
        __syncthreads();
        for (int k = wave; k < nseg; k += G1_NW) {
            if (!last[k]) continue;
            float v0 = 0.f, v1 = 0.f;
#pragma unroll
            for (int ww = 0; ww < G1_NW; ww++) {
                const float2 p = *reinterpret_cast<const float2*>(red + (k * G1_NW + ww) * 128 + 2 * lane);
                v0 += p.x;
                v1 += p.y;
            }
            finish(k, v0, v1);
        }
    }
}

// ---------------------------------------------------------------- host side

template <int K, int CB>
static const void* g1_fn(bool one)
{
    return one ? reinterpret_cast<const void*>(&gemv1_kernel<K, CB, true>)
               : reinterpret_cast<const void*>(&gemv1_kernel<K, CB, false>);
}

static const void* g1_fn_kcb(int K, int cb, bool one)
{
#define EXL3_CASE(KK) case KK: return cb == CB_MCG ? g1_fn<KK, CB_MCG>(one) : g1_fn<KK, CB_3INST>(one);
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

static G1Div g1_magic(uint32_t d)
{
    int l = 0;
    while ((1ull << l) < d) l++;
    return G1Div{(uint32_t)(((1ull << (31 + l)) / d) + 1), l - 1};
}

// Dynamic LDS a launch needs: a partial row per wave and a flag for the most segments
// (shard, column group) a workgroup range of ceil(U / G) units can touch.
static size_t g1_lds_bytes(int U, int G, int ntr)
{
    const int L = (U + G - 1) / G;
    const int nseg = (L - 1 + ntr - 1) / ntr + 1;
    return (size_t)nseg * (G1_NW * 128 * sizeof(float) + 4);
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
        const int G = (int)std::min<long>(gmax, std::max<long>(1, U / G1_NW));
        const size_t lds = g1_lds_bytes((int)U, G, ntr);
        const size_t need = (size_t)(G + nsegs) * 128 * sizeof(float);
        if (sbase + need > slot_bytes)
            return set_error(EXL3_ERR_WORKSPACE, "exl3_gemv: slot area of %zu bytes, %zu needed", slot_bytes,
                             sbase + need);
        args.U = (int)U;
        args.G = G;
        args.q = (int)(U / G);
        args.r = (int)(U % G);
        // divisors are >= 8 (ntr = ic / 16 with ic >= 128; G <= U / 8), as g1_div requires
        args.dntr = g1_magic((uint32_t)ntr);
        args.dq = g1_magic((uint32_t)args.q);
        args.dq1 = g1_magic((uint32_t)args.q + 1);
        args.nsegs = nsegs;
        args.counters = counters + cbase;
        args.slots = reinterpret_cast<float*>(slots + sbase);
        cbase += nsegs;
        sbase += need;
        const void* fn = g1_fn_kcb(shards[i].K, shards[i].cb, args.nshards == 1);
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
