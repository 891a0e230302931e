// Fused EXL3 decode-GEMV for one to four activation rows (batch-1..4 decode):
//   y_r (oc) = fp16( H( fp16(H(x_r * suh)) . W_q ) * svh ),  r < nrows
// with W_q decoded from the packed trellis in registers and never stored.  Replaces
// exllamav3_ext.exl3_gemm as called at orcasaq2/ops.py:46-49 for rows <= 4 (rows 2..4 only
// where the launch keeps three workgroups per CU resident; gemv.hip's split kernels take
// the rest, gemm_sk.hip's 16-row tiles take 5..16 rows).
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
//   1. the workgroup transforms the activation blocks its range meets, fp16(H128(x_r * suh))
//      for every row r, into an LDS table of duplicated fp16 pairs; then each wave issues the
//      loads of its first unit;
//   2. main loop over the run: each unit's loads are issued in the previous unit's
//      iteration (g1_depth: one unit in flight per wave, eight waves per SIMD).
//      The tail-biting word before a lane's chunk is the previous lane's last word (DPP
//      rotate within the tile's 8 lanes).  Each position is decoded with three VALU ops
//      (dot2_word); the masked words go into the B operand of v_mfma_f32_16x16x32_f16
//      (each word's two fp16 halves as two k-slots against one activation twice, so
//      lo * x + hi * x is summed in fp32) and the unit's activations into A (g1_mfma16),
//      one MFMA serving up to four activation rows.  A wave's priority steps down as its
//      run progresses (s_setprio 3 -> 0): the sequencer otherwise issues the oldest waves
//      first, the youngest workgroup on each CU starts its loop last, and the launch ends
//      with that workgroup running alone;
//   3. per segment, the waves' partial sums are added in a fixed order through LDS.  If the
//      segment lies inside this workgroup's range it is finished here (output Hadamard,
//      * svh, fp16 store); otherwise the partial goes to this workgroup's slot in the
//      workspace, and gemv1_finish_kernel, enqueued right after the launch, adds each split
//      segment's slots in workgroup order (deterministic) and finishes it.  The kernel
//      boundary orders the slot stores before the reads: no counters, fences or waits
//      inside the launch (measured on MI355X against a last-arriving-workgroup finish with
//      agent-scope stores and a counter: 4-9% faster on every 27B projection shape).
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

constexpr int G1_NW = 8;                 // waves per workgroup
constexpr int G1_MAXSH = 8;              // shards per launch
constexpr int G1_WG_PER_CU = 4;          // target resident workgroups per CU (8 waves / SIMD)
constexpr int G1_GMAX = 2048;            // workgroups per launch (bounds the slot area)

// Units a wave keeps in flight: one.  Eight waves per SIMD already keep enough loads in
// flight, and every unit more per wave lengthens the memory queues that a launch's first
// units and activation loads wait behind: measured on MI355X (down_proj, per call), depth 1
// against 2 and against 24 / (K + 3) clamped to 2..6: K = 2 18.6 / 18.7 / 19.6 us, K = 3
// 18.9 / 19.6 / 20.9, K = 4 19.4 / 19.8 / 20.7, K = 5 19.4 / 20.4 / 21.4.
constexpr int g1_depth(int) { return 1; }

struct G1Shard {
    const uint32_t* trellis;   // (ic/16, oc/16, 8K) u32
    const uint16_t* suh;       // (ic)
    const uint16_t* svh;       // (oc)
    uint16_t* C;               // (nrows, ldc) fp16 output, columns [0, oc)
    long ldc;
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

// One group of shards with the same K and codebook, decoded by G workgroups.
struct G1Group {
    const uint16_t* x;         // (nrows, ic) fp16
    int nrows;                 // activation rows, 1 .. R of the kernel
    float* slots;              // (G + segments) x R x 128 fp32 partials of split segments
    int U, G, ntr, nshards, nsegs;
    int q, r;                  // U = q G + r: workgroup g owns q + (g < r) units
    G1Div dntr, dq, dq1;       // division by ntr, q, q + 1
};

// A launch of one group (shards 0 .. nshards - 1 of the table).
struct G1Args {
    G1Group grp;
    G1Shard sh[G1_MAXSH];
};

// A launch of several groups of one codebook, one K each: group i owns workgroups
// gbeg[i] .. gbeg[i + 1] - 1 and shards sh0[i] .. sh0[i] + grp[i].nshards - 1; in the finish
// kernel it owns blocks fbeg[i] .. fbeg[i] + grp[i].nsegs - 1 (one per segment).
struct G1Multi {
    G1Group grp[G1_MAXSH];
    G1Shard sh[G1_MAXSH];
    int gbeg[G1_MAXSH], sh0[G1_MAXSH], K[G1_MAXSH], fbeg[G1_MAXSH];
    int ngrp;
};

// First unit of workgroup g: the first r workgroups own q + 1 units, the others q.
__device__ __forceinline__ int g1_first_unit(const G1Group& a, int g)
{
    return g * a.q + min(g, a.r);
}

// Workgroup whose unit range holds unit u.
__device__ __forceinline__ int g1_wg_of(const G1Group& a, int u)
{
    const int big = a.r * (a.q + 1);
    return u < big ? g1_div(u, a.dq1) : a.r + g1_div(u - big, a.dq);
}

// Shard holding segment S / unit u.  Every table entry is read at a constant offset, so the
// scalar loads of the whole table issue together instead of as a chain of dependent loads
// (each a few hundred cycles); a single-shard launch (ONE) reads nothing.
template <bool ONE>
__device__ __forceinline__ int g1_shard_of_seg(const G1Group& a, const G1Shard* sht, int S)
{
    int s = 0;
    if constexpr (!ONE) {
#pragma unroll
        for (int i = 1; i < G1_MAXSH; i++)
            if (i < a.nshards && S >= sht[i].sbeg) s = i;
    }
    return s;
}

template <bool ONE>
__device__ __forceinline__ int g1_shard_of_unit(const G1Group& a, const G1Shard* sht, int u)
{
    int s = 0;
    if constexpr (!ONE) {
#pragma unroll
        for (int i = 1; i < G1_MAXSH; i++)
            if (i < a.nshards && u >= sht[i].ubeg) s = i;
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

// One lane's chunk (32 positions) multiplied into its two output columns with eight
// v_mfma_f32_16x16x32_f16.  The unit's 64 lanes are four groups j = l / 16 of two tiles
// (tiles 2j, 2j + 1, one tile row); lane l supplies B column n = l % 16 of k-block j: the
// masked codebook words of four positions, each word's two fp16 halves as two k-slots against
// one activation twice -- so the weight's fp16 half-sum is never rounded.  MFMA (m, h) takes
// positions 8m + 4h + t (t = 0..3): rows 2m + {0, 1, 8, 9} of the tile row, column c + 8h of
// the chunk.  A row i = 4r + j holds activation row r of those four rows (duplicated) in
// k-block j and zeros in the other k-blocks, so C row 4r + j sums group j alone: C[4r + j][n]
// (lane 16r + n, element j) is activation row r's partial for output 32j + 16(n / 8) + n % 8
// + 8h of the unit's 128.  The MFMA's long latency lets other waves' decode VALU work issue
// beside it (on MI355X it hides most of its 15 cycles; a v_mfma_f32_4x4x4_16b_f16 form with
// twice the instructions hid under half of its 8).
template <int K, int CB, int M, int H>
__device__ __forceinline__ void g1_mfma16(const uint32_t (&w)[K + 1], const f16x8& a, f32x4 (&acc)[2],
                                          const Dot2Consts& kc)
{
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    constexpr int q = 8 * M + 4 * H;
    const u4 b = {dot2_word<K, CB, q>(w, kc), dot2_word<K, CB, q + 1>(w, kc), dot2_word<K, CB, q + 2>(w, kc),
                  dot2_word<K, CB, q + 3>(w, kc)};
    acc[H] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(f16x8, b), acc[H], 0, 0, 0);
}

template <int K, int CB>
__device__ __forceinline__ void g1_mfma_chunk(const uint32_t (&w)[K + 1], const f16x8 (&a)[4], f32x4 (&acc)[2],
                                              const Dot2Consts& kc)
{
    g1_mfma16<K, CB, 0, 0>(w, a[0], acc, kc);
    g1_mfma16<K, CB, 0, 1>(w, a[0], acc, kc);
    g1_mfma16<K, CB, 1, 0>(w, a[1], acc, kc);
    g1_mfma16<K, CB, 1, 1>(w, a[1], acc, kc);
    g1_mfma16<K, CB, 2, 0>(w, a[2], acc, kc);
    g1_mfma16<K, CB, 2, 1>(w, a[2], acc, kc);
    g1_mfma16<K, CB, 3, 0>(w, a[3], acc, kc);
    g1_mfma16<K, CB, 3, 1>(w, a[3], acc, kc);
}

__device__ __forceinline__ uint32_t g1_dup(float v)
{
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)v);
    return h | (h << 16);
}

// ---------------------------------------------------------------- decode kernel

// Workgroup g of group a (shard table sht) -- the whole kernel body.
template <int K, int CB, bool ONE, int R>
__device__ __forceinline__ void g1_body(const G1Group& a, const G1Shard* sht, const int g, uint32_t* lds)
{
    // shard table entry; a single-shard group (ONE) only ever reads entry 0
    auto sh = [&](int s) -> const G1Shard& { return sht[ONE ? 0 : s]; };
    constexpr int D = g1_depth(K);

    const int ntr = a.ntr;
    const int ub = g1_first_unit(a, g), L = a.q + (g < a.r ? 1 : 0);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    __builtin_amdgcn_s_setprio(3);

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
        q.s = g1_shard_of_unit<ONE>(a, sht, u);
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

    // A unit's loads: the lane's K words.  Prefetch cursor (D units ahead; it stops at the
    // wave's last unit, whose data is then loaded again and not used) and processing cursor.
    // D = g1_depth(K) = 1 on MI355X; the ring stays general.
    struct Slot {
        uint32_t w[K + 1];
    };
    auto load = [&](Slot& sl, const Cursor& q) { g1_load<K>(sl.w, q.p, lk); };
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

    // ---- this workgroup's segments: S_first .. S_first + nseg - 1
    const int s_first = g1_shard_of_unit<ONE>(a, sht, ub);
    const int S_first = sh(s_first).sbeg + g1_div(ub - sh(s_first).ubeg, a.dntr);
    const int nseg = [&] {
        const int u = ub + L - 1;
        const int s = g1_shard_of_unit<ONE>(a, sht, u);
        return sh(s).sbeg + g1_div(u - sh(s).ubeg, a.dntr) - S_first + 1;
    }();
    // The range's 128-input blocks in the order its units meet them ("occurrences"): the
    // first segment's tile rows tr0 .. tre0 (blocks tr0 / 8 .. tre0 / 8), then every later
    // segment from tile row 0 on (ntr / 8 blocks each, the last one possibly fewer).
    // Occurrence of unit (segment S_first + k, tile row tr): see occ_of.
    const int tr0 = ub - sh(s_first).ubeg - (S_first - sh(s_first).sbeg) * ntr;
    const int nbpc = ntr >> 3;
    const int nb0 = (min(ntr - 1, tr0 + L - 1) >> 3) - (tr0 >> 3) + 1;
    auto occ_of = [&](int k, int tr) { return k == 0 ? (tr >> 3) - (tr0 >> 3) : nb0 + (k - 1) * nbpc + (tr >> 3); };
    const int nocc = [&] {
        const int u = ub + L - 1;
        const int s = g1_shard_of_unit<ONE>(a, sht, u);
        const int rel = u - sh(s).ubeg;
        const int cg = g1_div(rel, a.dntr);
        return occ_of(sh(s).sbeg + cg - S_first, rel - cg * ntr) + 1;
    }();

    // LDS: red[nseg][G1_NW][R][128] fp32 partial rows | act[nocc][8][R][16] duplicated fp16
    // activations | zero[16] (the A operand of the lanes whose k-block is not theirs)
    float* red = reinterpret_cast<float*>(lds);
    uint32_t* act = reinterpret_cast<uint32_t*>(red + nseg * G1_NW * R * 128);
    uint32_t* zero = act + nocc * R * 128;
    if (threadIdx.x < 16) zero[threadIdx.x] = 0u;
    for (int k = 0; k < nseg; k++)
#pragma unroll
        for (int r = 0; r < R; r++)
            *reinterpret_cast<float2*>(red + ((k * G1_NW + wave) * R + r) * 128 + 2 * lane) = float2{0.f, 0.f};
    const Dot2Consts kc = dot2_consts();
    const long ic = (long)ntr * 16;

    // Activations, once per workgroup: the waves share out the occurrences; each transforms its block of every activation row r,
    // fp16(H128(x_r * suh)) (lane l: outputs 2l, 2l + 1 = rows 2(l % 8), 2(l % 8) + 1 of the
    // block's tile row l / 8) and stores each output as a duplicated fp16 pair in the order
    // the MFMAs read them: act[occurrence][tile row][r][m][t] holds row 2m + {0, 1, 8, 9}[t]
    // (so lane l's two rows go to m = l % 4, t = 2 ((l % 8) / 4) and t + 1).  Rows
    // r >= nrows repeat the last row (their results are not stored).
    for (int i = wave; i < nocc; i += G1_NW) {
        int k = 0, blk = (tr0 >> 3) + i;
        if (i >= nb0) {
            const int j = i - nb0;
            k = 1 + g1_div(8 * j, a.dntr);          // j / nbpc
            blk = j - (k - 1) * nbpc;
        }
        const int s = g1_shard_of_seg<ONE>(a, sht, S_first + k);
        const uint32_t sw = reinterpret_cast<const uint32_t*>(sh(s).suh + blk * 128)[lane];
#pragma unroll 1
        for (int r = 0; r < R; r++) {
            const uint32_t xw = reinterpret_cast<const uint32_t*>(a.x + min(r, a.nrows - 1) * ic + blk * 128)[lane];
            float v0 = g1_lo(xw) * g1_lo(sw), v1 = g1_hi(xw) * g1_hi(sw);
            wave_fwht128(v0, v1);
            *reinterpret_cast<uint2*>(act + ((i * 8 + (lane >> 3)) * R + r) * 16 + 4 * (lane & 3) + 2 * ((lane >> 2) & 1)) =
                uint2{g1_dup(v0), g1_dup(v1)};
        }
    }
    // The first unit's loads go out after the wave's activation loads have returned, so those
    // never wait behind a launch-wide burst of trellis loads (measured: 0.1-0.2 us per call
    // faster at every K than issuing them first).
    if (n > 0) {
        load(ring[0], pf);
#pragma unroll
        for (int d = 1; d < D; d++) load(ring[d], next_pf());
    }
    __syncthreads();

    // ---- main loop.  Scalar bookkeeping (cursor steps, column-group crossings, flushes of a
    // finished segment's sums to the wave's LDS row) sits between units, so each unit's work
    // is one basic block the scheduler can interleave; the loads sit outside every branch,
    // so the wait before a unit covers only that unit's own loads.  The occurrence index
    // steps whenever a unit starts a block (its tile row a multiple of 8, which includes
    // every segment start).
    // yacc[h][e] of lane 16r + n: activation row r's sum for output 32e + 16(n / 8) + n % 8 + 8h
    // (lanes 16r + n with r >= R hold copies of row R - 1).
    f32x4 yacc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    const int yrow = lane >> 4, ycol = 16 * ((lane >> 3) & 1) + (lane & 7);
    // This lane's A operand: row i = lane % 16 in k-block lane / 16, which carries activation
    // row i / 4 when i % 4 is that k-block and zeros otherwise.  Its LDS byte address for a
    // unit whose table entry starts at byte e: e * asel + aoff.
    const uint32_t asel = ((lane & 15) & 3) == (lane >> 4) ? 1u : 0u;
    const uint32_t aoff = asel ? (uint32_t)((reinterpret_cast<char*>(act) - reinterpret_cast<char*>(lds)) +
                                            min((lane & 15) >> 2, R - 1) * 64)
                               : (uint32_t)(reinterpret_cast<char*>(zero) - reinterpret_cast<char*>(lds));
    int cur = cu.S - S_first;
    int occ = occ_of(cur, cu.tr);
    const int pq1 = (n + 3) >> 2, pq2 = (n + 1) >> 1, pq3 = (3 * n + 3) >> 2;
    auto flush = [&](int k) {
        if (yrow < R) {
            float* rr = red + ((cur * G1_NW + wave) * R + yrow) * 128 + ycol;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                rr[32 * e] = yacc[0][e];
                rr[32 * e + 8] = yacc[1][e];
            }
        }
        yacc[0] = yacc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
        cur = k;
    };
    for (int j = 0; j < n; j += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            if (d == 0 || j + d < n) {
                if (cu.S - S_first != cur) flush(cu.S - S_first);
                const uint32_t e = (uint32_t)((occ * 8 + (cu.tr & 7)) * R) * 64u;
                const f16x8* ap = reinterpret_cast<const f16x8*>(reinterpret_cast<const char*>(lds) + (__umul24(e, asel) + aoff));
                const f16x8 av[4] = {ap[0], ap[1], ap[2], ap[3]};
                chunk_prev_dpp<K>(ring[d].w, first_lane);
                g1_mfma_chunk<K, CB>(ring[d].w, av, yacc, kc);
                if (j + d + 1 < n) {
                    advance(cu);
                    occ += (cu.tr & 7) == 0;
                }
                // priority 3, 2, 1, 0 over the run's four quarters
                const int done = j + d + 1;
                if (done == pq1) __builtin_amdgcn_s_setprio(2);
                if (done == pq2) __builtin_amdgcn_s_setprio(1);
                if (done == pq3) __builtin_amdgcn_s_setprio(0);
            }
            load(ring[d], next_pf());
        }
    }
    __builtin_amdgcn_s_setprio(3);
    if (n > 0) flush(cur);
    __syncthreads();

    // ---- per segment: fixed-order sum of the waves; finish here, or via the slots
    auto finish = [&](int k, int r, float v0, float v1) {
        const int S = S_first + k;
        const int s = g1_shard_of_seg<ONE>(a, sht, S);
        const int cg = S - sh(s).sbeg;
        wave_fwht128(v0, v1);
        const uint32_t sv = reinterpret_cast<const uint32_t*>(sh(s).svh + cg * 128)[lane];
        v0 *= g1_lo(sv);
        v1 *= g1_hi(sv);
        const uint32_t out = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v0) |
                             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v1) << 16);
        reinterpret_cast<uint32_t*>(sh(s).C + r * sh(s).ldc + cg * 128)[lane] = out;
    };
    auto contributors = [&](int k, int& g_lo, int& g_hi) {
        const int S = S_first + k;
        const int s = g1_shard_of_seg<ONE>(a, sht, S);
        const int segU0 = sh(s).ubeg + (S - sh(s).sbeg) * ntr;
        g_lo = g1_wg_of(a, segU0);
        g_hi = g1_wg_of(a, segU0 + ntr - 1);
    };
    const int nr = R == 1 ? 1 : a.nrows;
    for (int k = wave; k < nseg; k += G1_NW) {
        float v0[R], v1[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            v0[r] = v1[r] = 0.f;
#pragma unroll
            for (int ww = 0; ww < G1_NW; ww++) {
                const float2 p = *reinterpret_cast<const float2*>(red + ((k * G1_NW + ww) * R + r) * 128 + 2 * lane);
                v0[r] += p.x;
                v1[r] += p.y;
            }
        }
        int g_lo, g_hi;
        contributors(k, g_lo, g_hi);
        if (g_hi > g_lo) {
            // split segment: slot (S + g) holds this workgroup's R rows of 128 partials, which
            // gemv1_finish_kernel adds after the launch
            uint64_t* my = reinterpret_cast<uint64_t*>(a.slots + (long)(S_first + k + g) * R * 128) + lane;
#pragma unroll
            for (int r = 0; r < R; r++)
                my[r * 64] = (uint64_t)__builtin_bit_cast(uint32_t, v0[r]) |
                             ((uint64_t)__builtin_bit_cast(uint32_t, v1[r]) << 32);
        } else {
            for (int r = 0; r < nr; r++) finish(k, r, v0[r], v1[r]);
        }
    }
}

// Eight waves per SIMD need at most 64 VGPRs (measured on MI355X: 68 VGPRs leave room for
// only 6); the SGPR cap keeps the count well inside what eight waves per SIMD may hold.
template <int K, int CB, bool ONE, int R>
__global__ __launch_bounds__(64 * G1_NW) __attribute__((amdgpu_waves_per_eu(8, 8), amdgpu_num_sgpr(74))) void gemv1_kernel(const G1Args a)
{
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    g1_body<K, CB, ONE, R>(a.grp, a.sh, blockIdx.x, lds);
}

// Several groups (different K) in one launch: their start-up and reduction tails overlap
// instead of following each other.
template <int CB, int R>
__global__ __launch_bounds__(64 * G1_NW) __attribute__((amdgpu_waves_per_eu(8, 8), amdgpu_num_sgpr(74))) void gemv1_multi_kernel(const G1Multi)
{
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    // The argument read in place through the kernel-argument segment pointer: indexing the
    // by-value parameter with a run-time group would make the compiler copy all of it to
    // scratch memory first.
    const G1Multi& mm = *(const G1Multi*)__builtin_amdgcn_kernarg_segment_ptr();
    int i = 0;
#pragma unroll
    for (int j = 1; j < G1_MAXSH; j++)
        if (j < mm.ngrp && (int)blockIdx.x >= mm.gbeg[j]) i = j;
    i = __builtin_amdgcn_readfirstlane(i);
    const G1Group& a = mm.grp[i];
    const G1Shard* sht = mm.sh + mm.sh0[i];
    const int g = blockIdx.x - mm.gbeg[i];
    switch (mm.K[i]) {
    case 1: g1_body<1, CB, false, R>(a, sht, g, lds); break;
    case 2: g1_body<2, CB, false, R>(a, sht, g, lds); break;
    case 3: g1_body<3, CB, false, R>(a, sht, g, lds); break;
    case 4: g1_body<4, CB, false, R>(a, sht, g, lds); break;
    case 5: g1_body<5, CB, false, R>(a, sht, g, lds); break;
    case 6: g1_body<6, CB, false, R>(a, sht, g, lds); break;
    case 7: g1_body<7, CB, false, R>(a, sht, g, lds); break;
    case 8: g1_body<8, CB, false, R>(a, sht, g, lds); break;
    }
}

// ---------------------------------------------------------------- finish kernel

// Segment S of group a (shards sht), if a launch split it over several workgroups: its slots
// (written by the launch just before, on the same stream) added in workgroup order -- the
// same order on every call: deterministic -- then the output Hadamard, * svh and the fp16
// store, by one wave.  A segment inside one workgroup's range was finished by that
// workgroup.  Up to 32 slots are loaded per batch, all before the first add, so a segment
// split over <= 32 workgroups costs one round trip to memory.
template <int R, bool ONE>
__device__ __forceinline__ void g1_finish_body(const G1Group& a, const G1Shard* sht, int S)
{
    auto sh = [&](int s) -> const G1Shard& { return sht[ONE ? 0 : s]; };
    if (S >= a.nsegs) return;
    const int s = g1_shard_of_seg<ONE>(a, sht, S);
    const int cg = S - sh(s).sbeg;
    const int segU0 = sh(s).ubeg + cg * a.ntr;
    const int g_lo = g1_wg_of(a, segU0), g_hi = g1_wg_of(a, segU0 + a.ntr - 1);
    if (g_hi == g_lo) return;
    const int lane = threadIdx.x;
    const int nsl = g_hi - g_lo + 1;
    const int nr = R == 1 ? 1 : a.nrows;
    const uint32_t sv = reinterpret_cast<const uint32_t*>(sh(s).svh + cg * 128)[lane];
    const uint64_t* sl = reinterpret_cast<const uint64_t*>(a.slots + (long)(S + g_lo) * R * 128) + lane;
    constexpr int B = 32;
    for (int r = 0; r < nr; r++) {
        float v0 = 0.f, v1 = 0.f;
        for (int t0 = 0; t0 < nsl; t0 += B) {
            uint64_t xv[B];
#pragma unroll
            for (int t = 0; t < B; t++) xv[t] = sl[((long)min(t0 + t, nsl - 1) * R + r) * 64];
#pragma unroll
            for (int t = 0; t < B; t++)
                if (t0 + t < nsl) {
                    v0 += __builtin_bit_cast(float, (uint32_t)xv[t]);
                    v1 += __builtin_bit_cast(float, (uint32_t)(xv[t] >> 32));
                }
        }
        wave_fwht128(v0, v1);
        v0 *= g1_lo(sv);
        v1 *= g1_hi(sv);
        reinterpret_cast<uint32_t*>(sh(s).C + r * sh(s).ldc + cg * 128)[lane] =
            (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v0) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v1) << 16);
    }
}

// A single-group launch's split segments (block = segment): every argument field is read at
// a constant offset, so its scalar loads issue together.
template <int R, bool ONE>
__global__ __launch_bounds__(64) void gemv1_finish_kernel(const G1Args a)
{
    g1_finish_body<R, ONE>(a.grp, a.sh, blockIdx.x);
}

// A multi-group launch's split segments: block b is segment b - fbeg[i] of group i.
template <int R>
__global__ __launch_bounds__(64) void gemv1_finish_multi_kernel(const G1Multi)
{
    const G1Multi& mm = *(const G1Multi*)__builtin_amdgcn_kernarg_segment_ptr();
    int i = 0;
#pragma unroll
    for (int j = 1; j < G1_MAXSH; j++)
        if (j < mm.ngrp && (int)blockIdx.x >= mm.fbeg[j]) i = j;
    i = __builtin_amdgcn_readfirstlane(i);
    g1_finish_body<R, false>(mm.grp[i], mm.sh + mm.sh0[i], blockIdx.x - mm.fbeg[i]);
}

// ---------------------------------------------------------------- host side

template <int K, int CB, int R>
static const void* g1_fn(bool one)
{
    return one ? reinterpret_cast<const void*>(&gemv1_kernel<K, CB, true, R>)
               : reinterpret_cast<const void*>(&gemv1_kernel<K, CB, false, R>);
}

template <int R>
static const void* g1_fn_kcb(int K, int cb, bool one)
{
#define EXL3_CASE(KK) case KK: return cb == CB_MCG ? g1_fn<KK, CB_MCG, R>(one) : g1_fn<KK, CB_3INST, R>(one);
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

// Dynamic LDS a launch needs: a partial row per wave for the most segments (shard, column
// group) a workgroup range of ceil(U / G) units can touch, a transformed activation block for
// each 128-input block it can meet (at most ceil(L / 8) + nseg + 1: a piece of a segment
// meets one block more than its length in blocks when it starts inside a block, and only the
// first piece can), and the 64-byte zero operand.
static size_t g1_lds_bytes(int U, int G, int ntr, int R)
{
    const int L = (U + G - 1) / G;
    const int nseg = (L - 1 + ntr - 1) / ntr + 1;
    const int nocc = (L + 7) / 8 + nseg + 1;
    return (size_t)nseg * G1_NW * R * 128 * sizeof(float) + (size_t)nocc * R * 128 * sizeof(uint32_t) + 64;
}

// Row-count template of a call: one activation row, or up to four (G1_ROWS).
constexpr int G1_ROWS = 4;
static int g1_R(int rows) { return rows == 1 ? 1 : G1_ROWS; }

// Per-shard share of the workspace after the counter area: slots of R rows for up to
// G1_GMAX workgroups and one per column group.
size_t gemv1_slot_bytes(int ic, int oc, int rows)
{
    (void)ic;
    return (size_t)(G1_GMAX + oc / 128) * g1_R(rows) * 128 * sizeof(float);
}

// Units per workgroup the launch aims for: fewer, longer ranges cut the cross-workgroup
// reduction (fewer contributors per column group) and the per-wave start-up, while a
// launch still spreads over up to G1_WG_PER_CU workgroups per CU.  Measured on MI355X
// over the 27B projection shapes: 32 is best or within 3% of best for each.
constexpr int G1_UNITS_PER_WG = 32;

// Fills one group from shards[idx[0..n-1]] (same K and codebook) into table entries
// tab[0..n-1]; returns its unit count.
static long g1_group(G1Group& grp, G1Shard* tab, const GemvShard* shards, const int* idx, int n, const uint16_t* A,
                     int ntr, int rows)
{
    grp = G1Group{};
    grp.x = A;
    grp.nrows = rows;
    grp.ntr = ntr;
    grp.nshards = n;
    long U = 0;
    int nsegs = 0;
    for (int j = 0; j < n; j++) {
        const GemvShard& d = shards[idx[j]];
        G1Shard& e = tab[j];
        e.trellis = d.trellis;
        e.suh = d.suh;
        e.svh = d.svh;
        e.C = d.C;
        e.ldc = d.ldc;
        e.ubeg = (int)U;
        e.sbeg = nsegs;
        e.oc16 = d.oc / 16;
        e.ncg = d.oc / 128;
        U += (long)(d.oc / 128) * ntr;
        nsegs += d.oc / 128;
    }
    grp.nsegs = nsegs;
    return U;
}

// Workgroup split of a group of U units into G ranges, and its share of the slots.
static int g1_place(G1Group& grp, long U, int G, int R, char* slots, size_t& sbase, size_t slot_bytes)
{
    if (U > (1L << 30))
        return set_error(EXL3_ERR_ARG, "exl3_gemv: %ld tile-row units in one launch (limit 2^30)", U);
    const size_t need = (size_t)(G + grp.nsegs) * R * 128 * sizeof(float);
    if (sbase + need > slot_bytes)
        return set_error(EXL3_ERR_WORKSPACE, "exl3_gemv: slot area of %zu bytes, %zu needed", slot_bytes,
                         sbase + need);
    grp.U = (int)U;
    grp.G = G;
    grp.q = (int)(U / G);
    grp.r = (int)(U % G);
    // divisors are >= 8 (ntr = ic / 16 with ic >= 128; G <= U / 8), as g1_div requires
    grp.dntr = g1_magic((uint32_t)grp.ntr);
    grp.dq = g1_magic((uint32_t)grp.q);
    grp.dq1 = g1_magic((uint32_t)grp.q + 1);
    grp.slots = reinterpret_cast<float*>(slots + sbase);
    sbase += need;
    return EXL3_OK;
}

// Whether some segment of the group lies in more than one workgroup range (then the
// launch needs gemv1_finish_kernel): segment S is units S ntr .. S ntr + ntr - 1.
static bool g1_any_split(const G1Group& grp)
{
    const long big = (long)grp.r * (grp.q + 1);
    auto wg_of = [&](long u) { return u < big ? u / (grp.q + 1) : grp.r + (u - big) / grp.q; };
    for (int S = 0; S < grp.nsegs; S++)
        if (wg_of((long)S * grp.ntr) != wg_of((long)S * grp.ntr + grp.ntr - 1)) return true;
    return false;
}

// The finish kernel of a single-group launch, if any of its segments is split.
static int g1_finish(G1Args& args, int R, bool one, hipStream_t stream)
{
    if (!g1_any_split(args.grp)) return EXL3_OK;
    const void* fn = R == 1 ? (one ? reinterpret_cast<const void*>(&gemv1_finish_kernel<1, true>)
                                   : reinterpret_cast<const void*>(&gemv1_finish_kernel<1, false>))
                            : (one ? reinterpret_cast<const void*>(&gemv1_finish_kernel<G1_ROWS, true>)
                                   : reinterpret_cast<const void*>(&gemv1_finish_kernel<G1_ROWS, false>));
    void* kargs[] = {&args};
    hipLaunchKernel(fn, dim3(args.grp.nsegs), dim3(64), kargs, 0, stream);
    return check_launch("exl3_gemv (1-4 rows, split segments)");
}

// The finish kernel of a multi-group launch (m.grp[0 .. m.ngrp - 1], m.sh, m.sh0 set), if any
// of its segments is split.
static int g1_finish(G1Multi& m, int R, hipStream_t stream)
{
    bool any = false;
    int nb = 0;
    for (int t = 0; t < m.ngrp; t++) {
        m.fbeg[t] = nb;
        nb += m.grp[t].nsegs;
        any = any || g1_any_split(m.grp[t]);
    }
    if (!any) return EXL3_OK;
    const void* fn = R == 1 ? reinterpret_cast<const void*>(&gemv1_finish_multi_kernel<1>)
                            : reinterpret_cast<const void*>(&gemv1_finish_multi_kernel<G1_ROWS>);
    void* kargs[] = {&m};
    hipLaunchKernel(fn, dim3(nb), dim3(64), kargs, 0, stream);
    return check_launch("exl3_gemv (1-4 rows, split segments)");
}

static int g1_launch(const void* fn, void* arg, int G, size_t lds, hipStream_t stream)
{
    if (lds > 64 * 1024) {
        hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        (void)hipGetLastError();
    }
    void* kargs[] = {arg};
    hipLaunchKernel(fn, dim3(G), dim3(64 * G1_NW), kargs, lds, stream);
    return check_launch("exl3_gemv (1-4 rows)");
}

// Workgroup counts G[0..ns) of one launch whose groups have U[t] units, for the most
// workgroups per CU (up to G1_WG_PER_CU) whose LDS lets them all stay resident; returns
// that number and the launch's LDS per workgroup.
static int g1_split(const long* U, int ns, int ntr, int R, int cus, int* G, size_t& lds)
{
    constexpr size_t LDS_PER_CU = 160 * 1024;
    int wgpc = G1_WG_PER_CU;
    for (; wgpc >= 1; wgpc--) {
        const int gmax = std::min(G1_GMAX, wgpc * cus);
        long Gsum = 0;
        for (int t = 0; t < ns; t++) {
            G[t] = (int)std::min<long>(gmax, std::max<long>(1, U[t] / G1_UNITS_PER_WG));
            Gsum += G[t];
        }
        if (Gsum > gmax)   // share the resident workgroups in proportion to the groups' sizes
            for (int t = 0; t < ns; t++) G[t] = std::max(1, (int)((long)G[t] * gmax / Gsum));
        lds = 0;
        for (int t = 0; t < ns; t++) lds = std::max(lds, g1_lds_bytes((int)U[t], G[t], ntr, R));
        if ((size_t)wgpc * lds <= LDS_PER_CU) break;
    }
    return std::max(wgpc, 1);
}

// Whether 2..4 rows of these shards run well here: every launch keeps at least three
// workgroups per CU resident (with four rows the LDS per workgroup grows with its range).
// The caller takes the split kernels otherwise.
bool gemv1_rows_fit(const GemvShard* shards, int nshards)
{
    const int ntr = shards[0].ic / 16;
    const int cus = g1_cu_count();
    // the launches group shards of one codebook; bound each launch by all of its shards
    for (int cb = 0; cb < 2; cb++) {
        long U[G1_MAXSH];
        int ns = 0, G[G1_MAXSH];
        for (int i = 0; i < nshards; i++) {
            if (shards[i].cb != cb) continue;
            const long u = (long)(shards[i].oc / 128) * ntr;
            if (ns < G1_MAXSH) U[ns++] = u;
            else U[G1_MAXSH - 1] += u;
        }
        if (!ns) continue;
        size_t lds;
        if (g1_split(U, ns, ntr, G1_ROWS, cus, G, lds) < 3) return false;
    }
    return true;
}

// 1..4 activation rows: the shards are grouped by (K, codebook), at most G1_MAXSH shards a
// group.  A launch takes whole groups of one codebook, at most G1_MAXSH shards in all: one
// group is a gemv1_kernel launch, several share a gemv1_multi_kernel launch with their
// workgroup counts scaled to the resident limit together.  Workgroups per CU: four, or
// fewer where a launch's LDS per workgroup (larger with four rows) would not let four
// stay resident.
int gemv1_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* slots,
                   size_t slot_bytes, hipStream_t stream)
{
    if (rows < 1 || rows > G1_ROWS) return set_error(EXL3_ERR_ARG, "exl3_gemv: rows=%d is not in 1..%d", rows, G1_ROWS);
    const int R = g1_R(rows);
    const int ic = shards[0].ic;
    const int ntr = ic / 16;
    const int cus = g1_cu_count();

    // groups: shard indices by (codebook, K) in first-seen order, split every G1_MAXSH shards
    constexpr int MAXG = EXL3_MAX_SHARDS;
    int gidx[MAXG][G1_MAXSH], gn[MAXG] = {0}, gK[MAXG], gcb[MAXG], ng = 0;
    for (int i = 0; i < nshards; i++) {
        if (shards[i].K < 1 || shards[i].K > 8)
            return set_error(EXL3_ERR_ARG, "exl3_gemv: K=%d is not in 1..8", shards[i].K);
        int j = ng - 1;
        while (j >= 0 && !(gK[j] == shards[i].K && gcb[j] == shards[i].cb && gn[j] < G1_MAXSH)) j--;
        if (j < 0) {
            j = ng++;
            gK[j] = shards[i].K;
            gcb[j] = shards[i].cb;
        }
        gidx[j][gn[j]++] = i;
    }

    size_t sbase = 0;
    bool done[MAXG] = {false};
    for (int j0 = 0; j0 < ng; j0++) {
        if (done[j0]) continue;
        // this launch: group j0 and the following groups of its codebook while they fit
        int sel[G1_MAXSH], ns = 0, nsh = 0;
        for (int j = j0; j < ng; j++)
            if (!done[j] && gcb[j] == gcb[j0] && nsh + gn[j] <= G1_MAXSH) {
                sel[ns++] = j;
                nsh += gn[j];
                done[j] = true;
            }
        const int cb = gcb[j0];
        G1Multi m = {};
        long U[G1_MAXSH];
        int G[G1_MAXSH], sh0 = 0;
        for (int t = 0; t < ns; t++) {
            const int j = sel[t];
            m.sh0[t] = sh0;
            m.K[t] = gK[j];
            U[t] = g1_group(m.grp[t], m.sh + sh0, shards, gidx[j], gn[j], A, ntr, rows);
            sh0 += gn[j];
        }
        size_t lds = 0;
        g1_split(U, ns, ntr, R, cus, G, lds);
        if (ns == 1) {
            G1Args args = {};
            args.grp = m.grp[0];
            for (int i = 0; i < gn[sel[0]]; i++) args.sh[i] = m.sh[i];
            int rc = g1_place(args.grp, U[0], G[0], R, slots, sbase, slot_bytes);
            if (rc != EXL3_OK) return rc;
            const bool one = gn[sel[0]] == 1;
            const void* fn = R == 1 ? g1_fn_kcb<1>(gK[sel[0]], cb, one) : g1_fn_kcb<G1_ROWS>(gK[sel[0]], cb, one);
            rc = g1_launch(fn, &args, G[0], lds, stream);
            if (rc != EXL3_OK) return rc;
            rc = g1_finish(args, R, one, stream);
            if (rc != EXL3_OK) return rc;
            continue;
        }
        int gb = 0;
        for (int t = 0; t < ns; t++) {
            const int rc = g1_place(m.grp[t], U[t], G[t], R, slots, sbase, slot_bytes);
            if (rc != EXL3_OK) return rc;
            m.gbeg[t] = gb;
            gb += G[t];
        }
        m.ngrp = ns;
        const void* fn = R == 1 ? (cb == CB_MCG ? reinterpret_cast<const void*>(&gemv1_multi_kernel<CB_MCG, 1>)
                                               : reinterpret_cast<const void*>(&gemv1_multi_kernel<CB_3INST, 1>))
                                : (cb == CB_MCG ? reinterpret_cast<const void*>(&gemv1_multi_kernel<CB_MCG, G1_ROWS>)
                                               : reinterpret_cast<const void*>(&gemv1_multi_kernel<CB_3INST, G1_ROWS>));
        int rc = g1_launch(fn, &m, gb, lds, stream);
        if (rc != EXL3_OK) return rc;
        rc = g1_finish(m, R, stream);
        if (rc != EXL3_OK) return rc;
    }
    return EXL3_OK;
}

}  // namespace exl3
