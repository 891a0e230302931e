// Fused EXL3 decode-GEMV for one to four activation rows (batch-1..4 decode):
//   y_r (oc) = fp16( H( fp16(H(x_r * suh)) . W_q ) * svh ),  r < nrows
// with W_q decoded from the packed trellis in registers and never stored.  Replaces
// exllamav3_ext.exl3_gemm as called at orcasaq2/ops.py:46-49 for rows <= 4 (rows 2..4
// wherever this plan takes the shards; gemv16.hip takes the rest and 5..16 rows).
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
//      iteration (D = g1_depth: one unit in flight per wave, eight waves per SIMD; two for
//      the four-row template when the launch's LDS leaves fewer workgroups resident).
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
//      * svh, fp16 store).  A segment split over several workgroups is finished in the
//      same launch without any wait: each workgroup puts its partials through the output
//      Hadamard and * svh (both linear) and adds them, in fixed point, into the segment's
//      accumulator words in the workspace with one 64-bit atomic add per output, whose top
//      bits count the contributions; the add that completes a word's count returns the sum
//      of all the others, so that lane stores the finished output and clears the word
//      (g1_acc_add).  One memory round trip, exact integer sums (the same bits whatever
//      order the workgroups arrive in), no second launch: on MI355X a down_proj call went
//      from 20.1 to 18.7 us and the 64-layer stack from 5.14 to 4.52 ms per token against
//      the former finish kernel (which is kept for calls whose accumulators would not fit
//      the workspace's area: its slots are added in workgroup order after the launch).
#include "exl3_common.h"
#include "gemv1_plan.h"

namespace exl3 {

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

// A transformed partial output as an accumulator increment: one contribution in the count
// bits plus the value in fixed point, rounded to nearest (the format is gemv1_plan.h's).
__device__ __forceinline__ unsigned long long g1_fx(float v)
{
    v = fminf(fmaxf(v, -G1_FX_MAX), G1_FX_MAX);
    const long long f = (long long)__builtin_rint((double)v * (double)(1 << G1_FX_FRAC));
    return (1ull << G1_FX_CBIT) + (unsigned long long)f;
}

// Split segment S, activation row r, n contributing workgroups, accumulators in a.acc, sv the
// lane's svh pair of the column group: this
// workgroup's partial outputs (v0, v1: outputs 2 lane, 2 lane + 1 of the column group) go
// through the output Hadamard and * svh here -- both linear, so the transformed partials of
// the n workgroups add up to the finished outputs -- and are added into the segment's words.
// The add that brings a word's count to n returns the sum of the other n - 1, so its lane
// holds the finished output: it stores it as fp16 and clears the word for the next call.
// Integer adds are exact and commute: the result is the same whatever order the workgroups
// arrive in.  Relaxed agent-scope atomics suffice: every word is read and written only by
// these adds and the final clear, and the kernel boundary orders the clear before the next
// call's adds.
template <bool ONE>
__device__ __forceinline__ void g1_acc_add(const G1Group& a, const G1Shard* sht, int S, int R, int r, int n,
                                           float v0, float v1, int lane, uint32_t sv)
{
    const int s = g1_shard_of_seg<ONE>(a, sht, S);
    const G1Shard& e = g1_sh<ONE>(sht, s);
    const int cg = S - e.sbeg;
    wave_fwht128(v0, v1);
    const unsigned long long m0 = g1_fx(v0 * g1_lo(sv)), m1 = g1_fx(v1 * g1_hi(sv));
    unsigned long long* p = a.acc + g1_acc_word(S, R, r, lane, 0);
    const unsigned long long o0 = __hip_atomic_fetch_add(p, m0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long o1 = __hip_atomic_fetch_add(p + 1, m1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // count of an old word: its value part lies in [-2^51, 2^51)
    constexpr unsigned long long half = 1ull << (G1_FX_CBIT - 1);
    const unsigned long long last = (unsigned long long)(n - 1);
    const bool f0 = ((o0 + half) >> G1_FX_CBIT) == last, f1 = ((o1 + half) >> G1_FX_CBIT) == last;
    if (!f0 && !f1) return;
    const unsigned long long all = (unsigned long long)n << G1_FX_CBIT;
    constexpr double unit = 1.0 / (double)(1 << G1_FX_FRAC);
    const uint16_t h0 = __builtin_bit_cast(uint16_t, (_Float16)(float)((double)(long long)(o0 + m0 - all) * unit));
    const uint16_t h1 = __builtin_bit_cast(uint16_t, (_Float16)(float)((double)(long long)(o1 + m1 - all) * unit));
    uint16_t* c = e.C + r * e.ldc + cg * 128 + 2 * lane;
    if (f0 && f1) {
        *reinterpret_cast<uint32_t*>(c) = (uint32_t)h0 | ((uint32_t)h1 << 16);
    } else if (f0) {
        c[0] = h0;
    } else {
        c[1] = h1;
    }
    if (f0) __hip_atomic_store(p, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (f1) __hip_atomic_store(p + 1, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t g1_dup(float v)
{
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)v);
    return h | (h << 16);
}

// ---------------------------------------------------------------- decode kernel

// Workgroup g of group a (shard table sht) -- the whole kernel body.  The range, cursor,
// occurrence, LDS and global index arithmetic is gemv1_plan.h's (shared with the CPU address
// replay).
template <int K, int CB, bool ONE, int R, int D>
__device__ __forceinline__ void g1_body(const G1Group& a, const G1Shard* sht, const int g, uint32_t* lds)
{
    auto sh = [&](int s) -> const G1Shard& { return g1_sh<ONE>(sht, s); };

    const G1Range w = g1_range<ONE>(a, sht, g);
    const int nr = R == 1 ? 1 : a.nrows;     // activation rows in the tables and results
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    __builtin_amdgcn_s_setprio(3);

    // ---- this wave's units: the contiguous run w.ub + lo .. w.ub + lo + n - 1 of the range
    const G1Run run = g1_wave_run(w.L, wave);
    const int n = run.n;
    const uint32_t lk = g1_lane_word(lane, K);
    const bool first_lane = (lane & 7) == 0;

    // A unit's loads: the lane's K words.  Prefetch cursor (D units ahead; it stops at the
    // wave's last unit, whose data is then loaded again and not used) and processing cursor.
    struct Slot {
        uint32_t w[K + 1];
    };
    auto load = [&](Slot& sl, const G1Cursor& q) { g1_load<K>(sl.w, q.p, lk); };
    G1Cursor pf = g1_cursor_at<K, ONE>(a, sht, w.ub + run.lo), cu = pf;
    int jpf = 0;
    auto next_pf = [&]() -> const G1Cursor& {
        g1_next_pf<K, ONE>(a, sht, pf, jpf, n);
        return pf;
    };
    Slot ring[D];

    const G1Lds ll = g1_lds_layout(w.nseg, w.nocc, nr);
    float* red = reinterpret_cast<float*>(lds);
    uint32_t* act = lds + ll.act;
    uint32_t* zero = lds + ll.zero;
    if (threadIdx.x < g1_zero_words(nr)) zero[threadIdx.x] = 0u;
    const Dot2Consts kc = dot2_consts();

    // Activations, once per workgroup: the waves share out the (occurrence, activation row)
    // pairs; each transforms one block of one row, fp16(H128(x_r * suh)) (lane l: outputs 2l,
    // 2l + 1 = rows 2(l % 8), 2(l % 8) + 1 of the block's tile row l / 8) and stores each
    // output as a duplicated fp16 pair in the order the MFMAs read them (g1_act_word).  A wave
    // issues the loads of up to G1_TBATCH of its pairs before transforming any of them.  The
    // task cursor steps without dividing, and the shard's suh pointer is read again only when
    // the shard changes: the scalar unit is shared by every wave of the CU, and all of them
    // run this loop at once.
    const int ntask = w.nocc * nr;
    const FwhtSigns fs = fwht_signs(lane);
    const G1TaskStep tst = g1_task_step(nr);
    G1Task tk = g1_task_first<ONE>(a, sht, w, wave, nr);
    int s_suh = tk.s;
    const uint16_t* suh = sh(s_suh).suh;
    // The first unit's loads go out right behind the wave's first batch of activation loads:
    // ahead of them they would make the activation loads wait behind a launch-wide burst of
    // trellis loads (0.1-0.2 us per call slower), and after the whole table they leave the
    // trellis latency exposed once per launch.  Measured on MI355X at settled clocks against
    // issuing them after the table: config 1 aggregate 2357-2359 -> 2411-2434 GB/s, the
    // 64-layer stack 4.53 -> 4.42-4.44 ms per token.
    bool first_out = false;
    while (tk.t < ntask) {
        uint32_t sw[G1_TBATCH], xw[G1_TBATCH];
        G1Task tb[G1_TBATCH];
#pragma unroll
        for (int j = 0; j < G1_TBATCH; j++) {
            tb[j] = tk;
            if (tk.t < ntask) {
                if (tk.s != s_suh) {
                    s_suh = tk.s;
                    suh = sh(s_suh).suh;
                }
                sw[j] = reinterpret_cast<const uint32_t*>(suh + tk.blk * 128)[lane];
                xw[j] = reinterpret_cast<const uint32_t*>(a.x + g1_x_elem(a, tk.r, tk.blk))[lane];
                g1_task_next<ONE>(a, sht, w, tk, nr, tst);
            }
        }
        if (!first_out) {
            first_out = true;
            if (n > 0) load(ring[0], pf);
        }
#pragma unroll
        for (int j = 0; j < G1_TBATCH; j++) {
            if (tb[j].t < ntask) {
                float v0 = g1_lo(xw[j]) * g1_lo(sw[j]), v1 = g1_hi(xw[j]) * g1_hi(sw[j]);
                wave_fwht128(v0, v1, fs);
                *reinterpret_cast<uint2*>(act + g1_act_word(tb[j].i, lane, nr, tb[j].r)) = uint2{g1_dup(v0), g1_dup(v1)};
            }
        }
    }
    // (a wave without table tasks issues its first unit's loads here; deeper rings the rest)
    if (n > 0) {
        if (!first_out) load(ring[0], pf);
#pragma unroll
        for (int d = 1; d < D; d++) load(ring[d], next_pf());
    }
    // The svh pair of this wave's first epilogue task (segment, row) = task `wave`, loaded now
    // so that its latency is not at the end of the launch.
    auto svh_of = [&](int t) -> uint32_t {
        const int S = w.S_first + (R == 1 ? t : t / nr);
        const G1Shard& e = sh(g1_shard_of_seg<ONE>(a, sht, S));
        return reinterpret_cast<const uint32_t*>(e.svh + (S - e.sbeg) * 128)[lane];
    };
    const uint32_t sv_first = wave < w.nseg * nr ? svh_of(wave) : 0u;
    __syncthreads();

    // ---- main loop.  Scalar bookkeeping (cursor steps, column-group crossings, flushes of a
    // finished segment's sums to the wave's LDS row) sits between units, so each unit's work
    // is one basic block the scheduler can interleave; the loads sit outside every branch,
    // so the wait before a unit covers only that unit's own loads.  The occurrence index
    // steps whenever a unit starts a block (its tile row a multiple of 8, which includes
    // every segment start).
    // yacc[h][e] of lane 16r + n: activation row r's sum for output 32e + 16(n / 8) + n % 8 + 8h
    // (lanes 16r + n with r >= nr hold copies of row nr - 1).
    f32x4 yacc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    const int yrow = g1_yrow(lane), ycol = g1_ycol(lane);
    const uint32_t asel = g1_asel(lane);
    const uint32_t aoff = g1_aoff(lane, nr, ll);
    constexpr int CH = g1_a_chunk(R == 1 ? 1 : G1_ROWS) / 16;   // f16x8 steps between A chunks
    int cur = cu.S - w.S_first;
    int occ = g1_occ_of(w, cur, cu.tr);
    const int pq1 = (n + 3) >> 2, pq2 = (n + 1) >> 1, pq3 = (3 * n + 3) >> 2;
    auto flush = [&](int k) {
        if (yrow < nr) {
            float* rr = red + g1_red_row(cur, wave, nr, yrow) + ycol;
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
                if (cu.S - w.S_first != cur) flush(cu.S - w.S_first);
                const uint32_t e = g1_a_entry(occ, cu.tr, nr);
                const f16x8* ap = reinterpret_cast<const f16x8*>(reinterpret_cast<const char*>(lds) + (__umul24(e, asel) + aoff));
                const f16x8 av[4] = {ap[0], ap[CH], ap[2 * CH], ap[3 * CH]};
                chunk_prev_dpp<K>(ring[d].w, first_lane);
                g1_mfma_chunk<K, CB>(ring[d].w, av, yacc, kc);
                if (j + d + 1 < n) {
                    g1_advance<K, ONE>(a, sht, cu);
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
    auto finish = [&](int k, int r, float v0, float v1, uint32_t sv) {
        const int S = w.S_first + k;
        const int s = g1_shard_of_seg<ONE>(a, sht, S);
        const int cg = S - sh(s).sbeg;
        wave_fwht128(v0, v1);
        v0 *= g1_lo(sv);
        v1 *= g1_hi(sv);
        const uint32_t out = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v0) |
                             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v1) << 16);
        reinterpret_cast<uint32_t*>(sh(s).C + r * sh(s).ldc + cg * 128)[lane] = out;
    };
    // (segment, activation row) tasks shared out over the waves
    for (int t = wave; t < w.nseg * nr; t += G1_NW) {
        const int k = R == 1 ? t : t / nr, r = t - k * nr;
        // the partial rows of the waves whose runs meet segment k, in wave order
        int ub, ue;
        g1_seg_units(w, a.ntr, k, ub, ue);
        float v0 = 0.f, v1 = 0.f;
#pragma unroll
        for (int ww = 0; ww < G1_NW; ww++) {
            if (!g1_run_meets(g1_wave_run(w.L, ww), ub, ue)) continue;
            const float2 p = *reinterpret_cast<const float2*>(red + g1_red_row(k, ww, nr, r) + 2 * lane);
            v0 += p.x;
            v1 += p.y;
        }
        const uint32_t sv = t == wave ? sv_first : svh_of(t);
        int g_lo, g_hi;
        g1_contributors<ONE>(a, sht, w.S_first + k, g_lo, g_hi);
        if (g_hi > g_lo && a.acc) {
            g1_acc_add<ONE>(a, sht, w.S_first + k, R, r, g_hi - g_lo + 1, v0, v1, lane, sv);
        } else if (g_hi > g_lo) {
            // split segment without accumulators: row r of slot (S, g) holds this workgroup's 128
            // partials, which gemv1_finish_kernel adds after the launch
            uint64_t* my = reinterpret_cast<uint64_t*>(a.slots + g1_slot(w.S_first + k, g, R)) + lane;
            my[g1_slot_word(0, R, r)] = (uint64_t)__builtin_bit_cast(uint32_t, v0) |
                                        ((uint64_t)__builtin_bit_cast(uint32_t, v1) << 32);
        } else {
            finish(k, r, v0, v1, sv);
        }
    }
}

// Eight waves per SIMD need at most 64 VGPRs (measured on MI355X: 68 VGPRs leave room for
// only 6); the SGPR cap keeps the count well inside what eight waves per SIMD may hold.
template <int K, int CB, bool ONE, int R>
__global__ __launch_bounds__(64 * G1_NW) __attribute__((amdgpu_waves_per_eu(8, 8), amdgpu_num_sgpr(74))) void gemv1_kernel(const G1Args a)
{
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    g1_body<K, CB, ONE, R, 1>(a.grp, a.sh, blockIdx.x, lds);
}

// The four-row template with G1_DEEP units in flight per wave (g1_depth).
template <int K, int CB, bool ONE>
__global__ __launch_bounds__(64 * G1_NW) __attribute__((amdgpu_waves_per_eu(8, 8), amdgpu_num_sgpr(74))) void gemv1_deep_kernel(const G1Args a)
{
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    g1_body<K, CB, ONE, G1_ROWS, G1_DEEP>(a.grp, a.sh, blockIdx.x, lds);
}

// Several groups (different K) in one launch: their start-up and reduction tails overlap
// instead of following each other.
template <int CB, int R, int D = 1>
__global__ __launch_bounds__(64 * G1_NW) __attribute__((amdgpu_waves_per_eu(8, 8), amdgpu_num_sgpr(74))) void gemv1_multi_kernel(const G1Multi)
{
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    // The argument read in place through the kernel-argument segment pointer: indexing the
    // by-value parameter with a run-time group would make the compiler copy all of it to
    // scratch memory first.
    const G1Multi& mm = *(const G1Multi*)__builtin_amdgcn_kernarg_segment_ptr();
    const int i = __builtin_amdgcn_readfirstlane(g1_group_of(mm.gbeg, mm.ngrp, (int)blockIdx.x));
    const G1Group& a = mm.grp[i];
    const G1Shard* sht = mm.sh + mm.sh0[i];
    const int g = blockIdx.x - mm.gbeg[i];
    switch (mm.K[i]) {
    case 1: g1_body<1, CB, false, R, D>(a, sht, g, lds); break;
    case 2: g1_body<2, CB, false, R, D>(a, sht, g, lds); break;
    case 3: g1_body<3, CB, false, R, D>(a, sht, g, lds); break;
    case 4: g1_body<4, CB, false, R, D>(a, sht, g, lds); break;
    case 5: g1_body<5, CB, false, R, D>(a, sht, g, lds); break;
    case 6: g1_body<6, CB, false, R, D>(a, sht, g, lds); break;
    case 7: g1_body<7, CB, false, R, D>(a, sht, g, lds); break;
    case 8: g1_body<8, CB, false, R, D>(a, sht, g, lds); break;
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
    auto sh = [&](int s) -> const G1Shard& { return g1_sh<ONE>(sht, s); };
    if (S >= a.nsegs || a.acc) return;   // a group with accumulators finished in its launch
    const int s = g1_shard_of_seg<ONE>(a, sht, S);
    const int cg = S - sh(s).sbeg;
    int g_lo, g_hi;
    g1_contributors<ONE>(a, sht, S, g_lo, g_hi);
    if (g_hi == g_lo) return;
    const int lane = threadIdx.x & 63;
    const int nsl = g_hi - g_lo + 1;
    const int nr = R == 1 ? 1 : a.nrows;
    const uint32_t sv = reinterpret_cast<const uint32_t*>(sh(s).svh + cg * 128)[lane];
    const uint64_t* sl = reinterpret_cast<const uint64_t*>(a.slots + g1_slot(S, g_lo, R)) + lane;
    constexpr int B = 32;
    // wave r of the block finishes activation row r
    for (int r = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); r < nr; r += R) {
        float v0 = 0.f, v1 = 0.f;
        for (int t0 = 0; t0 < nsl; t0 += B) {
            uint64_t xv[B];
#pragma unroll
            for (int t = 0; t < B; t++) xv[t] = sl[g1_slot_word(min(t0 + t, nsl - 1), R, r)];
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
__global__ __launch_bounds__(64 * R) void gemv1_finish_kernel(const G1Args a)
{
    g1_finish_body<R, ONE>(a.grp, a.sh, blockIdx.x);
}

// A multi-group launch's split segments: block b is segment b - fbeg[i] of group i.
template <int R>
__global__ __launch_bounds__(64 * R) void gemv1_finish_multi_kernel(const G1Multi)
{
    const G1Multi& mm = *(const G1Multi*)__builtin_amdgcn_kernarg_segment_ptr();
    const int i = __builtin_amdgcn_readfirstlane(g1_group_of(mm.fbeg, mm.ngrp, (int)blockIdx.x));
    g1_finish_body<R, false>(mm.grp[i], mm.sh + mm.sh0[i], blockIdx.x - mm.fbeg[i]);
}

// ---------------------------------------------------------------- host side

template <int K, int CB, int R, int D>
static const void* g1_fn(bool one)
{
    if constexpr (D > 1) {
        static_assert(R == G1_ROWS, "deep prefetch is instantiated for the four-row template only");
        return one ? reinterpret_cast<const void*>(&gemv1_deep_kernel<K, CB, true>)
                   : reinterpret_cast<const void*>(&gemv1_deep_kernel<K, CB, false>);
    } else {
        return one ? reinterpret_cast<const void*>(&gemv1_kernel<K, CB, true, R>)
                   : reinterpret_cast<const void*>(&gemv1_kernel<K, CB, false, R>);
    }
}

template <int R, int D = 1>
static const void* g1_fn_kcb(int K, int cb, bool one)
{
#define EXL3_CASE(KK) case KK: return cb == CB_MCG ? g1_fn<KK, CB_MCG, R, D>(one) : g1_fn<KK, CB_3INST, R, D>(one);
    switch (K) {
        EXL3_CASE(1) EXL3_CASE(2) EXL3_CASE(3) EXL3_CASE(4)
        EXL3_CASE(5) EXL3_CASE(6) EXL3_CASE(7) EXL3_CASE(8)
    }
#undef EXL3_CASE
    return nullptr;
}

size_t gemv1_slot_bytes(int ic, int oc, int rows)
{
    (void)ic;
    return g1_slot_bytes(oc, rows);
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

// Whether g1_plan takes these shards at this row count: the plan run without launching
// anything.  It refuses a launch whose workgroup ranges' activation tables would exceed a
// CU's LDS even at G1_GMAX workgroups (with four rows, some 2.6e9 weights in one launch);
// the refusal's message is dropped, since the caller then takes gemv16 instead.
bool gemv1_plan_fits(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* slots,
                     size_t slot_bytes)
{
    const int rc = g1_plan(A, shards, nshards, rows, slots, slot_bytes, nullptr, 0, device_cus(),
                           [](const G1Launch&) { return EXL3_OK; });
    if (rc != EXL3_OK) clear_error();
    return rc == EXL3_OK;
}

// The launches of g1_plan: the decode kernel, then (if some segment is split) the finish
// kernel, one block per segment.
int gemv1_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* slots,
                   size_t slot_bytes, char* acc, size_t acc_bytes, hipStream_t stream)
{
    return g1_plan(A, shards, nshards, rows, slots, slot_bytes, acc, acc_bytes, device_cus(), [&](const G1Launch& L) {
        const char* what = "exl3_gemv (1-4 rows, split segments)";
        if (!L.multi) {
            G1Args args = *L.args;
            const bool deep = g1_depth(L.R, L.lds) > 1;
            const void* fn = L.R == 1 ? g1_fn_kcb<1>(L.K, L.cb, L.one)
                           : deep     ? g1_fn_kcb<G1_ROWS, G1_DEEP>(L.K, L.cb, L.one)
                                      : g1_fn_kcb<G1_ROWS>(L.K, L.cb, L.one);
            int rc = g1_launch(fn, &args, L.G, L.lds, stream);
            if (rc != EXL3_OK || !L.finish) return rc;
            const void* ff = L.R == 1 ? (L.one ? reinterpret_cast<const void*>(&gemv1_finish_kernel<1, true>)
                                               : reinterpret_cast<const void*>(&gemv1_finish_kernel<1, false>))
                                      : (L.one ? reinterpret_cast<const void*>(&gemv1_finish_kernel<G1_ROWS, true>)
                                               : reinterpret_cast<const void*>(&gemv1_finish_kernel<G1_ROWS, false>));
            void* kargs[] = {&args};
            hipLaunchKernel(ff, dim3(L.fblocks), dim3(64 * L.R), kargs, 0, stream);
            return check_launch(what);
        }
        G1Multi m = *L.m;
        const bool deep = g1_depth(L.R, L.lds) > 1;
        const void* fn = L.R == 1 ? (L.cb == CB_MCG ? reinterpret_cast<const void*>(&gemv1_multi_kernel<CB_MCG, 1>)
                                                    : reinterpret_cast<const void*>(&gemv1_multi_kernel<CB_3INST, 1>))
                       : deep     ? (L.cb == CB_MCG ? reinterpret_cast<const void*>(&gemv1_multi_kernel<CB_MCG, G1_ROWS, G1_DEEP>)
                                                    : reinterpret_cast<const void*>(&gemv1_multi_kernel<CB_3INST, G1_ROWS, G1_DEEP>))
                                  : (L.cb == CB_MCG ? reinterpret_cast<const void*>(&gemv1_multi_kernel<CB_MCG, G1_ROWS>)
                                                    : reinterpret_cast<const void*>(&gemv1_multi_kernel<CB_3INST, G1_ROWS>));
        int rc = g1_launch(fn, &m, L.G, L.lds, stream);
        if (rc != EXL3_OK || !L.finish) return rc;
        const void* ff = L.R == 1 ? reinterpret_cast<const void*>(&gemv1_finish_multi_kernel<1>)
                                  : reinterpret_cast<const void*>(&gemv1_finish_multi_kernel<G1_ROWS>);
        void* kargs[] = {&m};
        hipLaunchKernel(ff, dim3(L.fblocks), dim3(64 * L.R), kargs, 0, stream);
        return check_launch(what);
    });
}

}  // namespace exl3
