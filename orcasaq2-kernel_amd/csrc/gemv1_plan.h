// Work plan of the 1..4-row decode GEMV (gemv1.hip): the launch argument blocks, the split of
// a launch's units into workgroup ranges and wave runs, the cursor over a run's units, the
// activation-table occurrences, the LDS layout, every global and LDS index the kernels form,
// and the host-side grouping of shards into launches.
//
// Everything here is plain integer arithmetic marked __host__ __device__: the kernels call
// these functions, and the CPU address replay (replay/addr_replay.hip) calls the very same
// ones to walk every workgroup, wave and lane of a launch and check each index against the
// buffer it addresses.
#pragma once

#include <algorithm>

#include "exl3_launch.h"

namespace exl3 {

#define G1_HD __host__ __device__ __forceinline__

constexpr int G1_NW = 8;                 // waves per workgroup
constexpr int G1_MAXSH = 8;              // shards per launch
constexpr int G1_WG_PER_CU = 4;          // target resident workgroups per CU (8 waves / SIMD)
constexpr int G1_GMAX = 2048;            // workgroups per launch (bounds the slot area)
constexpr int G1_ROWS = 4;               // activation rows of the multi-row template
constexpr int G1_TBATCH = 2;             // activation-table pairs a wave loads before transforming

// Units a wave keeps in flight: one.  Eight waves per SIMD already keep enough loads in
// flight, and every unit more per wave lengthens the memory queues that a launch's first
// units and activation loads wait behind: measured on MI355X (down_proj, per call), depth 1
// against 2 and against 24 / (K + 3) clamped to 2..6: K = 2 18.6 / 18.7 / 19.6 us, K = 3
// 18.9 / 19.6 / 20.9, K = 4 19.4 / 19.8 / 20.7, K = 5 19.4 / 20.4 / 21.4.  Two for the
// four-row template where a launch's LDS per workgroup leaves fewer than G1_WG_PER_CU
// workgroups resident (g1_depth, after the LDS constants): fewer waves per SIMD, so each
// keeps more bytes in flight.
constexpr int G1_DEEP = 2;

// Units per workgroup the launch aims for: fewer, longer ranges cut the cross-workgroup
// reduction (fewer contributors per column group) and the per-wave start-up, while a
// launch still spreads over up to G1_WG_PER_CU workgroups per CU.  Measured on MI355X
// over the 27B projection shapes: 32 is best or within 3% of best for each.
constexpr int G1_UNITS_PER_WG = 32;

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

G1_HD int g1_div(int x, G1Div d)
{
    return (int)((uint32_t)(((uint64_t)(uint32_t)x * d.m) >> 32) >> d.sh);
}

// One group of shards with the same K and codebook, decoded by G workgroups.
struct G1Group {
    const uint16_t* x;         // (nrows, ic) fp16
    int nrows;                 // activation rows, 1 .. R of the kernel
    float* slots;              // (G + segments) x R x 128 fp32 partials of split segments (acc null)
    unsigned long long* acc;   // segments x R x 128 accumulator words of split segments, or null
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

// Group of a multi-group launch that owns block b, given the first block of each group
// (gbeg for the decode kernel, fbeg for the finish kernel).
G1_HD int g1_group_of(const int (&beg)[G1_MAXSH], int ngrp, int b)
{
    int i = 0;
#pragma unroll
    for (int j = 1; j < G1_MAXSH; j++)
        if (j < ngrp && b >= beg[j]) i = j;
    return i;
}

// First unit of workgroup g: the first r workgroups own q + 1 units, the others q.
G1_HD int g1_first_unit(const G1Group& a, int g)
{
    return g * a.q + (g < a.r ? g : a.r);
}

// Units of workgroup g.
G1_HD int g1_units(const G1Group& a, int g)
{
    return a.q + (g < a.r ? 1 : 0);
}

// Workgroup whose unit range holds unit u.
G1_HD int g1_wg_of(const G1Group& a, int u)
{
    const int big = a.r * (a.q + 1);
    return u < big ? g1_div(u, a.dq1) : a.r + g1_div(u - big, a.dq);
}

// Shard holding segment S / unit u.  Every table entry is read at a constant offset, so the
// scalar loads of the whole table issue together instead of as a chain of dependent loads
// (each a few hundred cycles); a single-shard launch (ONE) reads nothing.
template <bool ONE>
G1_HD int g1_shard_of_seg(const G1Group& a, const G1Shard* sht, int S)
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
G1_HD int g1_shard_of_unit(const G1Group& a, const G1Shard* sht, int u)
{
    int s = 0;
    if constexpr (!ONE) {
#pragma unroll
        for (int i = 1; i < G1_MAXSH; i++)
            if (i < a.nshards && u >= sht[i].ubeg) s = i;
    }
    return s;
}

// Shard table entry s; a single-shard group (ONE) only ever reads entry 0.
template <bool ONE>
G1_HD const G1Shard& g1_sh(const G1Shard* sht, int s)
{
    return sht[ONE ? 0 : s];
}

// ---------------------------------------------------------------- a wave's run and its cursor

// The wave's units: the contiguous run lo .. lo + n - 1 of its workgroup's L units.
struct G1Run {
    int lo, n;
};

G1_HD G1Run g1_wave_run(int L, int wave)
{
    const int lo = (wave * L) >> 3;
    return G1Run{lo, (((wave + 1) * L) >> 3) - lo};
}

// Wave-uniform cursor over a run's units: shard, column group, tile row, segment and the
// first word of the unit's 8 tiles.  Consecutive units are consecutive tile rows (ntr >= 8);
// only a column-group crossing reads the shard table again.
struct G1Cursor {
    int s, cg, tr, S;
    long stride;               // words between consecutive tile rows
    const uint32_t* p;
};

template <int K, bool ONE>
G1_HD void g1_seat(const G1Shard* sht, G1Cursor& q)
{
    const G1Shard& e = g1_sh<ONE>(sht, q.s);
    q.stride = (long)e.oc16 * (8 * K);
    q.p = e.trellis + ((long)q.tr * e.oc16 + 8 * q.cg) * (8 * K);
}

template <int K, bool ONE>
G1_HD G1Cursor g1_cursor_at(const G1Group& a, const G1Shard* sht, int u)
{
    G1Cursor q;
    q.s = g1_shard_of_unit<ONE>(a, sht, u);
    const int rel = u - g1_sh<ONE>(sht, q.s).ubeg;
    q.cg = g1_div(rel, a.dntr);
    q.tr = rel - q.cg * a.ntr;
    q.S = g1_sh<ONE>(sht, q.s).sbeg + q.cg;
    g1_seat<K, ONE>(sht, q);
    return q;
}

template <int K, bool ONE>
G1_HD void g1_advance(const G1Group& a, const G1Shard* sht, G1Cursor& q)
{
    q.tr++;
    q.p += q.stride;
    if (q.tr == a.ntr) {
        q.tr = 0;
        q.S++;
        if (++q.cg == g1_sh<ONE>(sht, q.s).ncg) {
            q.s++;
            q.cg = 0;
        }
        g1_seat<K, ONE>(sht, q);
    }
}

// The prefetch cursor steps with its unit count j until the run's last unit (whose data is
// then loaded again and not used).
template <int K, bool ONE>
G1_HD void g1_next_pf(const G1Group& a, const G1Shard* sht, G1Cursor& pf, int& j, int n)
{
    if (j + 1 < n) {
        j++;
        g1_advance<K, ONE>(a, sht, pf);
    }
}

// First word, relative to a unit's first word, of lane l's K words (its chunk).
G1_HD uint32_t g1_lane_word(int lane, int K)
{
    return (uint32_t)(lane * K);
}

// ---------------------------------------------------------------- a workgroup's range

// Workgroup g's range: units ub .. ub + L - 1, segments S_first .. S_first + nseg - 1, and the
// 128-input blocks in the order its units meet them ("occurrences"): the first segment's tile
// rows tr0 .. (blocks tr0 / 8 ..), then every later segment from tile row 0 on (nbpc blocks
// each, the last one possibly fewer); nocc occurrences in all.
struct G1Range {
    int ub, L;
    int S_first, nseg;
    int tr0, nbpc, nb0, nocc;
};

// Occurrence of the unit at tile row tr of the range's k-th segment.
G1_HD int g1_occ_of(const G1Range& w, int k, int tr)
{
    return k == 0 ? (tr >> 3) - (w.tr0 >> 3) : w.nb0 + (k - 1) * w.nbpc + (tr >> 3);
}

template <bool ONE>
G1_HD G1Range g1_range(const G1Group& a, const G1Shard* sht, int g)
{
    G1Range w;
    w.ub = g1_first_unit(a, g);
    w.L = g1_units(a, g);
    const int ntr = a.ntr;
    const int s_first = g1_shard_of_unit<ONE>(a, sht, w.ub);
    w.S_first = g1_sh<ONE>(sht, s_first).sbeg + g1_div(w.ub - g1_sh<ONE>(sht, s_first).ubeg, a.dntr);
    const int ue = w.ub + w.L - 1;
    const int s_last = g1_shard_of_unit<ONE>(a, sht, ue);
    const int rel = ue - g1_sh<ONE>(sht, s_last).ubeg;
    const int cg = g1_div(rel, a.dntr);
    w.nseg = g1_sh<ONE>(sht, s_last).sbeg + cg - w.S_first + 1;
    w.tr0 = w.ub - g1_sh<ONE>(sht, s_first).ubeg - (w.S_first - g1_sh<ONE>(sht, s_first).sbeg) * ntr;
    w.nbpc = ntr >> 3;
    const int tre0 = ntr - 1 < w.tr0 + w.L - 1 ? ntr - 1 : w.tr0 + w.L - 1;
    w.nb0 = (tre0 >> 3) - (w.tr0 >> 3) + 1;
    w.nocc = g1_occ_of(w, g1_sh<ONE>(sht, s_last).sbeg + cg - w.S_first, rel - cg * ntr) + 1;
    return w;
}

// Segment k of the range and 128-input block blk that occurrence i stands for.
G1_HD void g1_occ_block(const G1Group& a, const G1Range& w, int i, int& k, int& blk)
{
    k = 0;
    blk = (w.tr0 >> 3) + i;
    if (i >= w.nb0) {
        const int j = i - w.nb0;
        k = 1 + g1_div(8 * j, a.dntr);          // j / nbpc
        blk = j - (k - 1) * w.nbpc;
    }
}

// A wave's activation-table tasks: the (occurrence i, activation row r) pairs t = i nr + r,
// t = wave, wave + G1_NW, ...  The cursor steps by G1_NW tasks (= q nr + rm) with no
// division and carries the occurrence's segment k, block blk (g1_occ_block), shard s and
// the first segment of shard s + 1 (nxt; INT_MAX past the last shard).
struct G1Task {
    int t, i, r, k, blk, s, nxt;
};

struct G1TaskStep {
    int q, rm;
};

G1_HD G1TaskStep g1_task_step(int nr)
{
    G1TaskStep st{0, G1_NW};
    while (st.rm >= nr) {
        st.rm -= nr;
        st.q++;
    }
    return st;
}

template <bool ONE>
G1_HD G1Task g1_task_first(const G1Group& a, const G1Shard* sht, const G1Range& w, int wave, int nr)
{
    G1Task c{wave, 0, wave, 0, 0, 0, 0};
    while (c.r >= nr) {
        c.r -= nr;
        c.i++;
    }
    g1_occ_block(a, w, c.i, c.k, c.blk);
    c.s = g1_shard_of_seg<ONE>(a, sht, w.S_first + c.k);
    c.nxt = !ONE && c.s + 1 < a.nshards ? sht[c.s + 1].sbeg : 0x7fffffff;
    return c;
}

// Occurrences run through the blocks of the first segment from tr0 / 8, then through every
// block 0 .. nbpc - 1 of each next segment, so the block steps like a mixed-radix counter;
// shards hold consecutive segments, so the shard index only grows.
template <bool ONE>
G1_HD void g1_task_next(const G1Group& a, const G1Shard* sht, const G1Range& w, G1Task& c, int nr, G1TaskStep st)
{
    c.t += G1_NW;
    int d = st.q;
    c.r += st.rm;
    if (c.r >= nr) {
        c.r -= nr;
        d++;
    }
    c.i += d;
    c.blk += d;
    while (c.blk >= w.nbpc) {
        c.blk -= w.nbpc;
        c.k++;
    }
    if constexpr (!ONE)
        while (w.S_first + c.k >= c.nxt) {
            c.s++;
            c.nxt = c.s + 1 < a.nshards ? sht[c.s + 1].sbeg : 0x7fffffff;
        }
}

// Workgroups g_lo .. g_hi whose ranges hold units of segment S (g_hi > g_lo: split).
template <bool ONE>
G1_HD void g1_contributors(const G1Group& a, const G1Shard* sht, int S, int& g_lo, int& g_hi)
{
    const int s = g1_shard_of_seg<ONE>(a, sht, S);
    const int segU0 = g1_sh<ONE>(sht, s).ubeg + (S - g1_sh<ONE>(sht, s).sbeg) * a.ntr;
    g_lo = g1_wg_of(a, segU0);
    g_hi = g1_wg_of(a, segU0 + a.ntr - 1);
}

// ---------------------------------------------------------------- LDS layout and indices

// Units [b, e) of the range's k-th segment, relative to the range (segments are ntr units;
// the first one starts at tile row tr0).
G1_HD void g1_seg_units(const G1Range& w, int ntr, int k, int& b, int& e)
{
    const int first = ntr - w.tr0;
    b = k == 0 ? 0 : first + (k - 1) * ntr;
    e = first + k * ntr;
    if (e > w.L) e = w.L;
}

// Whether a wave's run holds units of [b, e).
G1_HD bool g1_run_meets(const G1Run& run, int b, int e)
{
    return run.n > 0 && run.lo < e && run.lo + run.n > b;
}

// nr = activation rows the tables hold (1, or the call's rows for the multi-row template).
// red[nseg + G1_NW - 1][nr][128] fp32 partial rows | act: the duplicated fp16 activations
// (u32 words) | zero (the A operand of the lanes whose k-block is not theirs).
// Wave ww's partial rows of the range's k-th segment are red[k + ww]: a wave's run is one
// contiguous piece of the range and the runs are in wave order, so two (segment, wave) pairs
// that both hold units never share k + ww (if wave ww meets segment k + 1, wave ww + 1 starts
// at or after it and cannot meet segment k).  Only such pairs are written and read.
//
// A unit's A operand is four 16-byte LDS reads per lane (chunks c = 0..3 of its row's 16
// words), the same immediate offsets for every lane.  One row: act[nocc][8][4 c][4] (every
// A-carrying lane reads the same chunk, a broadcast) and zero[16], starting 8 words past a
// multiple of 16 so that its chunk c never shares a bank with the act chunk c read beside
// it.  Several rows: act[nocc][8][4 c][G1_ROWS slots][4] (chunk c of rows 0..3 is 16
// consecutive words) and zero, its four chunks 16 words apart, starting 16 words past a
// multiple of 32: the zero and act chunks of one read fall in distinct banks for 32 or 64
// banks of 4 bytes.  Measured on MI355X (config 2, SQ_LDS_BANK_CONFLICT per dispatch): one
// row 348,160 -> 0, four rows 2,047,968 -> 655,328 (the table stores and partial rows keep
// the rest), with no change in busy cycles -- the conflicts were off the critical path.
// Slots of rows >= nr are not written (their lanes read row nr - 1).
struct G1Lds {
    int act;                   // u32 offset of act
    int zero;                  // u32 offset of zero
    int words;                 // u32 words in all
};

// u32 words per table entry (occurrence, tile row), bytes between a lane's four A chunks,
// and zero words the kernel clears.
G1_HD constexpr int g1_entry_words(int nr) { return nr == 1 ? 16 : 16 * G1_ROWS; }
G1_HD constexpr int g1_a_chunk(int nr) { return nr == 1 ? 16 : 64; }
G1_HD constexpr int g1_zero_words(int nr) { return nr == 1 ? 16 : 3 * 16 + 4; }

G1_HD G1Lds g1_lds_layout(int nseg, int nocc, int nr)
{
    G1Lds l;
    l.act = (nseg + G1_NW - 1) * nr * 128;
    l.zero = l.act + nocc * 8 * g1_entry_words(nr) + (nr == 1 ? 8 : 16);
    l.words = l.zero + g1_zero_words(nr);
    return l;
}

// First float of wave ww's partial row r of the range's k-th segment in red.
G1_HD int g1_red_row(int k, int ww, int nr, int r)
{
    return ((k + ww) * nr + r) * 128;
}

// u32 word (of act) where lane l stores activation row r's outputs 2l, 2l + 1 of occurrence
// i as two duplicated fp16 pairs: chunk c = l % 4 of tile row l / 8 holds rows 2c +
// {0, 1, 8, 9}[t] of the tile row, lane l's are t = 2 ((l % 8) / 4), t + 1.
G1_HD int g1_act_word(int i, int lane, int nr, int r)
{
    const int c = lane & 3, t = 2 * ((lane >> 2) & 1);
    const int e = (i * 8 + (lane >> 3)) * g1_entry_words(nr);
    return nr == 1 ? e + 4 * c + t : e + (c * G1_ROWS + r) * 4 + t;
}

// The lane's A operand: row i = lane % 16 in k-block lane / 16, which carries activation row
// i / 4 when i % 4 is that k-block (asel = 1) and zeros otherwise (asel = 0).  Its chunk c
// for a unit whose table entry starts at byte e is at e * asel + aoff + c * g1_a_chunk(nr).
G1_HD uint32_t g1_asel(int lane)
{
    return ((lane & 15) & 3) == (lane >> 4) ? 1u : 0u;
}

G1_HD uint32_t g1_aoff(int lane, int nr, const G1Lds& l)
{
    const int rr = (lane & 15) >> 2;
    return g1_asel(lane) ? (uint32_t)(4 * l.act + (rr < nr - 1 ? rr : nr - 1) * 16) : (uint32_t)(4 * l.zero);
}

// Byte offset (relative to act) of the table entry of occurrence occ, tile row tr.
G1_HD uint32_t g1_a_entry(int occ, int tr, int nr)
{
    return (uint32_t)((occ * 8 + (tr & 7)) * g1_entry_words(nr)) * 4u;
}

// Where lane l's accumulators land in a partial row: activation row yrow, outputs
// ycol + 32 e (+ 8 for the second accumulator), e = 0..3.
G1_HD int g1_yrow(int lane) { return lane >> 4; }
G1_HD int g1_ycol(int lane) { return 16 * ((lane >> 3) & 1) + (lane & 7); }

// ---------------------------------------------------------------- global indices

// Element offset of activation row r's 128-input block blk in x (rows r >= nrows repeat the
// last row; their results are not stored).
G1_HD long g1_x_elem(const G1Group& a, int r, int blk)
{
    return (long)(r < a.nrows - 1 ? r : a.nrows - 1) * ((long)a.ntr * 16) + blk * 128;
}

// First float of slot (segment S, workgroup g): R rows of 128 partials.  Slots of one
// segment are S + g_lo .. S + g_hi: distinct for distinct (S, g) because workgroup ranges
// are ordered and non-empty.
G1_HD long g1_slot(int S, int g, int R)
{
    return (long)(S + g) * R * 128;
}

// u64 word, relative to the first slot a reader starts at, of row r of the t-th slot after
// it (each u64 holds a lane's two partials).
G1_HD long g1_slot_word(int t, int R, int r)
{
    return ((long)t * R + r) * 64;
}

// Accumulators of split segments.  Each output of a split segment has one 64-bit word: bits
// 52..63 count the workgroups that have added into it, bits 0..51 hold the sum of their
// transformed partial outputs as a two's complement fixed-point number with G1_FX_FRAC
// fractional bits.  A partial is clamped to +-G1_FX_MAX first, so the sum of at most G1_GMAX
// (2^11) of them stays inside +-2^51 (65504 * 2^24 * 2^11 < 2^51) and never carries into the
// count.  Outputs of magnitude 2^-14 and above (fp16 normals) keep at least the resolution of
// their own fp16 spacing; larger partials saturate, and a NaN partial reads as -G1_FX_MAX.
constexpr int G1_FX_CBIT = 52;
constexpr int G1_FX_FRAC = 24;
constexpr float G1_FX_MAX = 65504.f;

// Word of output 2 lane + j (j = 0, 1) of row r of segment S.
G1_HD long g1_acc_word(int S, int R, int r, int lane, int j)
{
    return ((long)S * R + r) * 128 + 2 * lane + j;
}

// Bytes of a group's accumulators.
inline size_t g1_acc_bytes(int nsegs, int R) { return (size_t)nsegs * R * 128 * sizeof(unsigned long long); }

// ---------------------------------------------------------------- host: planning

inline G1Div g1_magic(uint32_t d)
{
    int l = 0;
    while ((1ull << l) < d) l++;
    return G1Div{(uint32_t)(((1ull << (31 + l)) / d) + 1), l - 1};
}

// Dynamic LDS a launch needs for nr activation rows: partial rows for the most segments
// (shard, column group) a workgroup range of L = ceil(U / G) units can touch (nseg, plus
// G1_NW - 1: red[k + ww]), a transformed activation block for each 128-input block it can
// meet, and the 64-byte zero operand.  Segments are ntr units, a multiple of 8, so a
// range's blocks are the 8-unit-aligned pieces of the unit numbering it meets: at most
// floor((L + 6) / 8) + 1.
inline size_t g1_lds_bytes(int U, int G, int ntr, int nr)
{
    const int L = (U + G - 1) / G;
    const int nseg = (L - 1 + ntr - 1) / ntr + 1;
    const int nocc = (L + 6) / 8 + 1;
    return (size_t)g1_lds_layout(nseg, nocc, nr).words * sizeof(uint32_t);
}

// Row-count template of a call: one activation row, or up to four (G1_ROWS).
inline int g1_R(int rows) { return rows == 1 ? 1 : G1_ROWS; }

// Per-shard share of the slot area: slots of R rows for up to G1_GMAX workgroups and one
// per column group.
inline size_t g1_slot_bytes(int oc, int rows)
{
    return (size_t)(G1_GMAX + oc / 128) * g1_R(rows) * 128 * sizeof(float);
}

// Fills one group from shards[idx[0..n-1]] (same K and codebook) into table entries
// tab[0..n-1]; returns its unit count.
inline long g1_group(G1Group& grp, G1Shard* tab, const GemvShard* shards, const int* idx, int n, const uint16_t* A,
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

// Workgroup split of a group of U units into G ranges, and its share of the slots -- or, when
// the accumulator area (acc, acc_bytes; abase bytes of it taken by earlier groups of the call)
// still holds the group's words, its share of that instead.
inline int g1_place(G1Group& grp, long U, int G, int R, char* slots, size_t& sbase, size_t slot_bytes, char* acc,
                    size_t acc_bytes, size_t& abase)
{
    grp.acc = nullptr;
    if (acc && abase + g1_acc_bytes(grp.nsegs, R) <= acc_bytes) {
        grp.acc = reinterpret_cast<unsigned long long*>(acc + abase);
        abase += g1_acc_bytes(grp.nsegs, R);
    }
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

// Whether some segment of the group lies in more than one workgroup range and the group has
// no accumulators (then the launch needs gemv1_finish_kernel): segment S is units S ntr ..
// S ntr + ntr - 1.
inline bool g1_any_split(const G1Group& grp)
{
    if (grp.acc) return false;
    const long big = (long)grp.r * (grp.q + 1);
    auto wg_of = [&](long u) { return u < big ? u / (grp.q + 1) : grp.r + (u - big) / grp.q; };
    for (int S = 0; S < grp.nsegs; S++)
        if (wg_of((long)S * grp.ntr) != wg_of((long)S * grp.ntr + grp.ntr - 1)) return true;
    return false;
}

constexpr size_t G1_LDS_PER_CU = 160 * 1024;

// Units in flight per wave for a launch of the R-row template with `lds` bytes of LDS per
// workgroup: 1, or G1_DEEP for the four-row template when fewer than G1_WG_PER_CU workgroups
// fit a CU's LDS.  Measured on MI355X at settled clocks: the K = 6 lm_head (two resident) at
// 2 / 3 / 4 rows 149 / 154 / 161 -> 136 / 151 / 155 us per call, gate_up at 4 rows (three
// resident) 33.6-33.8 -> 32.7-33.3 us; with four resident (qkv at 4 rows) depth 2 was
// 0.2-0.5 us slower, and at one row it did not change the lm_head.
G1_HD int g1_depth(int R, size_t lds)
{
    return R > 1 && lds > G1_LDS_PER_CU / G1_WG_PER_CU ? G1_DEEP : 1;
}

// Workgroup counts G[0..ns) of one launch whose groups have U[t] units (nr activation rows in
// the tables), for the most
// workgroups per CU (up to G1_WG_PER_CU) whose LDS lets them all stay resident; returns
// that number and the launch's LDS per workgroup.  When even one workgroup per CU cannot hold
// its range (few CUs, or a very large shard), the launch takes more workgroups than stay
// resident -- G1_UNITS_PER_WG units each, up to G1_GMAX; no workgroup waits for another, so
// they simply run in turn -- and 0 is returned.  The caller refuses a launch whose LDS still
// exceeds G1_LDS_PER_CU.
inline int g1_split(const long* U, int ns, int ntr, int nr, int cus, int* G, size_t& lds)
{
    auto share = [&](int gmax) {
        long Gsum = 0;
        for (int t = 0; t < ns; t++) {
            G[t] = (int)std::min<long>(gmax, std::max<long>(1, U[t] / G1_UNITS_PER_WG));
            Gsum += G[t];
        }
        if (Gsum > gmax)   // share the workgroups in proportion to the groups' sizes
            for (int t = 0; t < ns; t++) G[t] = std::max(1, (int)((long)G[t] * gmax / Gsum));
        lds = 0;
        for (int t = 0; t < ns; t++) lds = std::max(lds, g1_lds_bytes((int)U[t], G[t], ntr, nr));
    };
    for (int wgpc = G1_WG_PER_CU; wgpc >= 1; wgpc--) {
        share(std::min(G1_GMAX, wgpc * cus));
        if ((size_t)wgpc * lds <= G1_LDS_PER_CU) return wgpc;
    }
    share(G1_GMAX);
    return 0;
}

// One launch of the plan: a single group (gemv1_kernel, args) or several (gemv1_multi_kernel,
// m), then, if `finish`, the finish kernel over `fblocks` blocks.
struct G1Launch {
    bool multi, one, finish;
    int K, cb, R, G, fblocks;
    size_t lds;
    const G1Args* args;
    const G1Multi* m;
};

// 1..4 activation rows: the shards are grouped by (K, codebook), at most G1_MAXSH shards a
// group.  A launch takes whole groups of one codebook, at most G1_MAXSH shards in all: one
// group is a gemv1_kernel launch, several share a gemv1_multi_kernel launch with their
// workgroup counts scaled to the resident limit together.  Workgroups per CU: four, or
// fewer where a launch's LDS per workgroup (larger with four rows) would not let four
// stay resident.  Calls emit(const G1Launch&) per launch in order; stops at the first
// status other than EXL3_OK.
template <class Emit>
int g1_plan(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* slots, size_t slot_bytes,
            char* acc, size_t acc_bytes, int cus, Emit&& emit)
{
    if (rows < 1 || rows > G1_ROWS) return set_error(EXL3_ERR_ARG, "exl3_gemv: rows=%d is not in 1..%d", rows, G1_ROWS);
    const int R = g1_R(rows);
    const int ic = shards[0].ic;
    const int ntr = ic / 16;

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

    size_t sbase = 0, abase = 0;
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
        G1Launch L = {};
        L.cb = gcb[j0];
        L.R = R;
        g1_split(U, ns, ntr, R == 1 ? 1 : rows, cus, G, L.lds);
        if (L.lds > G1_LDS_PER_CU)
            return set_error(EXL3_ERR_ARG,
                             "exl3_gemv: %ld tile-row units need %zu bytes of LDS per workgroup (limit %zu)",
                             U[0], L.lds, G1_LDS_PER_CU);
        if (ns == 1) {
            G1Args args = {};
            args.grp = m.grp[0];
            for (int i = 0; i < gn[sel[0]]; i++) args.sh[i] = m.sh[i];
            int rc = g1_place(args.grp, U[0], G[0], R, slots, sbase, slot_bytes, acc, acc_bytes, abase);
            if (rc != EXL3_OK) return rc;
            L.one = gn[sel[0]] == 1;
            L.K = gK[sel[0]];
            L.G = G[0];
            L.finish = g1_any_split(args.grp);
            L.fblocks = args.grp.nsegs;
            L.args = &args;
            rc = emit(static_cast<const G1Launch&>(L));
            if (rc != EXL3_OK) return rc;
            continue;
        }
        int gb = 0, nb = 0;
        for (int t = 0; t < ns; t++) {
            const int rc = g1_place(m.grp[t], U[t], G[t], R, slots, sbase, slot_bytes, acc, acc_bytes, abase);
            if (rc != EXL3_OK) return rc;
            m.gbeg[t] = gb;
            gb += G[t];
            m.fbeg[t] = nb;
            nb += m.grp[t].nsegs;
            L.finish = L.finish || g1_any_split(m.grp[t]);
        }
        m.ngrp = ns;
        L.multi = true;
        L.G = gb;
        L.fblocks = nb;
        L.m = &m;
        const int rc = emit(static_cast<const G1Launch&>(L));
        if (rc != EXL3_OK) return rc;
    }
    return EXL3_OK;
}

}  // namespace exl3
