// Work plan of the 5..16-row decode GEMV (gemv16.hip): argument blocks, the unit numbering and
// cursor, the set-up kernel's activation layout, the LDS layout and every index the kernels
// form, and the host-side grouping of shards into launches.  The workgroup ranges, wave runs
// and segment bookkeeping are gemv1_plan.h's (a gemv16 segment is a 32-output strip).
//
// As in gemv1_plan.h, everything the kernels compute an address from is a __host__ __device__
// function here, so the CPU address replay (replay/addr_replay.hip) walks the same arithmetic.
#pragma once

#include "gemv1_plan.h"

namespace exl3 {

constexpr int G16_ROWS = 16;             // activation rows of an MFMA (rows >= nrows unused)
constexpr int G16_STRIP = 32;            // outputs of a strip (two tile columns)
constexpr int G16_QIN = 64;              // inputs of a unit (four tile rows)
// Words (u32) of one unit's activation fragments: 4 MFMA steps m x 64 lanes x 2 u32 (four
// fp16 inputs, each duplicated into its two k-slots in registers).
constexpr int G16_AH_UNIT = 4 * 64 * 2;

// A unit is 4 tile rows x 2 tile columns (64 inputs x 32 outputs, 8 tiles, 64 chunks): lane
// l = 16 j + n decodes chunk c = n % 8 of tile (tile row 4 q + j, tile column 2 strip + n / 8),
// so the 16 lanes of each k-group j hold the same 16 output columns.  MFMA (m, h) takes
// positions 8 m + 4 h + t (t = 0..3) of every lane's chunk -- tile rows 2 m + {0, 1, 8, 9}[t]
// of column c + 8 h -- as B (each masked word's two fp16 halves as two k-slots), and as A the
// matching inputs of all 16 activation rows, each duplicated: A row i, k-group j holds row i's
// inputs 64 q + 16 j + 2 m + {0, 1, 8, 9} (stored once each, duplicated when loaded).  C column n of MFMA (m, h) is output
// 16 (n / 8) + n % 8 + 8 h of the strip; the four m accumulate into the same C.
struct G16Shard {
    const uint32_t* trellis;   // (ic/16, oc/16, 8K) u32
    const uint32_t* ah;        // activation fragments of this shard (gemv16 set-up kernel)
    const uint16_t* svh;       // (oc)
    uint16_t* C;               // (nrows, ldc) fp16 output, columns [0, oc)
    long ldc;
    int ubeg;                  // first unit of the shard
    int sbeg;                  // first strip of the shard
    int oc16;                  // tile columns
    int nstrip;                // strips (oc / 32)
};

// A group of shards with one K and codebook: G1Group's fields with ntr = units per strip
// (ic / 64), nsegs = strips, slots = (G + strips) x 16 x 32 fp32.
struct G16Args {
    G1Group grp;
    G16Shard sh[G1_MAXSH];
};

struct G16Multi {
    G1Group grp[G1_MAXSH];
    G16Shard sh[G1_MAXSH];
    int gbeg[G1_MAXSH], sh0[G1_MAXSH], K[G1_MAXSH], fbeg[G1_MAXSH];
    int ngrp;
};

template <bool ONE>
G1_HD const G16Shard& g16_sh(const G16Shard* sht, int s)
{
    return sht[ONE ? 0 : s];
}

template <bool ONE>
G1_HD int g16_shard_of_unit(const G1Group& a, const G16Shard* sht, int u)
{
    int s = 0;
    if constexpr (!ONE) {
#pragma unroll
        for (int i = 1; i < G1_MAXSH; i++)
            if (i < a.nshards && u >= sht[i].ubeg) s = i;
    }
    return s;
}

template <bool ONE>
G1_HD int g16_shard_of_seg(const G1Group& a, const G16Shard* sht, int S)
{
    int s = 0;
    if constexpr (!ONE) {
#pragma unroll
        for (int i = 1; i < G1_MAXSH; i++)
            if (i < a.nshards && S >= sht[i].sbeg) s = i;
    }
    return s;
}

// Workgroup g's range (G1Range's ub, L, S_first, nseg, tr0; no activation occurrences).
template <bool ONE>
G1_HD G1Range g16_range(const G1Group& a, const G16Shard* sht, int g)
{
    G1Range w = {};
    w.ub = g1_first_unit(a, g);
    w.L = g1_units(a, g);
    const int s_first = g16_shard_of_unit<ONE>(a, sht, w.ub);
    w.S_first = g16_sh<ONE>(sht, s_first).sbeg + g1_div(w.ub - g16_sh<ONE>(sht, s_first).ubeg, a.dntr);
    const int ue = w.ub + w.L - 1;
    const int s_last = g16_shard_of_unit<ONE>(a, sht, ue);
    w.nseg = g16_sh<ONE>(sht, s_last).sbeg + g1_div(ue - g16_sh<ONE>(sht, s_last).ubeg, a.dntr) - w.S_first + 1;
    w.tr0 = w.ub - g16_sh<ONE>(sht, s_first).ubeg - (w.S_first - g16_sh<ONE>(sht, s_first).sbeg) * a.ntr;
    return w;
}

// Workgroups g_lo .. g_hi whose ranges hold units of strip S.
template <bool ONE>
G1_HD void g16_contributors(const G1Group& a, const G16Shard* sht, int S, int& g_lo, int& g_hi)
{
    const int s = g16_shard_of_seg<ONE>(a, sht, S);
    const int segU0 = g16_sh<ONE>(sht, s).ubeg + (S - g16_sh<ONE>(sht, s).sbeg) * a.ntr;
    g_lo = g1_wg_of(a, segU0);
    g_hi = g1_wg_of(a, segU0 + a.ntr - 1);
}

// ---------------------------------------------------------------- cursor

struct G16Cursor {
    int s, strip, q, S;
    long stride;               // words between consecutive units of a strip (4 tile rows)
    const uint32_t* p;         // first word of tile (4 q, 2 strip)
    const uint32_t* ah;        // the unit's activation fragments
};

template <int K, bool ONE>
G1_HD void g16_seat(const G16Shard* sht, G16Cursor& c)
{
    const G16Shard& e = g16_sh<ONE>(sht, c.s);
    c.stride = 4L * e.oc16 * (8 * K);
    c.p = e.trellis + ((long)(4 * c.q) * e.oc16 + 2 * c.strip) * (8 * K);
    c.ah = e.ah + (long)c.q * G16_AH_UNIT;
}

template <int K, bool ONE>
G1_HD G16Cursor g16_cursor_at(const G1Group& a, const G16Shard* sht, int u)
{
    G16Cursor c;
    c.s = g16_shard_of_unit<ONE>(a, sht, u);
    const int rel = u - g16_sh<ONE>(sht, c.s).ubeg;
    c.strip = g1_div(rel, a.dntr);
    c.q = rel - c.strip * a.ntr;
    c.S = g16_sh<ONE>(sht, c.s).sbeg + c.strip;
    g16_seat<K, ONE>(sht, c);
    return c;
}

template <int K, bool ONE>
G1_HD void g16_advance(const G1Group& a, const G16Shard* sht, G16Cursor& c)
{
    c.q++;
    c.p += c.stride;
    c.ah += G16_AH_UNIT;
    if (c.q == a.ntr) {
        c.q = 0;
        c.S++;
        if (++c.strip == g16_sh<ONE>(sht, c.s).nstrip) {
            c.s++;
            c.strip = 0;
        }
        g16_seat<K, ONE>(sht, c);
    }
}

template <int K, bool ONE>
G1_HD void g16_next_pf(const G1Group& a, const G16Shard* sht, G16Cursor& pf, int& j, int n)
{
    if (j + 1 < n) {
        j++;
        g16_advance<K, ONE>(a, sht, pf);
    }
}

// First word of lane l's chunk relative to the unit's first word (shard with oc16 tile
// columns): tile row j = l / 16, tile column (l % 16) / 8, chunk l % 8.
G1_HD long g16_lane_word(int lane, int oc16, int K)
{
    return ((long)(lane >> 4) * oc16 + ((lane & 15) >> 3)) * (8 * K) + (lane & 7) * K;
}

// Workgroup of block b in an n-block single-group launch.  Blocks go to the 8 XCDs in turn
// (block b on XCD b % 8), each XCD with its own L2.  At odd K a unit's run of 64 K bytes per
// tile row is not a multiple of the 128-byte line, so the two strips of a pair share a line
// in every tile row; numbering each XCD's blocks consecutively puts neighbouring workgroups
// -- neighbouring strips -- on one XCD, which then reads each shared line once.  Measured
// on MI355X (gate_up, two 17408 x 5120 shards at K = 3, 16 rows): 45.2-45.3 -> 43.9-44.4 us
// per call.  At even K (whole lines) it was 1-2 us slower on the lm_head, and in a launch of
// several groups it gives each XCD one group's units (qkv: the K = 5 k and v on two XCDs),
// so both keep the plain order.  A bijection of [0, n).
G1_HD int g16_block_wg(int b, int n, int K)
{
    if (!(K & 1)) return b;
    const int x = b & 7, y = b >> 3, base = n >> 3, rem = n & 7;
    return x * base + (x < rem ? x : rem) + y;
}

// u32 offset of lane l's A fragment of MFMA step m in a unit's activation fragments (two
// words: slots 0, 1 and slots 2, 3, one fp16 input per slot).
G1_HD int g16_ah_word(int m, int lane)
{
    return (m * 64 + lane) * 2;
}

// The lane whose A fragment lane l reads when the call has nrows rows: lane 16 j + i holds
// activation row i, and a row past nrows (zeros from the set-up; its C row is never
// stored) reads row nrows - 1 of the same k-group instead.
G1_HD int g16_ah_lane(int lane, int nrows)
{
    const int i = lane & 15;
    return (lane & ~15) | (i < nrows ? i : nrows - 1);
}

// Where the set-up kernel puts input k (of ic) of activation row i: fp16 (u16) offset in the
// shard's fragments.  k = 64 q + 16 j + rr, rr = 2 m + o, o in {0, 1, 8, 9} at slot
// t = o % 2 + 2 (o / 8); lane 16 j + i of step m reads slots 0..3 (u16 2 w + t of its words),
// so inputs k and k + 1 (k even) share one u32.
G1_HD long g16_ah_elem(int i, int k)
{
    const int q = k >> 6, j = (k >> 4) & 3, rr = k & 15;
    const int m = (rr & 7) >> 1, t = (rr & 1) + 2 * (rr >> 3);
    return 2 * ((long)q * G16_AH_UNIT + g16_ah_word(m, 16 * j + i)) + t;
}

// u32 words of one shard's activation fragments.
G1_HD long g16_ah_words(int ic)
{
    return (long)(ic / G16_QIN) * G16_AH_UNIT;
}

// ---------------------------------------------------------------- LDS and slots

// red[nseg + G1_NW - 1][16 rows][32 outputs] fp32: wave ww's partials of the range's k-th strip
// at red[k + ww] (the pairing of gemv1_plan.h's g1_red_row).
G1_HD int g16_red_bytes(int nseg)
{
    return (nseg + G1_NW - 1) * G16_ROWS * G16_STRIP * 4;
}

G1_HD int g16_red_row(int k, int ww)
{
    return (k + ww) * G16_ROWS * G16_STRIP;
}

// Lane l's accumulator (h, t) in a strip's 16 x 32 partials: row 4 (l / 16) + t, output
// 16 ((l % 16) / 8) + l % 8 + 8 h.
G1_HD int g16_acc_index(int lane, int h, int t)
{
    return (4 * (lane >> 4) + t) * G16_STRIP + 16 * ((lane & 15) >> 3) + (lane & 7) + 8 * h;
}

// Slot (strip S, workgroup g): 16 x 32 fp32 (distinct for distinct pairs, as g1_slot).
G1_HD long g16_slot(int S, int g)
{
    return (long)(S + g) * G16_ROWS * G16_STRIP;
}

// ---------------------------------------------------------------- host: planning

inline size_t g16_lds_bytes(int U, int G, int nq)
{
    const int L = (U + G - 1) / G;
    const int nseg = (L - 1 + nq - 1) / nq + 1;
    return (size_t)g16_red_bytes(nseg);
}

// Per-shard share of the 5..16-row workspace: the shard's activation fragments, then slots for
// up to G1_GMAX workgroups and one per strip.
inline size_t g16_shard_bytes(int ic, int oc)
{
    const size_t ah = ((size_t)g16_ah_words(ic) * 4 + 255) & ~(size_t)255;
    return ah + (size_t)(G1_GMAX + oc / G16_STRIP) * G16_ROWS * G16_STRIP * 4;
}

// Set-up kernel of a call: for every shard s and 128-input block b, one workgroup writes
// fp16(H128(A_r * suh_s)) of block b for the rows r < nrows (zeros for the others) into the
// shard's fragments.
struct G16Prep {
    const uint16_t* A;
    int rows, ic, nsh, nblk;
    const uint16_t* suh[EXL3_MAX_SHARDS];
    uint32_t* ah[EXL3_MAX_SHARDS];
};

// Set-up workgroup g (four waves) of a call: shard s, 128-input block b.  Wave wv transforms
// activation rows wv, wv + 4, wv + 8, wv + 12 (rows from `rows` on are zeros: no decode lane
// reads them, g16_ah_lane), then lane t of the workgroup stores words 4 t .. 4 t + 3 of the
// block's fragment area -- units 2 b and 2 b + 1, 2 G16_AH_UNIT words from word
// g16_prep_base(b) of the shard's fragments -- one 16-byte store each, in lane order.
constexpr int G16_PREP_LANES = 256;
G1_HD void g16_prep_wg(const G16Prep& p, int g, int& s, int& b)
{
    b = g % p.nblk;
    s = g / p.nblk;
}
G1_HD long g16_prep_base(int b) { return (long)b * 2 * G16_AH_UNIT; }
// Activation row i and input k (of the block's 128; k even) of the two inputs in word w of a
// block's fragment area: word (m 64 + 16 j + i) 2 + h of unit qq holds inputs
// 64 qq + 16 j + 8 h + 2 m and the next (g16_ah_elem).
G1_HD void g16_prep_src(int w, int& i, int& k)
{
    const int qq = w / G16_AH_UNIT, ww = w % G16_AH_UNIT;
    const int m = ww >> 7, lf = (ww >> 1) & 63, h = ww & 1;
    i = lf & 15;
    k = 64 * qq + 16 * (lf >> 4) + 8 * h + 2 * m;
}

struct G16Launch {
    bool multi, one;
    int K, cb, G, fblocks;
    size_t lds;
    const G16Args* args;
    const G16Multi* m;
};

// Fills one group from shards[idx[0..n-1]] into table entries tab[0..n-1] (fragments at
// ah[idx[j]]); returns its unit count.
inline long g16_group(G1Group& grp, G16Shard* tab, const GemvShard* shards, const int* idx, int n,
                      uint32_t* const* ah, int nq, int rows)
{
    grp = G1Group{};
    grp.nrows = rows;
    grp.ntr = nq;
    grp.nshards = n;
    long U = 0;
    int nsegs = 0;
    for (int j = 0; j < n; j++) {
        const GemvShard& d = shards[idx[j]];
        G16Shard& e = tab[j];
        e.trellis = d.trellis;
        e.ah = ah[idx[j]];
        e.svh = d.svh;
        e.C = d.C;
        e.ldc = d.ldc;
        e.ubeg = (int)U;
        e.sbeg = nsegs;
        e.oc16 = d.oc / 16;
        e.nstrip = d.oc / G16_STRIP;
        U += (long)(d.oc / G16_STRIP) * nq;
        nsegs += d.oc / G16_STRIP;
    }
    grp.nsegs = nsegs;
    return U;
}

inline int g16_place(G1Group& grp, long U, int G, char* slots, size_t& sbase, size_t slot_bytes)
{
    if (U > (1L << 30))
        return set_error(EXL3_ERR_ARG, "exl3_gemv: %ld units in one launch (limit 2^30)", U);
    const size_t need = (size_t)(G + grp.nsegs) * G16_ROWS * G16_STRIP * 4;
    if (sbase + need > slot_bytes)
        return set_error(EXL3_ERR_WORKSPACE, "exl3_gemv: slot area of %zu bytes, %zu needed", slot_bytes, sbase + need);
    grp.U = (int)U;
    grp.G = G;
    grp.q = (int)(U / G);
    grp.r = (int)(U % G);
    grp.dntr = g1_magic((uint32_t)grp.ntr);
    grp.dq = g1_magic((uint32_t)grp.q);
    grp.dq1 = g1_magic((uint32_t)grp.q + 1);
    grp.slots = reinterpret_cast<float*>(slots + sbase);
    sbase += need;
    return EXL3_OK;
}

// Units per workgroup the 5..16-row plan aims for (the batch-1 plan's G1_UNITS_PER_WG is 32):
// with fewer, a mid-size layer still fills every CU with G1_WG_PER_CU workgroups (qkv at 16
// rows: 640 -> 1024 workgroups, 21.3-21.8 -> 20.8 us per call on MI355X; gate_up and the
// lm_head are capped at G1_WG_PER_CU per CU either way and did not change).
constexpr int G16_UNITS_PER_WG = 16;

// Workgroup counts of one launch: G16_UNITS_PER_WG units each, up to G1_WG_PER_CU workgroups
// per CU resident, shared in proportion to the groups' sizes.  Where that leaves a range so long
// that its partial strips would not let G1_WG_PER_CU workgroups share a CU (few CUs, very large
// shards), a group takes more workgroups than stay resident (no workgroup waits for another).
inline void g16_split(const long* U, int ns, int nq, int cus, int* G, size_t& lds)
{
    const int gmax = std::min(G1_GMAX, G1_WG_PER_CU * cus);
    long Gsum = 0;
    for (int t = 0; t < ns; t++) {
        G[t] = (int)std::min<long>(gmax, std::max<long>(1, U[t] / G16_UNITS_PER_WG));
        Gsum += G[t];
    }
    if (Gsum > gmax)
        for (int t = 0; t < ns; t++) G[t] = std::max(1, (int)((long)G[t] * gmax / Gsum));
    lds = 0;
    for (int t = 0; t < ns; t++) {
        while (g16_lds_bytes((int)U[t], G[t], nq) > G1_LDS_PER_CU / G1_WG_PER_CU && G[t] < G1_GMAX && G[t] < U[t])
            G[t] = (int)std::min<long>(std::min<long>(G1_GMAX, U[t]), 2L * G[t]);
        lds = std::max(lds, g16_lds_bytes((int)U[t], G[t], nq));
    }
}

// 5..16 rows: shards grouped by (K, codebook) as in g1_plan; one set-up kernel for the call
// (fills prep), then per launch the decode kernel and the finish kernel (every strip goes
// through the slots: the output Hadamard needs four strips).  The workspace holds, per shard
// in call order, g16_shard_bytes: the fragments, then that shard's share of the slots.
template <class Emit>
int g16_plan(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* ws, size_t ws_bytes, int cus,
             G16Prep& prep, Emit&& emit)
{
    if (rows < 1 || rows > G16_ROWS) return set_error(EXL3_ERR_ARG, "exl3_gemv: rows=%d is not in 1..%d", rows, G16_ROWS);
    const int ic = shards[0].ic;
    const int nq = ic / G16_QIN;
    size_t need = 0;
    for (int i = 0; i < nshards; i++) need += g16_shard_bytes(ic, shards[i].oc);
    if (need > ws_bytes)
        return set_error(EXL3_ERR_WORKSPACE, "exl3_gemv: workspace of %zu bytes, %zu needed", ws_bytes, need);
    // fragments first (one region per shard), slots after all of them
    uint32_t* ah[EXL3_MAX_SHARDS];
    size_t off = 0;
    for (int i = 0; i < nshards; i++) {
        ah[i] = reinterpret_cast<uint32_t*>(ws + off);
        off += ((size_t)g16_ah_words(ic) * 4 + 255) & ~(size_t)255;
    }
    char* slots = ws + off;
    const size_t slot_bytes = need - off;
    prep = G16Prep{};
    prep.A = A;
    prep.rows = rows;
    prep.ic = ic;
    prep.nsh = nshards;
    prep.nblk = ic / 128;
    for (int i = 0; i < nshards; i++) {
        prep.suh[i] = shards[i].suh;
        prep.ah[i] = ah[i];
    }

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
        int sel[G1_MAXSH], ns = 0, nsh = 0;
        for (int j = j0; j < ng; j++)
            if (!done[j] && gcb[j] == gcb[j0] && nsh + gn[j] <= G1_MAXSH) {
                sel[ns++] = j;
                nsh += gn[j];
                done[j] = true;
            }
        G16Multi m = {};
        long U[G1_MAXSH];
        int G[G1_MAXSH], sh0 = 0;
        for (int t = 0; t < ns; t++) {
            const int j = sel[t];
            m.sh0[t] = sh0;
            m.K[t] = gK[j];
            U[t] = g16_group(m.grp[t], m.sh + sh0, shards, gidx[j], gn[j], ah, nq, rows);
            sh0 += gn[j];
        }
        G16Launch L = {};
        L.cb = gcb[j0];
        g16_split(U, ns, nq, cus, G, L.lds);
        if (L.lds > G1_LDS_PER_CU)
            return set_error(EXL3_ERR_ARG, "exl3_gemv: %ld units need %zu bytes of LDS per workgroup (limit %zu)", U[0],
                             L.lds, G1_LDS_PER_CU);
        if (ns == 1) {
            G16Args args = {};
            args.grp = m.grp[0];
            for (int i = 0; i < gn[sel[0]]; i++) args.sh[i] = m.sh[i];
            int rc = g16_place(args.grp, U[0], G[0], slots, sbase, slot_bytes);
            if (rc != EXL3_OK) return rc;
            L.one = gn[sel[0]] == 1;
            L.K = gK[sel[0]];
            L.G = G[0];
            L.fblocks = args.grp.nsegs / 4;
            L.args = &args;
            rc = emit(static_cast<const G16Launch&>(L));
            if (rc != EXL3_OK) return rc;
            continue;
        }
        int gb = 0, nb = 0;
        for (int t = 0; t < ns; t++) {
            const int rc = g16_place(m.grp[t], U[t], G[t], slots, sbase, slot_bytes);
            if (rc != EXL3_OK) return rc;
            m.gbeg[t] = gb;
            gb += G[t];
            m.fbeg[t] = nb;
            nb += m.grp[t].nsegs / 4;
        }
        m.ngrp = ns;
        L.multi = true;
        L.G = gb;
        L.fblocks = nb;
        L.m = &m;
        const int rc = emit(static_cast<const G16Launch&>(L));
        if (rc != EXL3_OK) return rc;
    }
    return EXL3_OK;
}

}  // namespace exl3
