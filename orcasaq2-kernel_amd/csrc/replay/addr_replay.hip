// CPU address replay of the GEMV and stream-K GEMM kernels (test tool, not part of the C ABI).
//
// A call plans a launch sequence with the product's own planning code (g1_plan of
// gemv1_plan.h, sk_plan_* of gemm_sk_plan.h) over fake device buffers, then walks every
// workgroup, wave and lane of each launch through the same __host__ __device__ index
// functions the kernels call, in the kernels' loop order, and checks
//   * every global load and store against the buffer it addresses (trellis, suh, svh,
//     activations, outputs, slots, counters), every LDS access against the launch's
//     dynamic LDS and the region it belongs to;
//   * coverage: each unit / K-step decoded exactly once, each output element written exactly
//     once, each slot read after the launch that writes it and holding the partial the
//     reader expects (segment or tile, workgroup, row), each activation-table read of the
//     occurrence and block the unit needs.
// Nothing here runs on a GPU; the library is built with hipcc only because the shared index
// functions are marked __host__ __device__.
#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "../gemm_sk_plan.h"
#include "../gemv16_plan.h"
#include "../gemv1_plan.h"

namespace exl3 {

// The product's error recorder, as the planning code calls it.
thread_local char g_err[512];

int set_error(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char*) { return EXL3_OK; }

}  // namespace exl3

using namespace exl3;

namespace {

thread_local std::string g_msg;

// Fake device buffers: buffer b starts at b << 40, so any address maps back to (buffer,
// byte offset) and an index outside a buffer cannot land in another one.
constexpr int FAKE_SHIFT = 40;
enum Buf { B_NONE, B_X, B_C, B_SLOTS, B_WS, B_ACC, B_TRELLIS = 16, B_SUH = 48, B_SVH = 80, B_AH = 112 };

inline uintptr_t fake(int b) { return (uintptr_t)b << FAKE_SHIFT; }
template <class T>
inline T* fake_ptr(int b) { return reinterpret_cast<T*>(fake(b)); }
inline int buf_of(const void* p) { return (int)((uintptr_t)p >> FAKE_SHIFT); }
inline long off_of(const void* p) { return (long)((uintptr_t)p & (((uintptr_t)1 << FAKE_SHIFT) - 1)); }

struct Fail {
    std::string what;
};

[[noreturn]] void fail(const char* fmt, ...)
{
    char b[640];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(b, sizeof b, fmt, ap);
    va_end(ap);
    throw Fail{b};
}

// A byte range [p, p + n) must lie inside buffer `buf` of `size` bytes.
void need_in(const void* p, long n, int buf, long size, const char* what)
{
    if (buf_of(p) != buf) fail("%s: address in buffer %d, expected buffer %d", what, buf_of(p), buf);
    const long o = off_of(p);
    if (o < 0 || o + n > size) fail("%s: bytes [%ld, %ld) outside [0, %ld)", what, o, o + n, size);
}

struct ShardSpec {
    int ic, oc, K, cb;
};

// ================================================================ gemv1

struct G1World {
    int rows, ic;
    std::vector<ShardSpec> sh;
    std::vector<int> col0;        // first output column of each shard in C
    long ldc;
    size_t slot_bytes;
    std::vector<uint8_t> out;     // writes per (row, column)
    long units_total = 0;
    std::vector<uint8_t> unit_seen;          // per shard-local unit id, offset by shard
    std::vector<long> unit_base;
    // slots: float offset of each row start -> (S, g, r) that wrote it
    std::map<long, std::tuple<int, int, int>> slot_rows;
    // accumulator words: byte offset -> (launch * 1e6 + segment, row, output) it sums, and the
    // adds it has had (each a distinct workgroup)
    std::map<long, std::tuple<long, int, int>> acc_owner;
    std::map<long, std::vector<int>> acc_adds;
    long loads = 0, lds_reads = 0;
};

int shard_index(const G1World& w, const GemvShard* shards, const uint32_t* trellis)
{
    for (size_t i = 0; i < w.sh.size(); i++)
        if (shards[i].trellis == trellis) return (int)i;
    return -1;
}

template <int K, bool ONE, int R>
void g1_replay_wg(G1World& W, const GemvShard* shards, const G1Group& a, const G1Shard* sht, int g, size_t lds,
                  int launch)
{
    const G1Range w = g1_range<ONE>(a, sht, g);
    if (w.L < 1) fail("launch %d wg %d: empty range", launch, g);
    if (w.nseg < 1 || w.nocc < 1) fail("launch %d wg %d: nseg %d nocc %d", launch, g, w.nseg, w.nocc);
    const int nr = R == 1 ? 1 : a.nrows;
    const G1Lds ll = g1_lds_layout(w.nseg, w.nocc, nr);
    if ((size_t)ll.words * 4 > lds)
        fail("launch %d wg %d: LDS layout %d bytes > launch LDS %zu", launch, g, ll.words * 4, lds);
    const int ntr = a.ntr;
    const long ic = (long)ntr * 16;

    auto shard_of = [&](int s) -> int {
        if (s < 0 || s >= a.nshards) fail("launch %d wg %d: shard %d of %d", launch, g, s, a.nshards);
        return shard_index(W, shards, g1_sh<ONE>(sht, s).trellis);
    };
    auto trellis_words = [&](int gi) { return (long)(W.sh[gi].ic / 16) * (W.sh[gi].oc / 16) * 8 * K; };

    // ---- zero operand
    for (int t = 0; t < g1_zero_words(nr); t++)
        if (ll.zero + t >= ll.words) fail("zero word out of LDS");
    if (g1_zero_words(nr) > 64 * G1_NW) fail("more zero words than threads clear them");
    std::vector<char> act_written((size_t)(ll.zero - ll.act), 0);

    // ---- activation table: tag of each occurrence (segment k, block); each (occurrence, row)
    // transformed once
    std::vector<int> occ_k(w.nocc, -1), occ_blk(w.nocc, -1), occ_rows(w.nocc, 0);
    // (the kernel's task cursor, checked against the division form of each task)
    const G1TaskStep tst = g1_task_step(nr);
    if (tst.q * nr + tst.rm != G1_NW || tst.rm < 0 || tst.rm >= nr) fail("task step %d %d for %d rows", tst.q, tst.rm, nr);
    for (int wave = 0; wave < G1_NW; wave++)
        for (G1Task tk = g1_task_first<ONE>(a, sht, w, wave, nr); tk.t < w.nocc * nr;
             g1_task_next<ONE>(a, sht, w, tk, nr, tst)) {
            const int t = tk.t, i = tk.i, r = tk.r;
            if (i != t / nr || r != t % nr) fail("task %d: cursor (%d, %d) for %d rows", t, i, r, nr);
            int k, blk;
            g1_occ_block(a, w, i, k, blk);
            if (tk.k != k || tk.blk != blk)
                fail("task %d: cursor at (segment %d, block %d), occurrence %d is (%d, %d)", t, tk.k, tk.blk, i, k, blk);
            if (tk.s != g1_shard_of_seg<ONE>(a, sht, w.S_first + k)) fail("task %d: cursor shard %d", t, tk.s);
            if (k < 0 || k >= w.nseg) fail("occurrence %d: segment %d of %d", i, k, w.nseg);
            if (blk < 0 || blk >= ntr / 8) fail("occurrence %d: block %d of %d", i, blk, ntr / 8);
            if (occ_k[i] >= 0 && (occ_k[i] != k || occ_blk[i] != blk)) fail("occurrence %d: two blocks", i);
            occ_k[i] = k;
            occ_blk[i] = blk;
            if (occ_rows[i] & (1 << r)) fail("occurrence %d row %d transformed twice", i, r);
            occ_rows[i] |= 1 << r;
            const int s = g1_shard_of_seg<ONE>(a, sht, w.S_first + k);
            const int gi = shard_of(s);
            const G1Shard& e = g1_sh<ONE>(sht, s);
            for (int lane = 0; lane < 64; lane++) {
                need_in(reinterpret_cast<const uint32_t*>(e.suh + blk * 128) + lane, 4, B_SUH + gi,
                        (long)W.sh[gi].ic * 2, "suh load");
                need_in(reinterpret_cast<const uint32_t*>(a.x + g1_x_elem(a, r, blk)) + lane, 4, B_X,
                        (long)W.rows * ic * 2, "activation load");
                if (g1_x_elem(a, r, blk) / ic != r) fail("activation row %d reads row %ld", r, g1_x_elem(a, r, blk) / ic);
                const int aw = g1_act_word(i, lane, nr, r);
                if (aw < 0 || aw + 2 > ll.zero - ll.act) fail("act store outside act (word %d)", aw);
                if (aw % 2) fail("act store at odd word %d (an 8-byte store)", aw);
                if (act_written[aw]++ || act_written[aw + 1]++) fail("act word %d stored twice", aw);
            }
        }
    for (int i = 0; i < w.nocc; i++)
        if (occ_rows[i] != (1 << nr) - 1) fail("occurrence %d: rows %x transformed, %d needed", i, occ_rows[i], nr);

    // ---- per wave: prefetch and processing cursors, LDS reads, flushes
    std::vector<int> red_written((size_t)w.nseg * G1_NW, 0);
    std::vector<int> red_slot((size_t)w.nseg + G1_NW, -1);   // which (segment, wave) holds red[k + ww]
    for (int wave = 0; wave < G1_NW; wave++) {
        const G1Run run = g1_wave_run(w.L, wave);
        const int n = run.n;
        if (n < 0 || run.lo < 0 || run.lo + n > w.L) fail("wave %d run [%d, +%d) of %d", wave, run.lo, n, w.L);
        auto check_load = [&](const G1Cursor& q, const char* what) {
            const int gi = shard_of(q.s);
            const G1Shard& e = g1_sh<ONE>(sht, q.s);
            if (q.cg < 0 || q.cg >= e.ncg || q.tr < 0 || q.tr >= ntr)
                fail("%s: cursor cg %d tr %d (ncg %d, ntr %d)", what, q.cg, q.tr, e.ncg, ntr);
            if (q.p != e.trellis + ((long)q.tr * e.oc16 + 8 * q.cg) * (8 * K))
                fail("%s: cursor pointer does not match its tile row", what);
            for (int lane = 0; lane < 64; lane++)
                need_in(q.p + g1_lane_word(lane, K), 4L * K, B_TRELLIS + gi, trellis_words(gi) * 4, what);
            W.loads++;
        };
        G1Cursor pf = g1_cursor_at<K, ONE>(a, sht, w.ub + run.lo), cu = pf;
        int jpf = 0;
        const int D = g1_depth(R, lds);   // the kernel's ring depth for this launch
        if (D < 1 || D > G1_DEEP) fail("prefetch depth %d", D);
        if (n > 0) {
            check_load(pf, "first trellis load");
            for (int d = 1; d < D; d++) {
                g1_next_pf<K, ONE>(a, sht, pf, jpf, n);
                check_load(pf, "prefetch");
            }
        }
        int cur = cu.S - w.S_first;
        int occ = g1_occ_of(w, cur, cu.tr);
        auto flush = [&](int k) {
            if (cur < 0 || cur >= w.nseg) fail("flush of segment %d of %d", cur, w.nseg);
            for (int lane = 0; lane < 64; lane++) {
                const int yrow = g1_yrow(lane), ycol = g1_ycol(lane);
                if (yrow >= nr) continue;
                const int base = g1_red_row(cur, wave, nr, yrow) + ycol;
                for (int e = 0; e < 4; e++)
                    if (base + 32 * e + 8 >= ll.act || base + 32 * e < 0) fail("flush outside red");
            }
            if (red_written[(size_t)cur * G1_NW + wave]++) fail("wave %d flushes segment %d twice", wave, cur);
            if (red_slot[cur + wave] >= 0) fail("partial rows (%d, %d) and %d share red[%d]", cur, wave, red_slot[cur + wave], cur + wave);
            red_slot[cur + wave] = cur * G1_NW + wave;
            cur = k;
        };
        for (int j = 0; j < n; j += D)
            for (int d = 0; d < D; d++) {
                if (d == 0 || j + d < n) {
                    if (cu.S - w.S_first != cur) flush(cu.S - w.S_first);
                    // the unit this iteration decodes
                    const int gi = shard_of(cu.s);
                    const G1Shard& e = g1_sh<ONE>(sht, cu.s);
                    if (cu.S != e.sbeg + cu.cg) fail("cursor segment %d != shard segment %d", cu.S, e.sbeg + cu.cg);
                    const long uid = W.unit_base[gi] + (long)cu.cg * ntr + cu.tr;
                    if (W.unit_seen[uid]++) fail("unit (shard %d, cg %d, tr %d) decoded twice", gi, cu.cg, cu.tr);
                    // A operand: act entry of (occ, tr) or the zero operand, 64 bytes per lane
                    if (occ < 0 || occ >= w.nocc) fail("occurrence %d of %d", occ, w.nocc);
                    if (occ_k[occ] != cur || occ_blk[occ] != (cu.tr >> 3))
                        fail("unit (seg %d, tr %d) reads occurrence %d = (seg %d, block %d)", cur, cu.tr, occ,
                             occ_k[occ], occ_blk[occ]);
                    const uint32_t ent = g1_a_entry(occ, cu.tr, nr);
                    for (int lane = 0; lane < 64; lane++) {
                        const uint32_t asel = g1_asel(lane), aoff = g1_aoff(lane, nr, ll);
                        const int want_r = std::min((lane & 15) >> 2, nr - 1);
                        for (int c = 0; c < 4; c++) {
                            // chunk c: 16 bytes at the kernel's immediate offset c * g1_a_chunk
                            const uint32_t byte = ent * asel + aoff + c * g1_a_chunk(nr);
                            if (byte % 16) fail("A chunk at byte %u is not 16-byte aligned", byte);
                            if (byte + 16 > 4u * ll.words) fail("A read beyond the LDS layout");
                            if (asel) {
                                // the 4 words the table store of (occurrence, tile row, activation
                                // row, chunk c) wrote: lanes 8 (tr % 8) + c and + 4 of that store
                                const int wa = g1_act_word(occ, 8 * (cu.tr & 7) + c, nr, want_r);
                                const int wb = g1_act_word(occ, 8 * (cu.tr & 7) + c + 4, nr, want_r);
                                if (byte != 4u * (ll.act + wa) || wb != wa + 2)
                                    fail("A chunk %d of lane %d reads byte %u, table word %d", c, lane, byte, ll.act + wa);
                                if (byte + 16 > 4u * ll.zero) fail("A read outside act");
                            } else {
                                const uint32_t z = byte - 4u * ll.zero;
                                if (byte < 4u * ll.zero || z + 16 > 4u * g1_zero_words(nr))
                                    fail("zero-operand lane %d chunk %d reads byte %u, not the cleared words", lane, c, byte);
                            }
                        }
                    }
                    W.lds_reads++;
                    if (j + d + 1 < n) {
                        g1_advance<K, ONE>(a, sht, cu);
                        occ += (cu.tr & 7) == 0;
                    }
                }
                g1_next_pf<K, ONE>(a, sht, pf, jpf, n);
                check_load(pf, "trellis load");
            }
        if (n > 0) flush(cur);
    }

    // ---- tail: per segment, finish here or store the slot
    for (int wave = 0; wave < G1_NW; wave++)
        for (int k = wave; k < w.nseg; k += G1_NW) {
            // the tail sums the rows of the waves whose runs meet segment k: each must have been
            // flushed, and every flushed row of segment k must be among them
            int ub, ue;
            g1_seg_units(w, a.ntr, k, ub, ue);
            for (int ww = 0; ww < G1_NW; ww++) {
                const bool meets = g1_run_meets(g1_wave_run(w.L, ww), ub, ue);
                if (meets != (red_written[(size_t)k * G1_NW + ww] == 1))
                    fail("segment %d: wave %d meets %d but flushed %d times", k, ww, meets, red_written[(size_t)k * G1_NW + ww]);
                if (!meets) continue;
                for (int r = 0; r < nr; r++)
                    if (g1_red_row(k, ww, nr, r) + 128 > ll.act) fail("red read outside red");
            }
            const int S = w.S_first + k;
            int g_lo, g_hi;
            g1_contributors<ONE>(a, sht, S, g_lo, g_hi);
            if (g < g_lo || g > g_hi) fail("wg %d holds segment %d but contributors are %d..%d", g, S, g_lo, g_hi);
            const int s = g1_shard_of_seg<ONE>(a, sht, S);
            const int gi = shard_of(s);
            const G1Shard& e = g1_sh<ONE>(sht, s);
            const int cg = S - e.sbeg;
            if (cg < 0 || cg >= e.ncg) fail("segment %d: column group %d of %d", S, cg, e.ncg);
            if (g_hi > g_lo && a.acc) {
                // the transformed partials are added into the segment's words; the add that
                // completes a word's count (n = g_hi - g_lo + 1 workgroups) stores its output
                const int n = g_hi - g_lo + 1;
                for (int r = 0; r < nr; r++)
                    for (int lane = 0; lane < 64; lane++) {
                        need_in(reinterpret_cast<const uint32_t*>(e.svh + cg * 128) + lane, 4, B_SVH + gi,
                                (long)W.sh[gi].oc * 2, "svh load (accumulate)");
                        for (int j = 0; j < 2; j++) {
                            const unsigned long long* wp = a.acc + g1_acc_word(S, R, r, lane, j);
                            need_in(wp, 8, B_ACC, (long)GEMV_ACC_BYTES, "accumulator add");
                            need_in(wp, 8, B_ACC, off_of(a.acc) + (long)g1_acc_bytes(a.nsegs, R),
                                    "accumulator add (group share)");
                            if (off_of(wp) < off_of(a.acc)) fail("accumulator add before the group's share");
                            const auto key = std::make_tuple((long)launch * 1000000 + S, r, 2 * lane + j);
                            auto ow = W.acc_owner.find(off_of(wp));
                            if (ow == W.acc_owner.end()) W.acc_owner[off_of(wp)] = key;
                            else if (ow->second != key) fail("accumulator word of segment %d row %d output %d shared", S, r, 2 * lane + j);
                            auto& adds = W.acc_adds[off_of(wp)];
                            for (int gg : adds)
                                if (gg == g) fail("wg %d adds twice into segment %d row %d", g, S, r);
                            adds.push_back(g);
                            if ((int)adds.size() > n) fail("segment %d row %d: %zu adds, %d workgroups", S, r, adds.size(), n);
                            if ((int)adds.size() == n) {
                                const uint16_t* o = e.C + r * e.ldc + cg * 128 + 2 * lane + j;
                                need_in(o, 2, B_C, (long)W.rows * W.ldc * 2, "output store (last add)");
                                const long el = off_of(o) / 2;
                                const long col = el % W.ldc, row = el / W.ldc;
                                if (row != r || col < W.col0[gi] || col + 1 > W.col0[gi] + W.sh[gi].oc)
                                    fail("output store at row %ld column %ld outside shard %d", row, col, gi);
                                W.out[el]++;
                            }
                        }
                    }
            } else if (g_hi > g_lo) {
                const float* base = a.slots + g1_slot(S, g, R);
                for (int r = 0; r < nr; r++) {
                    const uint64_t* row = reinterpret_cast<const uint64_t*>(base) + g1_slot_word(0, R, r);
                    need_in(row, 64 * 8, B_SLOTS, (long)W.slot_bytes, "slot store");
                    need_in(row, 64 * 8, B_SLOTS, off_of(a.slots) + (long)(a.G + a.nsegs) * R * 128 * 4,
                            "slot store (group share)");
                    if (off_of(row) < off_of(a.slots)) fail("slot store before the group's share");
                    auto it = W.slot_rows.find(off_of(row));
                    if (it != W.slot_rows.end()) fail("slot row written twice (segment %d, wg %d, row %d)", S, g, r);
                    W.slot_rows[off_of(row)] = std::make_tuple(launch * 1000000 + S, g, r);
                }
            } else {
                for (int r = 0; r < nr; r++)
                    for (int lane = 0; lane < 64; lane++) {
                        need_in(reinterpret_cast<const uint32_t*>(e.svh + cg * 128) + lane, 4, B_SVH + gi,
                                (long)W.sh[gi].oc * 2, "svh load");
                        const uint16_t* o = e.C + r * e.ldc + cg * 128 + 2 * lane;
                        need_in(o, 4, B_C, (long)W.rows * W.ldc * 2, "output store");
                        const long el = off_of(o) / 2;
                        const long col = el % W.ldc, row = el / W.ldc;
                        if (row != r || col < W.col0[gi] || col + 2 > W.col0[gi] + W.sh[gi].oc)
                            fail("output store at row %ld column %ld outside shard %d", row, col, gi);
                        W.out[el]++;
                        W.out[el + 1]++;
                    }
            }
        }
}

template <bool ONE, int R>
void g1_replay_wg_k(int K, G1World& W, const GemvShard* shards, const G1Group& a, const G1Shard* sht, int g,
                    size_t lds, int launch)
{
    switch (K) {
    case 1: g1_replay_wg<1, ONE, R>(W, shards, a, sht, g, lds, launch); break;
    case 2: g1_replay_wg<2, ONE, R>(W, shards, a, sht, g, lds, launch); break;
    case 3: g1_replay_wg<3, ONE, R>(W, shards, a, sht, g, lds, launch); break;
    case 4: g1_replay_wg<4, ONE, R>(W, shards, a, sht, g, lds, launch); break;
    case 5: g1_replay_wg<5, ONE, R>(W, shards, a, sht, g, lds, launch); break;
    case 6: g1_replay_wg<6, ONE, R>(W, shards, a, sht, g, lds, launch); break;
    case 7: g1_replay_wg<7, ONE, R>(W, shards, a, sht, g, lds, launch); break;
    case 8: g1_replay_wg<8, ONE, R>(W, shards, a, sht, g, lds, launch); break;
    default: fail("K=%d", K);
    }
}

void g1_replay_group(G1World& W, const GemvShard* shards, int K, bool one, int R, const G1Group& a,
                     const G1Shard* sht, int g, size_t lds, int launch)
{
    if (one) {
        if (R == 1) g1_replay_wg_k<true, 1>(K, W, shards, a, sht, g, lds, launch);
        else g1_replay_wg_k<true, G1_ROWS>(K, W, shards, a, sht, g, lds, launch);
    } else {
        if (R == 1) g1_replay_wg_k<false, 1>(K, W, shards, a, sht, g, lds, launch);
        else g1_replay_wg_k<false, G1_ROWS>(K, W, shards, a, sht, g, lds, launch);
    }
}

// gemv1_finish_kernel / gemv1_finish_multi_kernel for segment S of group a.
template <bool ONE>
void g1_replay_finish(G1World& W, const GemvShard* shards, int R, const G1Group& a, const G1Shard* sht, int S,
                      int launch)
{
    if (S >= a.nsegs) return;
    const int s = g1_shard_of_seg<ONE>(a, sht, S);
    if (s < 0 || s >= a.nshards) fail("finish: shard %d", s);
    const G1Shard& e = g1_sh<ONE>(sht, s);
    const int gi = shard_index(W, shards, e.trellis);
    const int cg = S - e.sbeg;
    if (cg < 0 || cg >= e.ncg) fail("finish: column group %d of %d", cg, e.ncg);
    int g_lo, g_hi;
    g1_contributors<ONE>(a, sht, S, g_lo, g_hi);
    if (g_hi == g_lo) return;
    if (g_lo < 0 || g_hi >= a.G) fail("finish: contributors %d..%d of %d", g_lo, g_hi, a.G);
    const int nsl = g_hi - g_lo + 1;
    const int nr = R == 1 ? 1 : a.nrows;
    const uint64_t* sl = reinterpret_cast<const uint64_t*>(a.slots + g1_slot(S, g_lo, R));
    constexpr int B = 32;
    for (int r = 0; r < nr; r++) {
        for (int t0 = 0; t0 < nsl; t0 += B)
            for (int t = 0; t < B; t++) {
                const int tt = std::min(t0 + t, nsl - 1);
                const uint64_t* row = sl + g1_slot_word(tt, R, r);
                need_in(row, 64 * 8, B_SLOTS, (long)W.slot_bytes, "slot load");
                auto it = W.slot_rows.find(off_of(row));
                if (it == W.slot_rows.end()) fail("finish reads a slot row nobody wrote (segment %d, wg %d)", S, g_lo + tt);
                if (it->second != std::make_tuple(launch * 1000000 + S, g_lo + tt, r))
                    fail("finish of segment %d reads the slot row of another (segment, wg, row)", S);
            }
        for (int lane = 0; lane < 64; lane++) {
            need_in(reinterpret_cast<const uint32_t*>(e.svh + cg * 128) + lane, 4, B_SVH + gi, (long)W.sh[gi].oc * 2,
                    "svh load (finish)");
            const uint16_t* o = e.C + r * e.ldc + cg * 128 + 2 * lane;
            need_in(o, 4, B_C, (long)W.rows * W.ldc * 2, "output store (finish)");
            const long el = off_of(o) / 2;
            W.out[el]++;
            W.out[el + 1]++;
        }
    }
}

int g1_replay(G1World& W, const GemvShard* shards, int nshards, int cus, long long* stats)
{
    int launch = 0;
    const int rc = g1_plan(fake_ptr<uint16_t>(B_X), shards, nshards, W.rows, fake_ptr<char>(B_SLOTS), W.slot_bytes,
                           fake_ptr<char>(B_ACC), GEMV_ACC_BYTES, cus,
                           [&](const G1Launch& L) {
        if (L.lds > 160 * 1024) fail("launch %d: %zu bytes of LDS per workgroup", launch, L.lds);
        if (L.G < 1 || L.G > G1_GMAX * G1_MAXSH) fail("launch %d: %d workgroups", launch, L.G);
        bool any_split = false;
        // split segments by plain division (independent of the magic-number divisions)
        auto note_split = [&](const G1Group& a) {
            if (a.acc) return;   // split segments finished through the accumulators
            const long big = (long)a.r * (a.q + 1);
            auto wg_of = [&](long u) { return u < big ? u / (a.q + 1) : a.r + (u - big) / a.q; };
            for (int S = 0; S < a.nsegs; S++)
                any_split = any_split || wg_of((long)S * a.ntr + a.ntr - 1) > wg_of((long)S * a.ntr);
        };
        if (!L.multi) {
            const G1Group& a = L.args->grp;
            if (a.G != L.G) fail("launch %d: group G %d != launch G %d", launch, a.G, L.G);
            note_split(a);
            for (int g = 0; g < L.G; g++) g1_replay_group(W, shards, L.K, L.one, L.R, a, L.args->sh, g, L.lds, launch);
            if (L.finish) {
                if (L.fblocks != a.nsegs) fail("finish blocks %d != segments %d", L.fblocks, a.nsegs);
                for (int S = 0; S < L.fblocks; S++) {
                    if (L.one) g1_replay_finish<true>(W, shards, L.R, a, L.args->sh, S, launch);
                    else g1_replay_finish<false>(W, shards, L.R, a, L.args->sh, S, launch);
                }
            }
        } else {
            const G1Multi& m = *L.m;
            for (int t = 0; t < m.ngrp; t++) note_split(m.grp[t]);
            for (int b = 0; b < L.G; b++) {
                const int i = g1_group_of(m.gbeg, m.ngrp, b);
                const int g = b - m.gbeg[i];
                if (g < 0 || g >= m.grp[i].G) fail("multi launch: block %d -> group %d wg %d of %d", b, i, g, m.grp[i].G);
                g1_replay_group(W, shards, m.K[i], false, L.R, m.grp[i], m.sh + m.sh0[i], g, L.lds, launch);
            }
            if (L.finish)
                for (int b = 0; b < L.fblocks; b++) {
                    const int i = g1_group_of(m.fbeg, m.ngrp, b);
                    g1_replay_finish<false>(W, shards, L.R, m.grp[i], m.sh + m.sh0[i], b - m.fbeg[i], launch);
                }
        }
        if (any_split != L.finish) fail("launch %d: finish kernel %d but split segments %d", launch, L.finish, any_split);
        launch++;
        return EXL3_OK;
    });
    if (rc != EXL3_OK) fail("plan refused: %s", g_err);
    for (size_t u = 0; u < W.unit_seen.size(); u++)
        if (W.unit_seen[u] != 1) fail("unit %zu decoded %d times", u, W.unit_seen[u]);
    // an accumulator word that never reached its count would leave its output unwritten: the
    // output check below catches it (and so a word not cleared for the next call)
    for (int r = 0; r < W.rows; r++)
        for (size_t gi = 0; gi < W.sh.size(); gi++)
            for (int c = 0; c < W.sh[gi].oc; c++) {
                const uint8_t n = W.out[(size_t)r * W.ldc + W.col0[gi] + c];
                if (n != 1) fail("output row %d shard %zu column %d written %d times", r, gi, c, n);
            }
    if (stats) {
        stats[0] = launch;
        stats[1] = W.loads;
        stats[2] = W.lds_reads;
        stats[3] = (long long)W.slot_rows.size();
    }
    return 0;
}


// ================================================================ stream-K GEMM

struct SkWorld {
    int rows, ic;
    std::vector<ShardSpec> sh;
    std::vector<int> col0;
    long ldc;
    size_t ws_bytes;
    std::vector<uint8_t> out;
    std::vector<std::pair<long, long>> ws_regions;   // [begin, end) of each workspace use
    std::vector<int> ah_buf;                          // Ah of shard i: B_AH + i (single) or B_WS
    long loads = 0, pieces = 0, slot_writes = 0;
};

void ws_region(SkWorld& W, const void* p, long bytes, const char* what)
{
    need_in(p, bytes, B_WS, (long)W.ws_bytes, what);
    const long b = off_of(p), e = b + bytes;
    for (auto& r : W.ws_regions)
        if (b < r.second && r.first < e) fail("%s: workspace bytes [%ld, %ld) overlap [%ld, %ld)", what, b, e, r.first, r.second);
    W.ws_regions.push_back({b, e});
}

int sk_shard_index(const SkWorld& W, const GemvShard* shards, const uint32_t* trellis)
{
    for (size_t i = 0; i < W.sh.size(); i++)
        if (shards[i].trellis == trellis) return (int)i;
    return -1;
}

// The LDS tiles of a BM-row launch: every A / B element the MFMAs read is one a store wrote,
// and all accesses stay in their buffer's tile (independent of the piece, so checked once).
template <int BM>
void sk_check_lds()
{
    constexpr int MB = SkCfg<BM>::MB, NB = SkCfg<BM>::NB, AP = (BM + 63) / 64;
    const int lds_halves = sk_lds<BM>() / 2;
    for (int b = 0; b < 2; b++) {
        std::vector<uint8_t> aw((size_t)BM * SK_KS, 0), bw((size_t)SK_BN * SK_KS, 0);
        for (int tid = 0; tid < 64 * SK_WAVES; tid++) {
            const int arow = sk_arow(tid), aseg = sk_aseg(tid);
            for (int p = 0; p < AP; p++) {
                if (!sk_apass<BM>(p, arow)) continue;
                const int i = sk_a_store(p, arow, aseg);
                const int row = i / SK_LD, col = i % SK_LD;
                if (row >= BM || col + 8 > SK_KS) fail("A store outside the A tile (BM %d)", BM);
                if (sk_as<BM>(b) + i + 8 > sk_bs<BM>(b)) fail("A store into the B tile");
                for (int e = 0; e < 8; e++) aw[(size_t)row * SK_KS + col + e]++;
            }
            for (int j = 0; j < 4; j++) {
                const int i = sk_b_store(sk_bn0(tid), sk_bk0(tid), j);
                const int row = i / SK_LD, col = i % SK_LD;
                if (row >= SK_BN || col + 8 > SK_KS) fail("B store outside the B tile");
                if (sk_bs<BM>(b) + i + 8 > lds_halves) fail("B store beyond LDS");
                for (int e = 0; e < 8; e++) bw[(size_t)row * SK_KS + col + e]++;
            }
        }
        for (size_t i = 0; i < aw.size(); i++)
            if (aw[i] != 1) fail("A tile element %zu stored %d times (BM %d)", i, aw[i], BM);
        for (size_t i = 0; i < bw.size(); i++)
            if (bw[i] != 1) fail("B tile element %zu stored %d times", i, bw[i]);
        for (int wave = 0; wave < SK_WAVES; wave++) {
            const int wm = wave / SkCfg<BM>::WN, wn = wave % SkCfg<BM>::WN;
            for (int lane = 0; lane < 64; lane++)
                for (int h = 0; h < 2; h++) {
                    for (int nb = 0; nb < NB; nb++) {
                        const int i = sk_b_frag<BM>(wn, nb, lane, h);
                        if (i / SK_LD >= SK_BN || i % SK_LD + 8 > SK_KS) fail("B fragment outside the B tile");
                    }
                    for (int mb = 0; mb < MB; mb++) {
                        const int i = sk_a_frag<BM>(wm, mb, lane, h);
                        if (i / SK_LD >= BM || i % SK_LD + 8 > SK_KS) fail("A fragment outside the A tile (BM %d)", BM);
                    }
                }
        }
    }
    // epilogue staging
    const int lds_floats = sk_lds<BM>() / 4;
    for (int wave = 0; wave < SK_WAVES; wave++) {
        const int wm = wave / SkCfg<BM>::WN, wn = wave % SkCfg<BM>::WN;
        for (int lane = 0; lane < 64; lane++)
            for (int nb = 0; nb < NB; nb++)
                for (int e = 0; e < 4; e++) {
                    int i;
                    if (BM == 256) i = sk_c256(wm, wn >> 1, 4 * (lane >> 4) + e, 64 * (wn & 1) + 16 * nb + (lane & 15));
                    else i = sk_cx(4 * (lane >> 4) + e, NB * 16 * wn + 16 * nb + (lane & 15));
                    if (i < 0 || i >= lds_floats) fail("epilogue staging store beyond LDS (BM %d)", BM);
                }
    }
}

// Whether a BM-row launch of K bits runs the register-B kernel (gemm_sk.hip's sk_fn and
// sk_use_rb: 256-row tiles of one bit width, unless ORCA_EXL3_SK_RB=0).
template <int BM>
bool sk_replay_rb(int K)
{
    const char* e = getenv("ORCA_EXL3_SK_RB");
    return sk_rb<BM>() && K > 0 && !(e && e[0] == '0');
}

// The register-B kernel's LDS: three A buffers filled by direct-to-LDS loads (each logical
// (row, 16-byte chunk) of a K-step's 256 x 64 tile lands once, where the fragment reads look
// for it), the two fragment-exchange buffers (each wave's stores read back by its partner
// only, same fragment and lane), and the epilogue staging with the register-B column map.
void sk_check_lds_rb()
{
    const int lds_bytes = sk_rb_lds();
    const int a_halves = sk_rb_as(SK_RB_NBUF);
    for (int b = 0; b < SK_RB_NBUF; b++) {
        std::vector<int> who((size_t)256 * SK_KS / 8, -1);   // physical chunk -> logical row * 8 + chunk
        for (int wave = 0; wave < SK_WAVES; wave++)
            for (int p = 0; p < 4; p++)
                for (int lane = 0; lane < 64; lane++) {
                    // the DMA writes lane l's 16 bytes at the pass base + 16 l
                    const int h = sk_rb_as(b) + (64 * p + 8 * wave) * SK_KS + 8 * lane;
                    if (h < sk_rb_as(b) || h + 8 > sk_rb_as(b + 1)) fail("A load into LDS outside buffer %d", b);
                    const int r = sk_rb_dma_row(p, wave, lane), c = sk_rb_dma_chunk(p, wave, lane);
                    if (r < 0 || r >= 256 || c < 0 || c >= 8) fail("A load of row %d chunk %d", r, c);
                    if (sk_rb_as(b) + sk_rb_swz(r, c) != h) fail("A row %d chunk %d lands where reads do not look", r, c);
                    int& w = who[(h - sk_rb_as(b)) / 8];
                    if (w >= 0) fail("A buffer %d chunk %d written twice", b, (h - sk_rb_as(b)) / 8);
                    w = r * 8 + c;
                }
        for (size_t i = 0; i < who.size(); i++)
            if (who[i] < 0) fail("A buffer %d chunk %zu never written", b, i);
        for (int wave = 0; wave < SK_WAVES; wave++) {
            const int wm = wave / SkCfg<256>::WN;
            for (int lane = 0; lane < 64; lane++)
                for (int mb = 0; mb < SkCfg<256>::MB; mb++)
                    for (int rh = 0; rh < 2; rh++) {
                        const int h = sk_rb_a_frag(wm, mb, lane, rh);
                        if (h < 0 || h % 8 || h + 8 > 256 * SK_KS) fail("A fragment read outside the tile");
                        const int row = 128 * wm + 16 * mb + (lane & 15), chunk = 2 * (lane >> 4) + rh;
                        if (who[h / 8] != row * 8 + chunk) fail("A fragment (row %d, chunk %d) reads another chunk", row, chunk);
                    }
        }
    }
    // exchange buffers: after the A buffers, inside the launch's LDS
    if (sk_rb_bx_base() * 16 < a_halves * 2) fail("exchange buffers overlap the A buffers");
    std::vector<int> xw((size_t)SK_RB_BBUF * SK_WAVES * 4 * 64, -1);
    for (int b = 0; b < SK_RB_BBUF; b++)
        for (int wave = 0; wave < SK_WAVES; wave++)
            for (int f = 0; f < 4; f++)
                for (int lane = 0; lane < 64; lane++) {
                    const int i = sk_rb_bx(b, wave, f, lane);
                    if (i < 0 || (size_t)i >= xw.size() || (sk_rb_bx_base() + i + 1) * 16 > lds_bytes)
                        fail("fragment store outside the exchange buffers");
                    if (xw[i] >= 0) fail("exchange slot %d stored twice", i);
                    xw[i] = ((b * SK_WAVES + wave) * 4 + f) * 64 + lane;
                }
    for (int b = 0; b < SK_RB_BBUF; b++)
        for (int wave = 0; wave < SK_WAVES; wave++) {
            const int pw = sk_rb_partner(wave);
            if (pw == wave || sk_rb_partner(pw) != wave || pw % SkCfg<256>::WN != wave % SkCfg<256>::WN)
                fail("wave %d: partner %d does not share its outputs", wave, pw);
            for (int f = 0; f < 4; f++)
                for (int lane = 0; lane < 64; lane++)
                    if (xw[sk_rb_bx(b, pw, f, lane)] != ((b * SK_WAVES + pw) * 4 + f) * 64 + lane)
                        fail("wave %d reads another fragment than its partner stored", wave);
        }
    // epilogue staging (register-B column map): per output block and row half, every element
    // of the 16 x 128 staging rows written once by the block's two waves
    const int lds_floats = lds_bytes / 4;
    for (int wm = 0; wm < 2; wm++)
        for (int blk = 0; blk < 2; blk++) {
            std::vector<int> cnt(16 * 128, 0);
            for (int half = 0; half < 2; half++) {
                const int wn = 2 * blk + half;
                for (int lane = 0; lane < 64; lane++)
                    for (int nb = 0; nb < SkCfg<256>::NB; nb++)
                        for (int e = 0; e < 4; e++) {
                            const int row = 4 * (lane >> 4) + e, col = 64 * half + sk_rb_wcol(nb, lane);
                            if (col < 0 || col >= 128) fail("staging column %d", col);
                            const int i = sk_c256(wm, blk, row, col);
                            if (i < 0 || i >= lds_floats) fail("epilogue staging store beyond LDS (register-B)");
                            cnt[row * 128 + col]++;
                        }
            }
            for (int i = 0; i < 16 * 128; i++)
                if (cnt[i] != 1) fail("staging (wm %d, block %d) element %d written %d times", wm, blk, i, cnt[i]);
        }
}

// One BM-row launch (after the clear or set-up kernel): every workgroup's pieces, their loads,
// slot traffic and epilogue stores.
template <int BM>
void sk_replay_launch(SkWorld& W, const GemvShard* shards, const SkLaunch& L, int launch)
{
    constexpr int MB = SkCfg<BM>::MB, NB = SkCfg<BM>::NB, AP = (BM + 63) / 64;
    const SkArgs& a = *L.args;
    const int G = L.G;
    const long units = (long)a.ntiles * a.nks;
    if (G < 1) fail("launch %d: %d workgroups", launch, G);
    if (sk_first(a, G) != units) fail("launch %d: ranges end at %ld, not %ld", launch, sk_first(a, G), units);
    if (a.q < 1) fail("launch %d: %d K-steps per workgroup", launch, a.q);
    const bool rb = sk_replay_rb<BM>(L.K);
    if (rb) sk_check_lds_rb();
    else sk_check_lds<BM>();
    // counters and slots inside the workspace share of this launch
    ws_region(W, a.counters, (long)a.ntiles * 4, "tile counters");
    const long slot_floats = (long)(a.ntiles + G) * SK_WAVES * sk_acc<BM>() * 64;
    ws_region(W, a.slots, slot_floats * 4, "slots");
    if (off_of(a.slots) < off_of(a.counters) + (long)a.ntiles * 4) fail("slots before the counters end");

    std::vector<int> seen_g(G, 0);
    std::vector<int> partial(a.ntiles, 0);
    std::vector<int> tile_done(a.ntiles, 0);
    std::map<std::tuple<int, int>, int> slot_by;   // (tile, g) -> waves written

    auto epilogue = [&](int t) {
        int si = 0;
        for (int i = 1; i < SK_MAXSH; i++)
            if (i < a.nshards && t >= a.sh[i].tbeg) si = i;
        const SkShard& S = a.sh[si];
        const int gi = sk_shard_index(W, shards, S.trellis);
        const int tl = t - S.tbeg, tm = tl / S.ntn, tn = tl - tm * S.ntn, m0 = tm * BM, tc = S.oc >> 4;
        auto store_row = [&](int row, int ob, int lane) {
            if (!(ob < tc && row < a.rows)) return;
            need_in(reinterpret_cast<const uint32_t*>(S.svh + ob * 16) + lane, 4, B_SVH + gi, (long)W.sh[gi].oc * 2,
                    "svh load");
            const uint16_t* o = S.C + (long)row * S.ldc + ob * 16 + 2 * lane;
            need_in(o, 4, B_C, (long)W.rows * W.ldc * 2, "output store");
            const long el = off_of(o) / 2;
            const long col = el % W.ldc;
            if (el / W.ldc != row || col < W.col0[gi] || col + 2 > W.col0[gi] + W.sh[gi].oc)
                fail("output (%d, %ld) outside shard %d", row, col, gi);
            W.out[el]++;
            W.out[el + 1]++;
        };
        for (int wave = 0; wave < SK_WAVES; wave++) {
            const int wm = wave / SkCfg<BM>::WN, wn = wave % SkCfg<BM>::WN;
            for (int lane = 0; lane < 64; lane++) {
                if (BM == 256) {
                    const int blk = wn >> 1, half = wn & 1;
                    for (int mb = 0; mb < MB; mb++)
                        for (int r = 8 * half; r < 8 * half + 8; r++)
                            store_row(m0 + 128 * wm + 16 * mb + r, 16 * tn + 8 * blk, lane);
                } else {
                    for (int mb = 0; mb < MB; mb++)
                        for (int jj = 0; jj < 4; jj++) {
                            const int j = wave + SK_WAVES * jj;
                            store_row(m0 + 16 * mb + (j & 15), 16 * tn + 8 * (j >> 4), lane);
                        }
                }
            }
        }
        tile_done[t]++;
    };

    for (int b = 0; b < G; b++) {
        const int g = sk_logical(b, G);
        if (g < 0 || g >= G || seen_g[g]++) fail("launch %d: slot %d maps to logical workgroup %d twice/outside", launch, b, g);
        const long u_begin = sk_first(a, g), u_end = sk_first(a, g + 1);
        if (u_end - u_begin < 1) fail("launch %d: workgroup %d has no K-steps", launch, g);
        long u = u_begin;
        while (u < u_end) {
            const SkPiece pc = sk_piece<BM>(a, u, u_end);
            if (pc.t < 0 || pc.t >= a.ntiles) fail("piece tile %d of %d", pc.t, a.ntiles);
            if (pc.si < 0 || pc.si >= a.nshards) fail("piece shard %d", pc.si);
            if (!(0 <= pc.s0 && pc.s0 < pc.s1 && pc.s1 <= a.nks)) fail("piece steps %d..%d of %d", pc.s0, pc.s1, a.nks);
            const SkShard& S = a.sh[pc.si];
            const int gi = sk_shard_index(W, shards, S.trellis);
            const int nrb = (a.rows + BM - 1) / BM;
            if (pc.tm >= nrb || pc.tn >= S.ntn || pc.t - S.tbeg >= nrb * S.ntn) fail("piece tile (%d, %d) outside shard", pc.tm, pc.tn);
            const int KK = L.K > 0 ? L.K : S.K;
            if (KK != W.sh[gi].K) fail("piece decodes K=%d, shard has K=%d", KK, W.sh[gi].K);
            const long twords = (long)(W.sh[gi].ic / 16) * (W.sh[gi].oc / 16) * 8 * KK;
            auto load_step_rb = [&](int s) {
                // direct-to-LDS A loads (rows past the call's read the last row) and every lane's
                // chunk words (a column past the shard reads column 0); each chunk of the
                // K-step's tile rows and the piece's 16 tile columns decoded by one lane
                std::vector<uint8_t> dec(4 * 16 * 8, 0);
                for (int wave = 0; wave < SK_WAVES; wave++) {
                    const int wm = wave / SkCfg<256>::WN, wn = wave % SkCfg<256>::WN;
                    for (int lane = 0; lane < 64; lane++) {
                        for (int p = 0; p < 4; p++) {
                            const int row = std::min(pc.m0 + sk_rb_dma_row(p, wave, lane), a.rows - 1);
                            const long el = (long)row * a.ic + (long)s * SK_KS + 8 * sk_rb_dma_chunk(p, wave, lane);
                            need_in(S.Ah + el, 16, W.ah_buf[gi] >= 0 ? W.ah_buf[gi] : B_WS,
                                    W.ah_buf[gi] >= 0 ? (long)a.rows * a.ic * 2 : (long)W.ws_bytes, "A tile load");
                            if (el / a.ic != row || el % a.ic < (long)s * SK_KS || el % a.ic + 8 > (long)(s + 1) * SK_KS)
                                fail("A tile load of row %d K-step %d reads row %ld column %ld", row, s, el / a.ic, el % a.ic);
                        }
                        const int btn = sk_rb_btn(lane, pc.tn, wn, wm);
                        const long wd = sk_b_word(sk_rb_bti(lane, s), pc.tc, sk_bcol(btn, pc.tc), lane & 7, KK);
                        need_in(S.trellis + wd, 4L * KK, B_TRELLIS + gi, twords * 4, "trellis load");
                        const long tile = wd / (8 * KK), ti = tile / pc.tc, tj = tile % pc.tc;
                        if (ti != 4L * s + (lane >> 4) || wd % (8 * KK) != (long)(lane & 7) * KK)
                            fail("trellis load of K-step %d lane %d reads tile row %ld", s, lane, ti);
                        if (btn < pc.tc) {
                            if (tj != btn) fail("trellis load of column %d reads column %ld", btn, tj);
                            if (btn < 16 * pc.tn || btn >= 16 * pc.tn + 16) fail("column %d outside block %d", btn, pc.tn);
                            dec[((lane >> 4) * 16 + (btn - 16 * pc.tn)) * 8 + (lane & 7)]++;
                        } else if (tj != 0) {
                            fail("trellis load past the shard reads column %ld, not 0", tj);
                        }
                    }
                }
                for (int tr = 0; tr < 4; tr++)
                    for (int j = 0; j < 16; j++)
                        for (int c = 0; c < 8; c++) {
                            const int n = dec[(tr * 16 + j) * 8 + c];
                            if (n != (16 * pc.tn + j < pc.tc ? 1 : 0))
                                fail("K-step %d chunk (%d, %d, %d) decoded %d times", s, tr, j, c, n);
                        }
            };
            auto load_step = [&](int s) {
                if (s < pc.s0 || s >= pc.s1) fail("K-step %d loaded outside the piece %d..%d", s, pc.s0, pc.s1);
                if (rb) {
                    load_step_rb(s);
                    W.loads++;
                    return;
                }
                for (int tid = 0; tid < 64 * SK_WAVES; tid++) {
                    const int arow = sk_arow(tid), aseg = sk_aseg(tid);
                    for (int p = 0; p < AP; p++) {
                        const int row = pc.m0 + 64 * p + arow;
                        if (sk_apass<BM>(p, arow) && row < a.rows) {
                            const long el = sk_a_elem(a, row, s, aseg);
                            need_in(S.Ah + el, 16, W.ah_buf[gi] >= 0 ? W.ah_buf[gi] : B_WS,
                                    W.ah_buf[gi] >= 0 ? (long)a.rows * a.ic * 2 : (long)W.ws_bytes, "A tile load");
                            // the 8 halves are row `row`, inside K-step s's 64 columns
                            if (el / a.ic != row || el % a.ic < (long)s * SK_KS || el % a.ic + 8 > (long)(s + 1) * SK_KS)
                                fail("A tile load of row %d K-step %d reads row %ld column %ld", row, s, el / a.ic, el % a.ic);
                        }
                    }
                    const int btn = sk_btn(tid, pc.tn);
                    if (btn < pc.tc) {
                        const long wd = sk_b_word(sk_bti(tid, s), pc.tc, sk_bcol(btn, pc.tc), tid & 7, KK);
                        need_in(S.trellis + wd, 4L * KK, B_TRELLIS + gi, twords * 4, "trellis load");
                        // one chunk of one tile: a tile row of K-step s, a tile column of block tn
                        const long tile = wd / (8 * KK), ti = tile / pc.tc, tj = tile % pc.tc;
                        if (wd % (8 * KK) + KK > 8 * KK || ti < 4L * s || ti >= 4L * s + 4 || tj < 16L * pc.tn ||
                            tj >= 16L * pc.tn + 16)
                            fail("trellis load of K-step %d, column block %d reads tile (%ld, %ld)", s, pc.tn, ti, tj);
                    }
                }
                W.loads++;
            };
            // the kernel's load order
            load_step(pc.s0);
            load_step(std::min(pc.s0 + 1, pc.s1 - 1));
            for (int st = pc.s0; st < pc.s1; st++) load_step(std::min(st + 2, pc.s1 - 1));
            W.pieces++;
            u += pc.s1 - pc.s0;
            if (pc.s0 == 0 && pc.s1 == a.nks) {
                epilogue(pc.t);
                continue;
            }
            const int g_lo = sk_wg_of(a, (long)pc.t * a.nks), g_hi = sk_wg_of(a, (long)(pc.t + 1) * a.nks - 1);
            if (g < g_lo || g > g_hi) fail("workgroup %d holds a piece of tile %d (contributors %d..%d)", g, pc.t, g_lo, g_hi);
            for (int wave = 0; wave < SK_WAVES; wave++)
                for (int i = 0; i < MB * NB * 2; i++) {
                    const uint64_t* wp = reinterpret_cast<const uint64_t*>(a.slots + sk_slot<BM>(pc.t, g, wave)) + (long)i * 64;
                    need_in(wp, 64 * 8, B_WS, off_of(a.slots) + slot_floats * 4, "slot store");
                    if (off_of(wp) < off_of(a.slots)) fail("slot store before the slot area");
                }
            if (slot_by[{pc.t, g}]++) fail("tile %d: workgroup %d stores its slot twice", pc.t, g);
            W.slot_writes++;
            partial[pc.t]++;
        }
    }
    // the last arriver of each split tile: counter reaches g_hi - g_lo, slots g_lo..g_hi read
    for (int t = 0; t < a.ntiles; t++) {
        if (!partial[t]) continue;
        const int g_lo = sk_wg_of(a, (long)t * a.nks), g_hi = sk_wg_of(a, (long)(t + 1) * a.nks - 1);
        if (partial[t] != g_hi - g_lo + 1) fail("tile %d: %d partial pieces, %d contributors", t, partial[t], g_hi - g_lo + 1);
        for (int gg = g_lo; gg <= g_hi; gg++) {
            if (!slot_by.count({t, gg})) fail("tile %d: slot of workgroup %d read but never written", t, gg);
            // slots of distinct (tile, workgroup) pairs must not overlap: index t + gg is unique
            // per pair only if no other tile's contributor shares it
            for (int wave = 0; wave < SK_WAVES; wave++)
                need_in(a.slots + sk_slot<BM>(t, gg, wave), (long)sk_acc<BM>() * 64 * 4, B_WS,
                        off_of(a.slots) + slot_floats * 4, "slot load");
        }
        epilogue(t);
    }
    // distinct slot indices t + g across all written pairs
    std::map<long, int> by_index;
    for (auto& kv : slot_by)
        if (by_index[std::get<0>(kv.first) + std::get<1>(kv.first)]++) fail("two (tile, workgroup) pairs share slot %d", std::get<0>(kv.first) + std::get<1>(kv.first));
    for (int t = 0; t < a.ntiles; t++)
        if (tile_done[t] != 1) fail("tile %d finished %d times", t, tile_done[t]);
}

void sk_replay_prep(SkWorld& W, const GemvShard* shards, const SkLaunch& L)
{
    const SkPrepArgs& p = *L.prep_args;
    const long waves = 4 * ((L.prep_waves + 3) / 4);
    for (int s = 0; s < p.nsh; s++) {
        ws_region(W, p.Ah[s], (long)p.rows * p.ic * 2, "Ah");
        if (p.Ah[s] != L.args->sh[s].Ah) fail("set-up and launch disagree on shard %d's Ah", s);
    }
    for (long w = 0; w < waves; w++) {
        if (w < p.ntiles) need_in(p.counters + w, 4, B_WS, (long)W.ws_bytes, "counter clear");
        if (w >= (long)p.nsh * p.rows * p.nblk) continue;
        int s, r, b;
        sk_prep_wave(p, (int)w, s, r, b);
        if (s < 0 || s >= p.nsh || r >= p.rows || b >= p.nblk) fail("set-up wave %ld -> (%d, %d, %d)", w, s, r, b);
        const int gi = sk_shard_index(W, shards, L.args->sh[s].trellis);
        const long off = sk_prep_elem(p, r, b);
        for (int lane = 0; lane < 64; lane++) {
            need_in(reinterpret_cast<const uint32_t*>(p.A + off) + lane, 4, B_X, (long)W.rows * W.ic * 2, "A load (set-up)");
            need_in(reinterpret_cast<const uint32_t*>(p.suh[s] + b * 128) + lane, 4, B_SUH + gi, (long)W.ic * 2, "suh load");
            need_in(reinterpret_cast<const uint32_t*>(p.Ah[s] + off) + lane, 4, B_WS, (long)W.ws_bytes, "Ah store");
            if (off_of(p.Ah[s] + off) + 4L * (lane + 1) > off_of(p.Ah[s]) + (long)p.rows * p.ic * 2) fail("Ah store past the shard's Ah");
        }
    }
    if ((long)p.ntiles > waves) fail("set-up grid clears %ld of %d counters", waves, p.ntiles);
}

void sk_replay_any(SkWorld& W, const GemvShard* shards, const SkLaunch& L, int launch)
{
    if (L.prep) sk_replay_prep(W, shards, L);
    switch (L.BM) {
    case 32: sk_replay_launch<32>(W, shards, L, launch); break;
    case 48: sk_replay_launch<48>(W, shards, L, launch); break;
    case 64: sk_replay_launch<64>(W, shards, L, launch); break;
    case 96: sk_replay_launch<96>(W, shards, L, launch); break;
    case 128: sk_replay_launch<128>(W, shards, L, launch); break;
    case 256: sk_replay_launch<256>(W, shards, L, launch); break;
    default: fail("tile height %d", L.BM);
    }
    if (L.K == 0 && L.BM == 256) fail("per-shard-K launch of 256-row tiles");
}


// ================================================================ gemv16 (5..16 rows)

struct G16World {
    int rows, ic;
    std::vector<ShardSpec> sh;
    std::vector<int> col0;
    long ldc;
    size_t ws_bytes;
    std::vector<uint8_t> out;
    std::vector<long> unit_base;
    std::vector<uint8_t> unit_seen;
    std::vector<std::vector<uint8_t>> ah_written;   // per shard, per fragment word
    std::vector<long> ah_off;                       // workspace byte offset of each shard's fragments
    std::map<long, std::tuple<int, int, int>> slots;   // float offset -> (launch, strip, workgroup)
    std::map<long, int> slot_reads;
    long loads = 0;
};

int g16_shard_index(const G16World& W, const GemvShard* shards, const uint32_t* trellis)
{
    for (size_t i = 0; i < W.sh.size(); i++)
        if (shards[i].trellis == trellis) return (int)i;
    return -1;
}

void g16_replay_prep(G16World& W, const G16Prep& p)
{
    const long words = g16_ah_words(p.ic);
    for (long g = 0; g < (long)p.nsh * p.nblk; g++) {
        int s, b;
        g16_prep_wg(p, (int)g, s, b);
        if (s < 0 || s >= p.nsh || b < 0 || b >= p.nblk) fail("set-up workgroup %ld -> (%d, %d)", g, s, b);
        if (buf_of(p.ah[s]) != B_WS || off_of(p.ah[s]) != W.ah_off[s]) fail("fragments of shard %d misplaced", s);
        if (W.ah_off[s] % 16) fail("fragments of shard %d not 16-byte aligned", s);
        if (W.ah_off[s] + words * 4 > (long)W.ws_bytes) fail("fragments of shard %d beyond the workspace", s);
        for (int t = 0; t < G16_PREP_LANES; t++) {
            const int wv = t >> 6, lane = t & 63;
            for (int j = 0; j < 4; j++)   // rows wv + 4 j below rows are loaded
                if (wv + 4 * j < p.rows)
                    need_in(reinterpret_cast<const uint32_t*>(p.A + (long)(wv + 4 * j) * p.ic + b * 128) + lane, 4, B_X,
                            (long)W.rows * W.ic * 2, "A load (set-up)");
            need_in(reinterpret_cast<const uint32_t*>(p.suh[s] + b * 128) + lane, 4, B_SUH + s, (long)W.ic * 2, "suh load (set-up)");
            // the lane's 16-byte store: words 4 t .. 4 t + 3 of the block's area, each the two
            // inputs g16_prep_src names, at the word where the decode's reads look for them
            const long w0 = g16_prep_base(b) + 4 * t;
            if (w0 < 0 || w0 + 4 > words) fail("fragment store at word %ld of %ld", w0, words);
            for (int e = 0; e < 4; e++) {
                int i, k;
                g16_prep_src(4 * t + e, i, k);
                if (i < 0 || i >= 16 || k < 0 || k + 1 >= 128 || (k & 1)) fail("set-up word %d -> row %d input %d", 4 * t + e, i, k);
                const long el = g16_ah_elem(i, b * 128 + k);
                if (el != 2 * (w0 + e) || g16_ah_elem(i, b * 128 + k + 1) != el + 1)
                    fail("set-up word %ld holds row %d inputs %d, %d, which the reads look for at half %ld", w0 + e, i,
                         b * 128 + k, b * 128 + k + 1, el);
                if (W.ah_written[s][w0 + e]) fail("fragment word %ld of shard %d written twice", w0 + e, s);
                W.ah_written[s][w0 + e] = 1;
            }
        }
    }
}

template <int K, bool ONE>
void g16_replay_wg(G16World& W, const GemvShard* shards, const G1Group& a, const G16Shard* sht, int g, size_t lds,
                   int launch)
{
    const G1Range w = g16_range<ONE>(a, sht, g);
    if (w.L < 1 || w.nseg < 1) fail("gemv16 wg %d: L %d nseg %d", g, w.L, w.nseg);
    const int red_floats = g16_red_bytes(w.nseg) / 4;
    if ((size_t)red_floats * 4 > lds) fail("gemv16 wg %d: %d bytes of partial rows > launch LDS %zu", g, red_floats * 4, lds);
    const int nq = a.ntr;
    auto shard_of = [&](int s) {
        if (s < 0 || s >= a.nshards) fail("gemv16: shard %d of %d", s, a.nshards);
        return g16_shard_index(W, shards, g16_sh<ONE>(sht, s).trellis);
    };
    std::vector<int> flushed((size_t)w.nseg * G1_NW, 0), red_slot((size_t)w.nseg + G1_NW, -1);
    for (int wave = 0; wave < G1_NW; wave++) {
        const G1Run run = g1_wave_run(w.L, wave);
        const int n = run.n;
        G16Cursor pf = g16_cursor_at<K, ONE>(a, sht, w.ub + run.lo), cu = pf;
        int jpf = 0;
        auto check_load = [&](const G16Cursor& c) {
            const int gi = shard_of(c.s);
            const G16Shard& e = g16_sh<ONE>(sht, c.s);
            if (c.strip < 0 || c.strip >= e.nstrip || c.q < 0 || c.q >= nq) fail("gemv16 cursor strip %d q %d", c.strip, c.q);
            const long tw = (long)(W.sh[gi].ic / 16) * (W.sh[gi].oc / 16) * 8 * K;
            for (int lane = 0; lane < 64; lane++) {
                const uint32_t* p = c.p + g16_lane_word(lane, e.oc16, K);
                need_in(p, 4L * K, B_TRELLIS + gi, tw * 4, "gemv16 trellis load");
                const long wd = off_of(p) / 4, tile = wd / (8 * K), ti = tile / e.oc16, tj = tile % e.oc16;
                if (ti != 4 * c.q + (lane >> 4) || tj != 2 * c.strip + ((lane & 15) >> 3) || (wd % (8 * K)) != (lane & 7) * K)
                    fail("gemv16 lane %d loads tile (%ld, %ld) word %ld", lane, ti, tj, wd % (8 * K));
                // a live row's lane reads its own row; a dead row's lane the last live row
                const int lane_a = g16_ah_lane(lane, a.nrows);
                if ((lane_a >> 4) != (lane >> 4)) fail("gemv16 lane %d reads k-group of lane %d", lane, lane_a);
                if ((lane & 15) < a.nrows ? lane_a != lane : (lane_a & 15) != a.nrows - 1)
                    fail("gemv16 lane %d reads the fragment of lane %d at %d rows", lane, lane_a, a.nrows);
                for (int m = 0; m < 4; m++) {
                    const uint32_t* ap = c.ah + g16_ah_word(m, lane_a);
                    need_in(ap, 8, B_WS, W.ah_off[gi] + g16_ah_words(W.ic) * 4, "gemv16 fragment load");
                    if (off_of(ap) & 7) fail("gemv16 fragment load not 8-byte aligned");
                    const long rel = (off_of(ap) - W.ah_off[gi]) / 4;
                    if (rel < 0) fail("gemv16 fragment load before the shard's fragments");
                    // the two words' four halves are row i's inputs 64 q + 16 j + 2 m + {0, 1, 8, 9}
                    const int i = lane_a & 15, j = lane >> 4;
                    const int o[4] = {0, 1, 8, 9};
                    for (int t = 0; t < 4; t++) {
                        if (g16_ah_elem(i, 64 * c.q + 16 * j + 2 * m + o[t]) != 2 * rel + t) fail("gemv16 fragment half of the wrong input");
                        if (!W.ah_written[gi][rel + t / 2]) fail("gemv16 reads a fragment word the set-up did not write");
                    }
                }
            }
            W.loads++;
        };
        if (n > 0) check_load(pf);
        int cur = cu.S - w.S_first;
        auto flush = [&](int k) {
            if (cur < 0 || cur >= w.nseg) fail("gemv16 flush of strip %d of %d", cur, w.nseg);
            for (int lane = 0; lane < 64; lane++)
                for (int h = 0; h < 2; h++)
                    for (int t = 0; t < 4; t++) {
                        const int i = g16_red_row(cur, wave) + g16_acc_index(lane, h, t);
                        if (i < 0 || i >= red_floats) fail("gemv16 flush outside red");
                    }
            if (flushed[(size_t)cur * G1_NW + wave]++) fail("gemv16 wave %d flushes strip %d twice", wave, cur);
            if (red_slot[cur + wave] >= 0) fail("gemv16 partial rows share red[%d]", cur + wave);
            red_slot[cur + wave] = cur;
            cur = k;
        };
        for (int j = 0; j < n; j++) {
            if (cu.S - w.S_first != cur) flush(cu.S - w.S_first);
            const int gi = shard_of(cu.s);
            const G16Shard& e = g16_sh<ONE>(sht, cu.s);
            if (cu.S != e.sbeg + cu.strip) fail("gemv16 cursor strip bookkeeping");
            const long uid = W.unit_base[gi] + (long)cu.strip * nq + cu.q;
            if (W.unit_seen[uid]++) fail("gemv16 unit (shard %d, strip %d, q %d) twice", gi, cu.strip, cu.q);
            if (j + 1 < n) g16_advance<K, ONE>(a, sht, cu);
            g16_next_pf<K, ONE>(a, sht, pf, jpf, n);
            check_load(pf);
        }
        if (n > 0) flush(cur);
    }
    // tail: per strip into this workgroup's slot
    for (int k = 0; k < w.nseg; k++) {
        int ub, ue;
        g1_seg_units(w, nq, k, ub, ue);
        for (int ww = 0; ww < G1_NW; ww++) {
            const bool meets = g1_run_meets(g1_wave_run(w.L, ww), ub, ue);
            if (meets != (flushed[(size_t)k * G1_NW + ww] == 1)) fail("gemv16 strip %d wave %d meets %d flushed %d", k, ww, meets, flushed[(size_t)k * G1_NW + ww]);
            if (meets && g16_red_row(k, ww) + 512 > red_floats) fail("gemv16 red read outside red");
        }
        int g_lo, g_hi;
        g16_contributors<ONE>(a, sht, w.S_first + k, g_lo, g_hi);
        if (g < g_lo || g > g_hi) fail("gemv16 wg %d holds strip %d, contributors %d..%d", g, w.S_first + k, g_lo, g_hi);
        const float* sl = a.slots + g16_slot(w.S_first + k, g);
        need_in(sl, 16 * 32 * 4, B_WS, (long)W.ws_bytes, "gemv16 slot store");
        need_in(sl, 16 * 32 * 4, B_WS, off_of(a.slots) + (long)(a.G + a.nsegs) * 16 * 32 * 4, "gemv16 slot store (group share)");
        if (W.slots.count(off_of(sl))) fail("gemv16 slot of strip %d wg %d written twice", w.S_first + k, g);
        W.slots[off_of(sl)] = std::make_tuple(launch, w.S_first + k, g);
    }
}

template <bool ONE>
void g16_replay_wg_k(int K, G16World& W, const GemvShard* shards, const G1Group& a, const G16Shard* sht, int g,
                     size_t lds, int launch)
{
    switch (K) {
    case 1: g16_replay_wg<1, ONE>(W, shards, a, sht, g, lds, launch); break;
    case 2: g16_replay_wg<2, ONE>(W, shards, a, sht, g, lds, launch); break;
    case 3: g16_replay_wg<3, ONE>(W, shards, a, sht, g, lds, launch); break;
    case 4: g16_replay_wg<4, ONE>(W, shards, a, sht, g, lds, launch); break;
    case 5: g16_replay_wg<5, ONE>(W, shards, a, sht, g, lds, launch); break;
    case 6: g16_replay_wg<6, ONE>(W, shards, a, sht, g, lds, launch); break;
    case 7: g16_replay_wg<7, ONE>(W, shards, a, sht, g, lds, launch); break;
    case 8: g16_replay_wg<8, ONE>(W, shards, a, sht, g, lds, launch); break;
    default: fail("K=%d", K);
    }
}

template <bool ONE>
void g16_replay_finish(G16World& W, const GemvShard* shards, const G1Group& a, const G16Shard* sht, int cg4, int launch)
{
    if (cg4 * 4 >= a.nsegs) return;
    const int s = g16_shard_of_seg<ONE>(a, sht, 4 * cg4);
    const G16Shard& e = g16_sh<ONE>(sht, s);
    const int gi = g16_shard_index(W, shards, e.trellis);
    const int cg = cg4 - e.sbeg / 4;
    if (e.sbeg % 4 || cg < 0 || cg * 4 >= e.nstrip) fail("gemv16 finish: column group %d", cg);
    for (int lane = 0; lane < 64; lane++) {
        const int S = 4 * cg4 + (lane >> 4);
        if (g16_shard_of_seg<ONE>(a, sht, S) != s) fail("gemv16 finish: strips of one block in two shards");
        int g_lo, g_hi;
        g16_contributors<ONE>(a, sht, S, g_lo, g_hi);
        const int col = (2 * lane) & 31;
        for (int r = 0; r < a.nrows; r++) {
            for (int gg = g_lo; gg <= g_hi; gg++) {
                const float* p = a.slots + g16_slot(S, gg) + r * G16_STRIP + col;
                need_in(p, 8, B_WS, (long)W.ws_bytes, "gemv16 slot load");
                const long base = off_of(a.slots + g16_slot(S, gg));
                auto it = W.slots.find(base);
                if (it == W.slots.end() || it->second != std::make_tuple(launch, S, gg)) fail("gemv16 finish reads a slot not written for (strip %d, wg %d)", S, gg);
                W.slot_reads[base]++;
            }
            need_in(reinterpret_cast<const uint32_t*>(e.svh + cg * 128) + lane, 4, B_SVH + gi, (long)W.sh[gi].oc * 2, "gemv16 svh load");
            const uint16_t* o = e.C + r * e.ldc + cg * 128 + 2 * lane;
            need_in(o, 4, B_C, (long)W.rows * W.ldc * 2, "gemv16 output store");
            const long el = off_of(o) / 2;
            const long c = el % W.ldc;
            if (el / W.ldc != r || c < W.col0[gi] || c + 2 > W.col0[gi] + W.sh[gi].oc) fail("gemv16 output outside shard");
            W.out[el]++;
            W.out[el + 1]++;
        }
    }
}

}  // namespace

extern "C" {

// Message of the last failed replay ("" after a clean one).
const char* exl3r_message() { return g_msg.c_str(); }

// The 1..4-row GEMV (exl3_gemv with rows <= 4 on the gemv1 path) of nshards shards that share
// ic, on a device with `cus` CUs.  concat != 0: the shards write adjacent column ranges of one
// (rows, sum oc) output, as the grouped op does; else each its own (rows, oc) output (checked
// as one buffer with a column offset per shard, ldc = sum oc).  Returns 0 when every access is
// in bounds and every coverage check holds, 1 on a violation, 2 if the plan refused the call
// (exl3r_message says which).  stats (4 entries, may be null): launches, wave-unit loads
// checked, unit LDS reads checked, slot rows written.
int exl3r_gemv1(int rows, int ic, int nshards, const int* oc, const int* K, const int* cb, int cus, long long* stats)
{
    g_msg.clear();
    try {
        if (nshards < 1 || nshards > EXL3_MAX_SHARDS) fail("nshards %d", nshards);
        G1World W;
        W.rows = rows;
        W.ic = ic;
        std::vector<GemvShard> shards(nshards);
        long cols = 0;
        W.slot_bytes = 0;
        for (int i = 0; i < nshards; i++) {
            W.sh.push_back(ShardSpec{ic, oc[i], K[i], cb[i]});
            W.col0.push_back((int)cols);
            cols += oc[i];
            W.slot_bytes += (g1_slot_bytes(oc[i], rows) + 255) & ~(size_t)255;
        }
        W.ldc = cols;
        W.out.assign((size_t)rows * cols + 2, 0);
        long ub = 0;
        for (int i = 0; i < nshards; i++) {
            GemvShard& d = shards[i];
            d.trellis = fake_ptr<uint32_t>(B_TRELLIS + i);
            d.suh = fake_ptr<uint16_t>(B_SUH + i);
            d.svh = fake_ptr<uint16_t>(B_SVH + i);
            d.C = fake_ptr<uint16_t>(B_C) + W.col0[i];
            d.ic = ic;
            d.oc = oc[i];
            d.K = K[i];
            d.cb = cb[i];
            d.ldc = W.ldc;
            W.unit_base.push_back(ub);
            ub += (long)(oc[i] / 128) * (ic / 16);
        }
        W.unit_seen.assign(ub, 0);
        return g1_replay(W, shards.data(), nshards, cus, stats);
    } catch (const Fail& f) {
        g_msg = f.what;
        return g_msg.rfind("plan refused", 0) == 0 ? 2 : 1;
    }
}


// The stream-K GEMM for nshards shards sharing ic: mode 0 = exl3_gemm (one shard; up to
// SK_PREP_MAX_ROWS rows it is the one-shard grouped plan, as gemm_dispatch runs it), 1 =
// exl3_gemm_grouped; tile height by rows.  Workspaces are sized as the product sizes them for
// `cus` CUs.  Returns as exl3r_gemv1; stats: launches, K-step loads checked, pieces, slot
// stores.
int exl3r_gemm_sk(int mode, int rows, int ic, int nshards, const int* oc, const int* K, const int* cb, int cus,
                  long long* stats)
{
    g_msg.clear();
    try {
        if (nshards < 1 || nshards > EXL3_MAX_SHARDS || (mode == 0 && nshards != 1) || mode < 0 || mode > 1)
            fail("mode %d, nshards %d", mode, nshards);
        if (mode == 0 && rows <= SK_PREP_MAX_ROWS) {
            // exl3_gemm's workspace (its Hadamard output, then counters and slots) is exactly
            // the one-shard grouped launch's
            if (gemm_sk_ah_bytes(rows, ic) + sk_single_bytes(rows, oc[0], cus) !=
                sk_grouped_bytes_bm(gemm_sk_bm(rows), rows, ic, oc[0], cus))
                fail("exl3_gemm workspace %zu != one-shard grouped workspace %zu",
                     gemm_sk_ah_bytes(rows, ic) + sk_single_bytes(rows, oc[0], cus),
                     sk_grouped_bytes_bm(gemm_sk_bm(rows), rows, ic, oc[0], cus));
            mode = 1;
        }
        SkWorld W;
        W.rows = rows;
        W.ic = ic;
        std::vector<GemvShard> shards(nshards);
        long cols = 0;
        size_t ws = 0;
        const int bm = gemm_sk_bm(rows);
        for (int i = 0; i < nshards; i++) {
            W.sh.push_back(ShardSpec{ic, oc[i], K[i], cb[i]});
            W.col0.push_back((int)cols);
            W.ah_buf.push_back(mode == 0 ? B_AH + i : -1);
            cols += oc[i];
            if (mode == 0) ws += sk_single_bytes(rows, oc[i], cus);
            else ws += sk_grouped_bytes_bm(bm, rows, ic, oc[i], cus);
        }
        W.ldc = cols;
        W.ws_bytes = ws;
        W.out.assign((size_t)rows * cols + 2, 0);
        for (int i = 0; i < nshards; i++) {
            GemvShard& d = shards[i];
            d.trellis = fake_ptr<uint32_t>(B_TRELLIS + i);
            d.suh = fake_ptr<uint16_t>(B_SUH + i);
            d.svh = fake_ptr<uint16_t>(B_SVH + i);
            d.C = fake_ptr<uint16_t>(B_C) + W.col0[i];
            d.ic = ic;
            d.oc = oc[i];
            d.K = K[i];
            d.cb = cb[i];
            d.ldc = W.ldc;
        }
        int launch = 0;
        auto emit = [&](const SkLaunch& L) {
            sk_replay_any(W, shards.data(), L, launch++);
            return EXL3_OK;
        };
        int rc;
        if (mode == 0) {
            // above SK_PREP_MAX_ROWS exl3_gemm's Hadamard pass zeroes the launch's counters
            // instead of a clear kernel: sk_ntiles words at the start of its workspace
            auto emit_single = [&](const SkLaunch& L) {
                if (reinterpret_cast<const char*>(L.args->counters) != fake_ptr<char>(B_WS) ||
                    L.args->ntiles != sk_ntiles(rows, oc[0]))
                    fail("tile counters (%d) are not the %d words the Hadamard pass clears", L.args->ntiles,
                         sk_ntiles(rows, oc[0]));
                return emit(L);
            };
            rc = sk_plan_single(fake_ptr<uint16_t>(B_AH), shards[0].trellis, shards[0].C, shards[0].svh, fake_ptr<char>(B_WS),
                                ws, rows, ic, oc[0], K[0], cb[0], cus, emit_single);
        } else {
            const char* what = "exl3_gemm_grouped";
            switch (bm) {
            case 32: rc = sk_plan_grouped<32>(fake_ptr<uint16_t>(B_X), shards.data(), nshards, rows, fake_ptr<char>(B_WS), ws, what, cus, emit); break;
            case 48: rc = sk_plan_grouped<48>(fake_ptr<uint16_t>(B_X), shards.data(), nshards, rows, fake_ptr<char>(B_WS), ws, what, cus, emit); break;
            case 64: rc = sk_plan_grouped<64>(fake_ptr<uint16_t>(B_X), shards.data(), nshards, rows, fake_ptr<char>(B_WS), ws, what, cus, emit); break;
            case 96: rc = sk_plan_grouped<96>(fake_ptr<uint16_t>(B_X), shards.data(), nshards, rows, fake_ptr<char>(B_WS), ws, what, cus, emit); break;
            case 128: rc = sk_plan_grouped<128>(fake_ptr<uint16_t>(B_X), shards.data(), nshards, rows, fake_ptr<char>(B_WS), ws, what, cus, emit); break;
            default: rc = sk_plan_grouped<256>(fake_ptr<uint16_t>(B_X), shards.data(), nshards, rows, fake_ptr<char>(B_WS), ws, what, cus, emit); break;
            }
        }
        if (rc != EXL3_OK) fail("plan refused: %s", exl3::g_err);
        for (int r = 0; r < rows; r++)
            for (int i = 0; i < nshards; i++)
                for (int c = 0; c < oc[i]; c++) {
                    const uint8_t n = W.out[(size_t)r * W.ldc + W.col0[i] + c];
                    if (n != 1) fail("output row %d shard %d column %d written %d times", r, i, c, n);
                }
        if (stats) {
            stats[0] = launch;
            stats[1] = W.loads;
            stats[2] = W.pieces;
            stats[3] = W.slot_writes;
        }
        return 0;
    } catch (const Fail& f) {
        g_msg = f.what;
        return g_msg.rfind("plan refused", 0) == 0 ? 2 : 1;
    }
}


// The 5..16-row GEMV (exl3_gemv with 5..16 rows): the set-up kernel, each decode launch and its
// finish launch, as exl3r_gemv1.  stats: launches, unit loads checked, 0, slots written.
int exl3r_gemv16(int rows, int ic, int nshards, const int* oc, const int* K, const int* cb, int cus, long long* stats)
{
    g_msg.clear();
    try {
        if (nshards < 1 || nshards > EXL3_MAX_SHARDS) fail("nshards %d", nshards);
        G16World W;
        W.rows = rows;
        W.ic = ic;
        std::vector<GemvShard> shards(nshards);
        long cols = 0, ub = 0;
        size_t ws = 0;
        for (int i = 0; i < nshards; i++) {
            W.sh.push_back(ShardSpec{ic, oc[i], K[i], cb[i]});
            W.col0.push_back((int)cols);
            cols += oc[i];
            ws += (g16_shard_bytes(ic, oc[i]) + 255) & ~(size_t)255;
            W.unit_base.push_back(ub);
            ub += (long)(oc[i] / G16_STRIP) * (ic / G16_QIN);
            W.ah_written.emplace_back(g16_ah_words(ic), 0);
            W.ah_off.push_back((long)i * (((size_t)g16_ah_words(ic) * 4 + 255) & ~(size_t)255));
        }
        W.ldc = cols;
        W.ws_bytes = ws;
        W.out.assign((size_t)rows * cols + 2, 0);
        W.unit_seen.assign(ub, 0);
        for (int i = 0; i < nshards; i++) {
            GemvShard& d = shards[i];
            d.trellis = fake_ptr<uint32_t>(B_TRELLIS + i);
            d.suh = fake_ptr<uint16_t>(B_SUH + i);
            d.svh = fake_ptr<uint16_t>(B_SVH + i);
            d.C = fake_ptr<uint16_t>(B_C) + W.col0[i];
            d.ic = ic;
            d.oc = oc[i];
            d.K = K[i];
            d.cb = cb[i];
            d.ldc = W.ldc;
        }
        int launch = 0;
        bool prepped = false;
        G16Prep prep;
        const int rc = g16_plan(fake_ptr<uint16_t>(B_X), shards.data(), nshards, rows, fake_ptr<char>(B_WS), ws, cus, prep,
                                [&](const G16Launch& L) {
            if (!prepped) {
                g16_replay_prep(W, prep);
                prepped = true;
            }
            if (L.lds > G1_LDS_PER_CU) fail("gemv16 launch %d: %zu bytes of LDS", launch, L.lds);
            if (!L.multi) {
                const G1Group& a = L.args->grp;
                std::vector<char> wg_seen(L.G, 0);
                for (int blk = 0; blk < L.G; blk++) {   // the kernel's block -> workgroup order
                    const int g = g16_block_wg(blk, L.G, L.K);
                    if (g < 0 || g >= L.G || wg_seen[g]++)
                        fail("gemv16 launch %d: block %d -> workgroup %d of %d", launch, blk, g, L.G);
                    if (L.one) g16_replay_wg_k<true>(L.K, W, shards.data(), a, L.args->sh, g, L.lds, launch);
                    else g16_replay_wg_k<false>(L.K, W, shards.data(), a, L.args->sh, g, L.lds, launch);
                }
                if (L.fblocks * 4 != a.nsegs) fail("gemv16 finish blocks %d for %d strips", L.fblocks, a.nsegs);
                for (int b = 0; b < L.fblocks; b++) {
                    if (L.one) g16_replay_finish<true>(W, shards.data(), a, L.args->sh, b, launch);
                    else g16_replay_finish<false>(W, shards.data(), a, L.args->sh, b, launch);
                }
            } else {
                const G16Multi& m = *L.m;
                for (int b = 0; b < L.G; b++) {
                    const int i = g1_group_of(m.gbeg, m.ngrp, b);
                    const int g = b - m.gbeg[i];
                    if (g < 0 || g >= m.grp[i].G) fail("gemv16 multi: block %d -> group %d wg %d", b, i, g);
                    g16_replay_wg_k<false>(m.K[i], W, shards.data(), m.grp[i], m.sh + m.sh0[i], g, L.lds, launch);
                }
                for (int b = 0; b < L.fblocks; b++) {
                    const int i = g1_group_of(m.fbeg, m.ngrp, b);
                    g16_replay_finish<false>(W, shards.data(), m.grp[i], m.sh + m.sh0[i], b - m.fbeg[i], launch);
                }
            }
            launch++;
            return EXL3_OK;
        });
        if (rc != EXL3_OK) fail("plan refused: %s", exl3::g_err);
        for (size_t u = 0; u < W.unit_seen.size(); u++)
            if (W.unit_seen[u] != 1) fail("gemv16 unit %zu decoded %d times", u, W.unit_seen[u]);
        for (auto& kv : W.slots)
            if (W.slot_reads[kv.first] < 1) fail("gemv16 slot of strip %d wg %d never read", std::get<1>(kv.second), std::get<2>(kv.second));
        for (int r = 0; r < rows; r++)
            for (int i = 0; i < nshards; i++)
                for (int c = 0; c < oc[i]; c++) {
                    const uint8_t n = W.out[(size_t)r * W.ldc + W.col0[i] + c];
                    if (n != 1) fail("gemv16 output row %d shard %d column %d written %d times", r, i, c, n);
                }
        if (stats) {
            stats[0] = launch;
            stats[1] = W.loads;
            stats[2] = 0;
            stats[3] = (long long)W.slots.size();
        }
        return 0;
    } catch (const Fail& f) {
        g_msg = f.what;
        return g_msg.rfind("plan refused", 0) == 0 ? 2 : 1;
    }
}

}  // extern "C"
