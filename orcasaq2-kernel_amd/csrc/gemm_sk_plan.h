// Work plan of the stream-K GEMM (gemm_sk.hip): tile shapes and LDS sizes, the launch
// argument blocks, the split of a launch's K-steps into workgroup ranges, the tile pieces of a
// range, every global and LDS index the kernels form, the workspace layout, and the host-side
// grouping of shards into launches.
//
// Everything here is plain integer arithmetic marked __host__ __device__ (or host-only
// planning): the kernels call these functions, and the CPU address replay
// (replay/addr_replay.hip) calls the very same ones to walk every workgroup, wave and lane of
// a launch and check each index against the buffer it addresses.
#pragma once

#include <algorithm>

#include "exl3_launch.h"

namespace exl3 {

#define SK_HD __host__ __device__ __forceinline__

constexpr int SK_WAVES = 8;
constexpr int SK_BN = 256;
constexpr int SK_KS = 64;                     // inputs per K-step (4 tile rows)
constexpr int SK_LD = SK_KS + 8;              // halves per LDS row of the A and B tiles
constexpr int SK_CLD = 128 + 4;               // floats per epilogue row in LDS (BM = 256)
constexpr int SK_MAXSH = 8;                   // shards per launch
constexpr int SK_WPE = 2;                     // waves per SIMD the register budget is set for (one workgroup per CU)

// Wave grid of a BM x 256 tile: WM x WN waves, each MB x NB blocks of 16 x 16.
template <int BM>
struct SkCfg;
template <>
struct SkCfg<256> { static constexpr int WM = 2, WN = 4, MB = 8, NB = 4; };
template <>
struct SkCfg<128> { static constexpr int WM = 1, WN = 8, MB = 8, NB = 2; };
template <>
struct SkCfg<64> { static constexpr int WM = 1, WN = 8, MB = 4, NB = 2; };
template <>
struct SkCfg<96> { static constexpr int WM = 1, WN = 8, MB = 6, NB = 2; };
template <>
struct SkCfg<48> { static constexpr int WM = 1, WN = 8, MB = 3, NB = 2; };
template <>
struct SkCfg<32> { static constexpr int WM = 1, WN = 8, MB = 2, NB = 2; };

template <int BM>
constexpr int sk_acc() { return SkCfg<BM>::MB * SkCfg<BM>::NB * 4; }   // fp32 accumulators per lane
// LDS of a launch: the A and B tiles of one K-step, twice (the tiles of step s + 1 are written
// while the MFMAs read those of step s), one workgroup per CU.  Measured on MI355X at 17..64
// rows: the two-buffer pipeline with one workgroup per CU beats one buffer with two
// workgroups per CU by 28% on 17408 -> 5120 and 6% on 5120 -> 17408.
template <int BM>
constexpr int sk_buf() { return (BM + SK_BN) * SK_LD; }                   // halves per A + B buffer
template <int BM>
constexpr int sk_lds() { return 2 * sk_buf<BM>() * 2; }      // bytes

struct SkShard {
    const uint16_t* Ah;        // (rows, ic) fp16, fp16(H(A * suh)) of this shard
    const uint32_t* trellis;   // (ic/16, oc/16, 8K) u32
    const uint16_t* svh;       // (oc)
    uint16_t* C;               // (rows, ldc) fp16, columns [0, oc)
    long ldc;
    int oc, ntn, tbeg;         // outputs, 256-wide tile columns, first tile of the shard
    int K;                     // bits per weight (read by the per-shard-K kernel)
};

struct SkArgs {
    uint32_t* counters;        // one per tile, zeroed before the launch
    float* slots;              // (tiles + G) x SK_WAVES x acc x 64 fp32
    int rows, ic, nks, ntiles, nshards;
    int q, r;                  // K-steps per workgroup: q + (g < r)
    SkShard sh[SK_MAXSH];
};

// Set-up of a grouped launch in one kernel: the tile counters to zero and, for every
// shard, its activations Ah = fp16(H128(A * suh)) (rows x ic), one wave per (shard, row,
// 128-input block).
struct SkPrepArgs {
    const uint16_t* A;
    int rows, ic, nsh, nblk;
    const uint16_t* suh[SK_MAXSH];
    uint16_t* Ah[SK_MAXSH];
    uint32_t* counters;
    int ntiles;
};

// Shard s, row r and 128-input block b of set-up wave w (w < nsh * rows * nblk).
SK_HD void sk_prep_wave(const SkPrepArgs& a, int w, int& s, int& r, int& b)
{
    b = w % a.nblk;
    const int rs = w / a.nblk;
    r = rs % a.rows;
    s = rs / a.rows;
}

// Element offset of row r, 128-input block b in A and Ah (row-major, ic per row).
SK_HD long sk_prep_elem(const SkPrepArgs& a, int r, int b)
{
    return (long)r * a.ic + b * 128;
}

// Logical workgroup of launch slot b of G.  Launch slots go to the 8 XCDs round-robin (slot b
// on XCD b % 8), so when G is a multiple of 8 each XCD gets a contiguous block of logical
// workgroups -- for a 256-row GEMM, the tiles of one row block: their A rows are shared in
// that XCD's L2.  Any placement gives the same results; this one only saves traffic.
SK_HD int sk_logical(int b, int G)
{
    return (G & 7) ? b : (b & 7) * (G >> 3) + (b >> 3);
}

// First K-step (global numbering) of workgroup g, and the workgroup holding K-step u.
SK_HD long sk_first(const SkArgs& a, int g) { return (long)g * a.q + (g < a.r ? g : a.r); }
SK_HD int sk_wg_of(const SkArgs& a, long u)
{
    const long big = (long)a.r * (a.q + 1);
    return u < big ? (int)(u / (a.q + 1)) : a.r + (int)((u - big) / a.q);
}

// The tile piece that starts at K-step u of a range ending at u_end: tile t, its K-steps
// s0 .. s1 - 1, shard si, tile row block tm / column block tn, first row m0, tile columns tc
// of the shard's W_q.
struct SkPiece {
    int t, s0, s1, si, tm, tn, m0, tc;
};

template <int BM>
SK_HD SkPiece sk_piece(const SkArgs& a, long u, long u_end)
{
    SkPiece p;
    p.t = (int)(u / a.nks);
    p.s0 = (int)(u - (long)p.t * a.nks);
    const long left = p.s0 + (u_end - u);
    p.s1 = (int)(a.nks < left ? a.nks : left);
    p.si = 0;
#pragma unroll
    for (int i = 1; i < SK_MAXSH; i++)
        if (i < a.nshards && p.t >= a.sh[i].tbeg) p.si = i;
    const SkShard& S = a.sh[p.si];
    const int tl = p.t - S.tbeg;
    p.tm = tl / S.ntn;
    p.tn = tl - p.tm * S.ntn;
    p.m0 = p.tm * BM;
    p.tc = S.oc >> 4;
    return p;
}

// ---------------------------------------------------------------- per-thread indices

// A-tile loader: thread tid moves 16 bytes of row tid / 8 (+ 64 p), segment tid % 8; pass p
// moves rows 64 p + arow < BM.
SK_HD int sk_arow(int tid) { return tid >> 3; }
SK_HD int sk_aseg(int tid) { return tid & 7; }
template <int BM>
SK_HD bool sk_apass(int p, int arow) { return 64 * p + arow < BM; }
// Element offset in Ah of the 8 halves thread (arow, aseg) loads for pass p of K-step s.
SK_HD long sk_a_elem(const SkArgs& a, int row, int s, int aseg)
{
    return (long)row * a.ic + s * SK_KS + aseg * 8;
}

// B chunk of thread tid: chunk id tid = 8 * tile + c, tile = 16 ti_l + tn_l (a tile's 8 chunks
// on 8 consecutive lanes); output column bn0 (and bn0 + 8) and input row bk0 of the K-step's
// 64 x 256 B tile.
SK_HD int sk_btile(int tid) { return tid >> 3; }
SK_HD int sk_bn0(int tid) { return 16 * (sk_btile(tid) & 15) + (tid & 7); }
SK_HD int sk_bk0(int tid) { return 16 * (sk_btile(tid) >> 4); }
// Tile column of W_q this thread's chunk lies in for tile column block tn; a chunk beyond the
// shard's tc tile columns is not loaded (its address is taken at column 0).
SK_HD int sk_btn(int tid, int tn) { return 16 * tn + (sk_btile(tid) & 15); }
SK_HD int sk_bcol(int btn, int tc) { return btn < tc ? btn : 0; }
// Tile row of the chunk in K-step s.
SK_HD int sk_bti(int tid, int s) { return 4 * s + (sk_btile(tid) >> 4); }
// First u32 of the chunk's K words in the trellis: tile (ti, bcol), chunk c = tid % 8.
SK_HD long sk_b_word(int ti, int tc, int bcol, int c, int K)
{
    return ((long)ti * tc + bcol) * (8 * K) + c * K;
}

// LDS (halves): buffer b's A tile at b * sk_buf, its B tile BM rows of SK_LD later.
template <int BM>
SK_HD int sk_as(int b) { return b * sk_buf<BM>(); }
template <int BM>
SK_HD int sk_bs(int b) { return b * sk_buf<BM>() + BM * SK_LD; }
// A store of pass p / B stores (relative to the tile).
SK_HD int sk_a_store(int p, int arow, int aseg) { return (64 * p + arow) * SK_LD + aseg * 8; }
SK_HD int sk_b_store(int bn0, int bk0, int j) { return (bn0 + 8 * (j >> 1)) * SK_LD + bk0 + 8 * (j & 1); }
// MFMA fragment reads (16 bytes = 8 halves each), relative to the tile.
template <int BM>
SK_HD int sk_b_frag(int wn, int nb, int lane, int h)
{
    return (SkCfg<BM>::NB * 16 * wn + 16 * nb + (lane & 15)) * SK_LD + 32 * h + 8 * (lane >> 4);
}
template <int BM>
SK_HD int sk_a_frag(int wm, int mb, int lane, int h)
{
    return (SkCfg<BM>::MB * 16 * wm + 16 * mb + (lane & 15)) * SK_LD + 32 * h + 8 * (lane >> 4);
}

// ---------------------------------------------------------------- 256-row tiles: B in registers
//
// The 256-row form (gemm_rb_kernel) keeps only A in LDS (below).
// Each wave (wm, wn) owns rows 128 wm .. and outputs 64 wn .. of the tile: two chunk groups g
// of 32 outputs (two tile columns).  Per K-step lane l of the wave decodes one chunk of group
// g = wm -- chunk l % 8 of tile (4 s + l / 16, 16 tn + 4 wn + 2 g + (l % 16) / 8) -- and
// receives lane l's chunk of group 1 - wm from wave (1 - wm, wn); a chunk's four 8-row
// fragments (column half ch, row half rh) are the B operands of four
// v_mfma_f32_16x16x32_f16: the MFMA's k-group j = l / 16 is tile row 4 s + j, rows 8 rh ..
// 8 rh + 7, and its column n = l % 16 is output 16 (n / 8) + 8 ch + n % 8 of the group.  The
// A operand of row block mb and half rh: row 16 mb + l % 16 of the wave's 128, inputs
// 16 (l / 16) + 8 rh .. + 7 of the K-step.  Accumulator block nb = 2 g + ch.
template <int BM>
constexpr bool sk_rb() { return BM == 256; }
SK_HD int sk_rb_bti(int lane, int s) { return 4 * s + (lane >> 4); }
SK_HD int sk_rb_btn(int lane, int tn, int wn, int g) { return 16 * tn + 4 * wn + 2 * g + ((lane & 15) >> 3); }
// A tiles: SK_RB_NBUF buffers of 256 rows x 64 halves, unpadded; a row's eight 16-byte chunks
// are stored XOR-swizzled (logical chunk c of row r at chunk c ^ ((r / 2) % 8)).  A row is
// half of a 256-byte bank line, so the 16 rows of an MFMA fragment read (one logical chunk
// each) fall on 16 distinct 16-byte bank groups -- rows of equal parity are told apart by
// (r / 2) % 8 -- while each wave's 16-byte direct-to-LDS loads fill 8 whole rows (1 KiB) in
// lane order.
constexpr int SK_RB_NBUF = 3;
SK_HD int sk_rb_as(int b) { return b * 256 * SK_KS; }
SK_HD int sk_rb_chunk_swz(int r) { return (r >> 1) & 7; }
SK_HD int sk_rb_swz(int r, int c) { return r * SK_KS + 8 * (c ^ sk_rb_chunk_swz(r)); }
SK_HD int sk_rb_a_frag(int wm, int mb, int lane, int rh)
{
    return sk_rb_swz(128 * wm + 16 * mb + (lane & 15), 2 * (lane >> 4) + rh);
}
// Direct load of pass p (0..3) by wave wv: LDS rows 64 p + 8 wv .. + 7 in lane order; lane l
// fills chunk l % 8 of row 64 p + 8 wv + l / 8, i.e. logical chunk (l % 8) ^ ((row / 2) % 8).
SK_HD int sk_rb_dma_row(int p, int wv, int lane) { return 64 * p + 8 * wv + (lane >> 3); }
SK_HD int sk_rb_dma_chunk(int p, int wv, int lane) { return (lane & 7) ^ sk_rb_chunk_swz(sk_rb_dma_row(p, wv, lane)); }
// Output (0..63 within the wave's 64) of accumulator block nb, lane's column.
SK_HD int sk_rb_wcol(int nb, int lane)
{
    return 32 * (nb >> 1) + 16 * ((lane & 15) >> 3) + 8 * (nb & 1) + (lane & 7);
}
// B fragment exchange: two buffers (K-step parity) after the A buffers, each 8 waves x 4
// fragments x 64 lanes of 16 bytes; a wave stores its own chunk group's fragments in lane
// order and reads its partner's (conflict-free 16-byte accesses).  Partner of (wm, wn): (1 - wm, wn).
constexpr int SK_RB_BBUF = 2;
SK_HD int sk_rb_partner(int wave) { return wave ^ 4; }
SK_HD int sk_rb_bx_base() { return SK_RB_NBUF * 256 * SK_KS * 2 / 16; }   // in 16-byte units
SK_HD int sk_rb_bx(int b, int wave, int f, int lane) { return ((b * SK_WAVES + wave) * 4 + f) * 64 + lane; }
constexpr int sk_rb_lds() { return SK_RB_NBUF * 256 * SK_KS * 2 + SK_RB_BBUF * SK_WAVES * 4 * 64 * 16; }   // bytes

// Slot of (tile t, workgroup g, wave): float offset of its acc x 64 partials; the lane's
// 8-byte word i of it is u64 i * 64 + lane.
template <int BM>
SK_HD long sk_slot(int t, int g, int wave)
{
    return ((long)(t + g) * SK_WAVES + wave) * sk_acc<BM>() * 64;
}

// Epilogue LDS rows (floats): BM = 256, rows of SK_CLD per (wm, block); others, 16 rows of
// SK_BN + 4.
SK_HD int sk_c256(int wm, int blk, int row, int col) { return (wm * 2 + blk) * 16 * SK_CLD + row * SK_CLD + col; }
SK_HD int sk_cx(int row, int col) { return row * (SK_BN + 4) + col; }

// ---------------------------------------------------------------- host: workspace and planning

inline size_t sk_align(size_t x) { return (x + 255) & ~(size_t)255; }

// exl3_gemm's Hadamard output fp16(H(A * suh)) at the head of its workspace.
inline size_t gemm_sk_ah_bytes(int rows, int ic) { return sk_align((size_t)rows * ic * 2); }

// Workgroups per launch: one per CU, all resident at once.
template <int BM>
inline int sk_gmax(int cus) { return cus; }

template <int BM>
inline size_t sk_slot_bytes() { return (size_t)SK_WAVES * sk_acc<BM>() * 64 * sizeof(float); }

inline int sk_ntn(int oc) { return (oc + SK_BN - 1) / SK_BN; }

// Counters and slots of one launch of `tiles` tiles and up to G workgroups.
template <int BM>
inline size_t sk_ws(long tiles, int G) { return sk_align((size_t)tiles * 4) + (size_t)(tiles + G) * sk_slot_bytes<BM>(); }

// exl3_gemm up to this many rows runs as the one-shard grouped launch (its set-up kernel does
// the Hadamard pass and the counter clear in one launch); above, a Hadamard pass of its own
// that also clears the counters, then the stream-K kernel.  The workspace layout is the same.
constexpr int SK_PREP_MAX_ROWS = 384;

// Tile height of a prefill launch of `rows` rows.  Each weight is decoded once per row tile;
// a taller tile pays that decode over more rows but MFMA work for padding rows and bigger
// partial sums.  Measured on MI355X (17408 -> 5120, 5120 -> 17408, 5120 -> 6144): 32 is
// fastest up to 32 rows (13-22% below 64-row tiles), 48 up to 48 (8-15% below), 64 up to
// 64, 96 up to 96 (4-9% below 128-row tiles), 128 up to 384 (two or
// three 128-row tiles beat one 256-row tile: more tiles, fewer stream-K partial sums per
// tile), 256 above.
inline int gemm_sk_bm(int rows)
{
    return rows <= 32 ? 32 : rows <= 48 ? 48 : rows <= 64 ? 64 : rows <= 96 ? 96 : rows <= 384 ? 128 : 256;
}

template <int BM>
inline size_t gemm_sk_ws(int rows, int oc, int cus)
{
    return sk_ws<BM>((long)((rows + BM - 1) / BM) * sk_ntn(oc), sk_gmax<BM>(cus));
}

// Counters and slots of a single-shard prefill launch.
inline size_t sk_single_bytes(int rows, int oc, int cus)
{
    switch (gemm_sk_bm(rows)) {
    case 32: return gemm_sk_ws<32>(rows, oc, cus);
    case 48: return gemm_sk_ws<48>(rows, oc, cus);
    case 96: return gemm_sk_ws<96>(rows, oc, cus);
    case 64: return gemm_sk_ws<64>(rows, oc, cus);
    case 128: return gemm_sk_ws<128>(rows, oc, cus);
    default: return gemm_sk_ws<256>(rows, oc, cus);
    }
}

// Per-shard workspace of a grouped launch (several shards reading the same A): the shard's
// activations fp16(H(A * suh)), then its share of counters and slots (each launch has at
// least one shard, so the shares cover it).
template <int BM>
inline size_t sk_grouped_bytes(int rows, int ic, int oc, int cus)
{
    return sk_align((size_t)rows * ic * 2) + sk_ws<BM>((long)((rows + BM - 1) / BM) * sk_ntn(oc), sk_gmax<BM>(cus));
}

inline size_t sk_grouped_bytes_bm(int bm, int rows, int ic, int oc, int cus)
{
    switch (bm) {
    case 32: return sk_grouped_bytes<32>(rows, ic, oc, cus);
    case 48: return sk_grouped_bytes<48>(rows, ic, oc, cus);
    case 96: return sk_grouped_bytes<96>(rows, ic, oc, cus);
    case 64: return sk_grouped_bytes<64>(rows, ic, oc, cus);
    case 128: return sk_grouped_bytes<128>(rows, ic, oc, cus);
    default: return sk_grouped_bytes<256>(rows, ic, oc, cus);
    }
}

// The per-piece-K kernel (K = 0) exists for BM <= 128; a mixed-K group of 256-row tiles
// is launched once per K instead.
template <int BM>
constexpr bool sk_has_k0() { return BM <= 128; }

// One stream-K launch of the plan.
struct SkLaunch {
    int BM, K, cb, G;            // K = 0: each tile piece takes its shard's K
    bool prep;                   // the set-up kernel (prep) runs first
    long prep_waves;
    const SkArgs* args;
    const SkPrepArgs* prep_args;
};

// Workgroup count and workspace placement of a launch over a.sh[0 .. nshards) (tiles and
// K-steps set): at least 8 K-steps per workgroup (a tile then has at most nks / 8 + 2
// contributors), at most gmax, and no more than the slots `ws` holds.
template <int BM>
inline int sk_place(SkArgs& a, int gmax, char* ws, size_t ws_bytes, const char* what, int& G)
{
    const long units = (long)a.ntiles * a.nks;
    G = (int)std::min<long>(gmax, std::max<long>(1, units / 8));
    const size_t cbytes = sk_align((size_t)a.ntiles * 4);
    const long fit = ws_bytes > cbytes ? (long)((ws_bytes - cbytes) / sk_slot_bytes<BM>()) - a.ntiles : 0;
    if (fit < 1)
        return set_error(EXL3_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", what, ws_bytes,
                         sk_ws<BM>(a.ntiles, G));
    if (G > fit) G = (int)fit;   // a workspace sized on a device with fewer CUs
    a.q = (int)(units / G);
    a.r = (int)(units % G);
    a.counters = reinterpret_cast<uint32_t*>(ws);
    a.slots = reinterpret_cast<float*>(ws + cbytes);
    return EXL3_OK;
}

// Tiles of exl3_gemm's single-shard launch: its tile counters are the first this many
// 32-bit words of the launch's workspace.
inline int sk_ntiles(int rows, int oc)
{
    const int bm = gemm_sk_bm(rows);
    return ((rows + bm - 1) / bm) * sk_ntn(oc);
}

// exl3_gemm's stream-K launch over one shard (Ah already transformed; its tile counters
// cleared by the same Hadamard pass).
template <class Emit>
int sk_plan_single(const uint16_t* Ah, const uint32_t* trellis, uint16_t* C, const uint16_t* svh, char* ws,
                   size_t ws_bytes, int rows, int ic, int oc, int K, int cb, int cus, Emit&& emit)
{
    SkArgs a = {};
    a.rows = rows;
    a.ic = ic;
    a.nks = ic / SK_KS;
    a.nshards = 1;
    SkShard& s = a.sh[0];
    s.Ah = Ah;
    s.trellis = trellis;
    s.svh = svh;
    s.C = C;
    s.ldc = oc;
    s.oc = oc;
    s.ntn = sk_ntn(oc);
    s.tbeg = 0;
    s.K = K;
    const int bm = gemm_sk_bm(rows);
    a.ntiles = sk_ntiles(rows, oc);
    SkLaunch L = {};
    L.BM = bm;
    L.K = K;
    L.cb = cb;
    L.args = &a;
    const char* what = "exl3_gemm (stream-K)";
    int rc;
    switch (bm) {
    case 32: rc = sk_place<32>(a, sk_gmax<32>(cus), ws, ws_bytes, what, L.G); break;
    case 48: rc = sk_place<48>(a, sk_gmax<48>(cus), ws, ws_bytes, what, L.G); break;
    case 96: rc = sk_place<96>(a, sk_gmax<96>(cus), ws, ws_bytes, what, L.G); break;
    case 64: rc = sk_place<64>(a, sk_gmax<64>(cus), ws, ws_bytes, what, L.G); break;
    case 128: rc = sk_place<128>(a, sk_gmax<128>(cus), ws, ws_bytes, what, L.G); break;
    default: rc = sk_place<256>(a, sk_gmax<256>(cus), ws, ws_bytes, what, L.G); break;
    }
    if (rc != EXL3_OK) return rc;
    return emit(static_cast<const SkLaunch&>(L));
}

// Shards that read the same A (rows x ic): per codebook (and per K where no per-piece-K
// kernel exists), groups of up to SK_MAXSH shards; per group one set-up kernel (the
// shards' activations, the group's tile counters) and one stream-K launch -- a single-K
// kernel when the group's shards share K, else the per-shard-K one.
template <int BM, class Emit>
int sk_plan_grouped(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* ws, size_t ws_bytes,
                    const char* what, int cus, Emit&& emit)
{
    const int ic = shards[0].ic;
    const int nrb = (rows + BM - 1) / BM;
    bool done[EXL3_MAX_SHARDS] = {false};
    size_t off = 0;
    const size_t ah = sk_align((size_t)rows * ic * 2);
    for (int i = 0; i < nshards; i++) {
        if (done[i]) continue;
        SkArgs a = {};
        SkPrepArgs p = {};
        a.rows = p.rows = rows;
        a.ic = p.ic = ic;
        a.nks = ic / SK_KS;
        p.A = A;
        p.nblk = ic / 128;
        int tiles = 0, K = shards[i].K;
        for (int s = i; s < nshards && a.nshards < SK_MAXSH; s++) {
            if (done[s] || shards[s].cb != shards[i].cb) continue;
            if (!sk_has_k0<BM>() && shards[s].K != shards[i].K) continue;
            const GemvShard& d = shards[s];
            if (d.K < 1 || d.K > 8) return set_error(EXL3_ERR_ARG, "%s: K=%d is not in 1..8", what, d.K);
            if (off + ah > ws_bytes)
                return set_error(EXL3_ERR_WORKSPACE, "%s: workspace of %zu bytes is too small", what, ws_bytes);
            uint16_t* Ah = reinterpret_cast<uint16_t*>(ws + off);
            off += ah;
            p.suh[a.nshards] = d.suh;
            p.Ah[a.nshards] = Ah;
            SkShard& e = a.sh[a.nshards++];
            e.Ah = Ah;
            e.trellis = d.trellis;
            e.svh = d.svh;
            e.C = d.C;
            e.ldc = d.ldc;
            e.oc = d.oc;
            e.ntn = sk_ntn(d.oc);
            e.tbeg = tiles;
            e.K = d.K;
            if (d.K != K) K = 0;
            tiles += nrb * e.ntn;
            done[s] = true;
        }
        a.ntiles = p.ntiles = tiles;
        p.nsh = a.nshards;
        p.counters = reinterpret_cast<uint32_t*>(ws + off);
        SkLaunch L = {};
        L.BM = BM;
        L.K = K;
        L.cb = shards[i].cb;
        L.prep = true;
        L.prep_waves = std::max<long>((long)p.nsh * rows * p.nblk, tiles);
        L.args = &a;
        L.prep_args = &p;
        const size_t need = sk_ws<BM>(tiles, sk_gmax<BM>(cus));
        const size_t avail = ws_bytes > off ? ws_bytes - off : 0;
        int rc = sk_place<BM>(a, sk_gmax<BM>(cus), ws + off, std::min(need, avail), what, L.G);
        if (rc != EXL3_OK) return rc;
        rc = emit(static_cast<const SkLaunch&>(L));
        if (rc != EXL3_OK) return rc;
        off += std::min(need, avail);
    }
    return EXL3_OK;
}

}  // namespace exl3
