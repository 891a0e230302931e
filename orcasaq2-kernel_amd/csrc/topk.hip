// Top-k of each row of an fp16 matrix: the argmax / top-k epilogue of the output head.
// The lm_head (an ordinary EXL3 linear, reference orcasaq2/config.py:128-132) writes
// (rows, vocab) fp16 logits; greedy decoding takes each row's argmax and top-k sampling its
// k largest.  The reference leaves both to vLLM's sampler; here they run as two kernels on
// the GEMV's stream, reading the logits once.
//
// Order: by value, largest first; equal values by smaller column.  Every NaN ranks above
// +inf (as torch.max and torch.argmax propagate NaN), -0 equals +0.  An fp16 value maps to
// a 16-bit order key (tk_key); among equal keys the smaller column wins.
//
// Both kernels run one selection (tk_select) over keys held 16 a lane in column order
// (lane t holds positions 16t .. 16t + 15): bisection over the 16 key bits for the k-th
// largest key T (16 steps, each one ballot count per key and one barrier), then the keys
// > T and the first (k - #{> T}) keys == T in column order, marked and numbered in column
// order by two block scans.
//   1. topk_chunk_kernel, one 256-lane workgroup per 4096-column chunk of a row: the
//      chunk's k selected go to its k candidate slots in column order (a chunk with fewer
//      than k columns leaves its last slots 0, below every real candidate).
//   2. topk_merge_kernel, one workgroup per row (256 lanes for up to 4096 candidates, else
//      512): the same selection over the row's
//      candidates (chunk-major, so in column order), then the k selected ranked by (key,
//      column) into the outputs.
// A workgroup's waves share one CU and its scalar unit, which executes each wave's ballot
// counts: four and eight waves keep a step at a few hundred cycles.  k = 1 (argmax) skips
// the bisection: both kernels take the maximum of key << 19 | (2^19 - 1 - column) by a
// wave and a workgroup reduction.  Bounds: k <= 64 and n <= 2^19 columns (128 chunks, 8192
// candidates: 16 a lane in the merge).
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

constexpr int TK_PER = 16;                          // keys per lane
constexpr int TK_T1 = 256;                          // stage-1 lanes
constexpr int TK_CHUNK = TK_T1 * TK_PER;            // columns per stage-1 workgroup
constexpr int TK_T2 = 512;                          // merge lanes
constexpr int TK_IDX_BITS = 19;
static_assert(TK_MAX_N == 1 << TK_IDX_BITS, "column field of a candidate");
static_assert(TK_T2 * TK_PER >= TK_MAX_K * (TK_MAX_N / TK_CHUNK), "the merge holds every candidate");

// Order key of fp16 bits h: larger for larger values; -0 and +0 alike, every NaN 0xffff
// (above +inf = 0xfc00); -inf = 0x03ff, so 0 is below every value.
__device__ __forceinline__ uint32_t tk_key(uint32_t h)
{
    const uint32_t m = h & 0x7fffu;
    const uint32_t k = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
    return m > 0x7c00u ? 0xffffu : (m == 0 ? 0x8000u : k);
}

// Candidate word: key in bits 35..50, column in 16..34, the value's fp16 bits in 0..15.
__device__ __forceinline__ uint64_t tk_cand(uint32_t key, int col, uint32_t h)
{
    return ((uint64_t)key << (16 + TK_IDX_BITS)) | ((uint64_t)(uint32_t)col << 16) | h;
}
__device__ __forceinline__ uint32_t tk_cand_key(uint64_t c) { return (uint32_t)(c >> (16 + TK_IDX_BITS)); }
__device__ __forceinline__ int tk_cand_col(uint64_t c) { return (int)((c >> 16) & ((1u << TK_IDX_BITS) - 1u)); }

// Argmax order of a candidate: larger key first, then smaller column (an empty slot, key 0,
// is below every real candidate).
__device__ __forceinline__ uint64_t tk_ord(uint64_t c)
{
    return ((uint64_t)tk_cand_key(c) << TK_IDX_BITS) | (uint64_t)((1u << TK_IDX_BITS) - 1u - (uint32_t)tk_cand_col(c));
}

// The candidate of largest order in the workgroup (every lane gets it).
template <int NW>
__device__ __forceinline__ uint64_t tk_block_argmax(uint64_t c, uint64_t* buf)
{
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)c, d, 64), hi = __shfl_xor((uint32_t)(c >> 32), d, 64);
        const uint64_t o = ((uint64_t)hi << 32) | lo;
        if (tk_ord(o) > tk_ord(c)) c = o;
    }
    if ((threadIdx.x & 63) == 0) buf[threadIdx.x >> 6] = c;
    __syncthreads();
    uint64_t b = buf[0];
#pragma unroll
    for (int w = 1; w < NW; w++)
        if (tk_ord(buf[w]) > tk_ord(b)) b = buf[w];
    return b;
}

struct TkLds {
    int sums[2][TK_T2 / 64];
    uint32_t scan[2][TK_T2 / 64];
    uint64_t best[TK_T2 / 64];
};

// Workgroup sum of a wave-uniform count.  The buffers alternate between calls, so one
// barrier per call orders the writes before the reads (a buffer is written again two calls
// later, after every wave has passed the barrier of the call in between).
template <int NW>
__device__ __forceinline__ int tk_block_sum(int wave_count, int* buf)
{
    if ((threadIdx.x & 63) == 0) buf[threadIdx.x >> 6] = wave_count;
    __syncthreads();
    int s = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) s += buf[w];
    return s;
}

// Exclusive workgroup scan (in lane order) of v, and the total.
template <int NW>
__device__ __forceinline__ uint32_t tk_block_scan(uint32_t v, uint32_t* buf, uint32_t& total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    if (lane == 63) buf[wave] = incl;
    __syncthreads();
    uint32_t before = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        before += w < wave ? buf[w] : 0u;
        total += buf[w];
    }
    return before + incl - v;
}

// The k largest of the workgroup's keys (key 0 = no element), ties by position: bit j of
// the returned mask marks the lane's key j, `pos` is the number of selected keys before
// the lane's first, `nsel` the number selected (min(k, elements)).
template <int NW>
__device__ __forceinline__ uint32_t tk_select(const uint32_t (&key)[TK_PER], int k, TkLds& L, int& pos, int& nsel)
{
    uint32_t T = 0;
    for (int b = 15; b >= 0; b--) {
        const uint32_t t = T | (1u << b);
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < TK_PER; j++) cnt += __popcll(__ballot(key[j] >= t));
        if (tk_block_sum<NW>(cnt, L.sums[b & 1]) >= k) T = t;
    }
    // T = the largest t with count(key >= t) >= k, or 0 when fewer than k keys exist (then
    // every key > 0 is selected and no key == T is)
    uint32_t gt = 0, eq = 0;
#pragma unroll
    for (int j = 0; j < TK_PER; j++) {
        gt += key[j] > T ? 1u : 0u;
        eq += T > 0 && key[j] == T ? 1u : 0u;
    }
    uint32_t total;                                   // counts packed in 16-bit halves (<= 8192 each)
    const uint32_t excl = tk_block_scan<NW>(gt | (eq << 16), L.scan[0], total);
    const int need = k - (int)(total & 0xffffu);      // ties taken, first positions first
    int r = (int)(excl >> 16);
    uint32_t mask = 0;
#pragma unroll
    for (int j = 0; j < TK_PER; j++) {
        const bool tie = T > 0 && key[j] == T;
        if (key[j] > T || (tie && r < need)) mask |= 1u << j;
        r += tie ? 1 : 0;
    }
    uint32_t all;
    pos = (int)tk_block_scan<NW>(__popc(mask), L.scan[1], all);
    nsel = (int)all;
    return mask;
}

template <bool ARGMAX>
__global__ __launch_bounds__(TK_T1) void topk_chunk_kernel(const uint16_t* __restrict__ x, long ld, int n, int k,
                                                            int nchunk, uint64_t* __restrict__ cand)
{
    __shared__ TkLds L;
    const int c = blockIdx.x, row = blockIdx.y;
    const int i0 = c * TK_CHUNK + threadIdx.x * TK_PER;   // this lane's first column

    // Two 16-byte loads; a run starting below n may pass n but stays inside the row's ld
    // columns (ld is a multiple of 8).
    uint32_t h[TK_PER], key[TK_PER];
    const uint16_t* p = x + (long)row * ld + i0;
#pragma unroll
    for (int v = 0; v < TK_PER / 8; v++) {
        uint4 q = {0u, 0u, 0u, 0u};
        if (i0 + 8 * v < n) q = *reinterpret_cast<const uint4*>(p + 8 * v);
        const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            h[8 * v + 2 * j] = w4[j] & 0xffffu;
            h[8 * v + 2 * j + 1] = w4[j] >> 16;
        }
    }
#pragma unroll
    for (int j = 0; j < TK_PER; j++) key[j] = i0 + j < n ? tk_key(h[j]) : 0u;

    uint64_t* out = cand + ((long)row * nchunk + c) * k;
    if constexpr (ARGMAX) {
        uint64_t b = 0;
#pragma unroll
        for (int j = 0; j < TK_PER; j++) {
            const uint64_t cj = key[j] ? tk_cand(key[j], i0 + j, h[j]) : 0u;
            if (tk_ord(cj) > tk_ord(b)) b = cj;
        }
        b = tk_block_argmax<TK_T1 / 64>(b, L.best);
        if (threadIdx.x == 0) out[0] = b;
        return;
    }
    int pos, nsel;
    const uint32_t mask = tk_select<TK_T1 / 64>(key, k, L, pos, nsel);
#pragma unroll
    for (int j = 0; j < TK_PER; j++)
        if (mask & (1u << j)) {
            if (pos < k) out[pos] = tk_cand(key[j], i0 + j, h[j]);   // pos < k by construction
            pos++;
        }
    if ((int)threadIdx.x < k - nsel) out[nsel + threadIdx.x] = 0;    // a chunk of fewer than k columns
}

template <bool ARGMAX, int T2>
__global__ __launch_bounds__(T2) void topk_merge_kernel(const uint64_t* __restrict__ cand, int m, int k,
                                                            uint16_t* __restrict__ values, int64_t* __restrict__ idx)
{
    __shared__ TkLds L;
    __shared__ uint64_t sel[TK_MAX_K];
    const int row = blockIdx.x;
    const uint64_t* cr = cand + (long)row * m + threadIdx.x * TK_PER;
    uint64_t v[TK_PER];
    uint32_t key[TK_PER];
#pragma unroll
    for (int j = 0; j < TK_PER; j++) {
        v[j] = (int)threadIdx.x * TK_PER + j < m ? cr[j] : 0u;
        key[j] = tk_cand_key(v[j]);
    }
    if constexpr (ARGMAX) {
        uint64_t b = 0;
#pragma unroll
        for (int j = 0; j < TK_PER; j++)
            if (tk_ord(v[j]) > tk_ord(b)) b = v[j];
        b = tk_block_argmax<T2 / 64>(b, L.best);
        if (threadIdx.x == 0) {
            values[row] = (uint16_t)(b & 0xffffu);
            idx[row] = tk_cand_col(b);
        }
        return;
    }
    int pos, nsel;
    const uint32_t mask = tk_select<T2 / 64>(key, k, L, pos, nsel);   // nsel = k: k <= n real candidates
#pragma unroll
    for (int j = 0; j < TK_PER; j++)
        if (mask & (1u << j)) {
            if (pos < TK_MAX_K) sel[pos] = v[j];
            pos++;
        }
    __syncthreads();
    if ((int)threadIdx.x < k) {
        // rank by key, then column: the k selected sit in column order in sel
        const uint64_t me = sel[threadIdx.x];
        const uint32_t mk = tk_cand_key(me);
        int rank = 0;
        for (int j = 0; j < k; j++) {
            const uint32_t kj = tk_cand_key(sel[j]);
            rank += kj > mk || (kj == mk && j < (int)threadIdx.x) ? 1 : 0;
        }
        values[(long)row * k + rank] = (uint16_t)(me & 0xffffu);
        idx[(long)row * k + rank] = tk_cand_col(me);
    }
}

size_t topk_workspace_bytes(int rows, int n, int k)
{
    if (rows <= 0 || n <= 0 || k <= 0) return 0;
    const long nchunk = (n + TK_CHUNK - 1) / TK_CHUNK;
    return (size_t)rows * nchunk * k * sizeof(uint64_t);
}

int topk_dispatch(const uint16_t* x, int rows, int n, long ld, int k, uint16_t* values, int64_t* idx,
                  void* workspace, hipStream_t stream)
{
    if (rows == 0) return EXL3_OK;
    const int nchunk = (n + TK_CHUNK - 1) / TK_CHUNK;
    uint64_t* cand = static_cast<uint64_t*>(workspace);
    const bool am = k == 1;
    hipLaunchKernelGGL(am ? topk_chunk_kernel<true> : topk_chunk_kernel<false>, dim3(nchunk, rows), dim3(TK_T1), 0,
                       stream, x, ld, n, k, nchunk, cand);
    int rc = check_launch("exl3_topk (chunks)");
    if (rc != EXL3_OK) return rc;
    // fewer waves for fewer candidates: every wave's ballot counts run on the CU's scalar unit
    const int m = nchunk * k;
    const void* mk = m <= 256 * TK_PER ? (am ? (const void*)&topk_merge_kernel<true, 256> : (const void*)&topk_merge_kernel<false, 256>)
                                       : (am ? (const void*)&topk_merge_kernel<true, TK_T2> : (const void*)&topk_merge_kernel<false, TK_T2>);
    const uint64_t* cand_c = cand;
    void* kargs[] = {&cand_c, const_cast<int*>(&m), &k, &values, &idx};
    hipLaunchKernel(mk, dim3(rows), dim3(m <= 256 * TK_PER ? 256 : TK_T2), kargs, 0, stream);
    return check_launch("exl3_topk (merge)");
}

}  // namespace exl3
