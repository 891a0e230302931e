/*
 * libexl3hip -- C ABI of the MI355X (gfx950) EXL3 trellis linear path.
 *
 * Every entry point replaces one native call the reference plugin makes into the
 * exllamav3 v1.5.1 extension (jschang/OrcaSAQ2-kernel, orcasaq2/ops.py and
 * orcasaq2/__init__.py), or one torch op of its Python layer, and is cited below.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers (hipMalloc / torch CUDA tensors) unless noted; fp16
 *     data is passed as raw 16-bit patterns.  `stream` is a hipStream_t (NULL = the null
 *     stream); every call only enqueues work on it, never synchronises, never allocates.
 *   - Return EXL3_OK (0) or an error code; exl3_last_error() then holds a message for the
 *     calling thread.  Argument checks happen on the host before anything is enqueued.
 *   - Trellis tensors are int16 (ic/16, oc/16, 16K), K = bits per weight in 1..8,
 *     contiguous, 4-byte aligned (orcasaq2/ops.py:28-34).  ic and oc are multiples of 128
 *     for the GEMV/GEMM/Hadamard paths (one Hadamard block = 128), of 16 for reconstruct.
 *   - codebook: EXL3_CB_3INST (neither .mcg nor .mul1 tensor present), EXL3_CB_MCG
 *     (.mcg present) -- the flags of orcasaq2/config.py:218.  EXL3_CB_MUL1 is reported
 *     as EXL3_ERR_UNSUPPORTED.
 *   - Workspaces are caller-owned device buffers (256-byte aligned) of at least the
 *     *_workspace_bytes() size; a call uses its workspace until its last kernel has run,
 *     so calls that may overlap in time must not share one.  GEMM and top-k workspaces
 *     have no required contents.  A GEMV workspace is a reserved 16 KiB head (no call
 *     reads it), then EXL3_GEMV_ACC_BYTES of accumulators that must be zero-filled before
 *     the workspace's first call -- every call leaves them zero-filled again -- then
 *     scratch with no required contents.  So one buffer serves any sequence of calls
 *     issued in order on one stream -- also HIP-graph replays of captured calls.
 */
#ifndef EXL3HIP_H
#define EXL3HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXL3_OK 0
#define EXL3_ERR_ARG 1          /* bad shape, pointer, alignment or parameter */
#define EXL3_ERR_UNSUPPORTED 2  /* e.g. the mul1 codebook */
#define EXL3_ERR_WORKSPACE 3    /* workspace too small */
#define EXL3_ERR_HIP 4          /* HIP reported an error while enqueuing */

#define EXL3_CB_3INST 0
#define EXL3_CB_MCG 1
#define EXL3_CB_MUL1 2

#define EXL3_GEMV_MAX_ROWS 16
/* Zero-filled accumulator area at byte 16384 of every GEMV workspace (see above). */
#define EXL3_GEMV_ACC_BYTES (6u << 20)
#define EXL3_MAX_SHARDS 64

/* Message for the last failing call on this thread ("" if none). */
const char* exl3_last_error(void);

/* Library ABI version (bumped on any signature change). */
int exl3_abi_version(void);

/*
 * Capture state of `stream`: *id = 0 when the stream is not being captured into a HIP
 * graph, else the capture's unique id (hipStreamGetCaptureInfo).  No counterpart in the
 * reference: the Python layer keys its GEMV workspaces by capture.  A workspace made during
 * a capture comes from that graph's private memory pool, and its zero-fill is a node of
 * that graph that runs only when the graph replays, so it is never used outside it.
 * Host-only.
 */
int exl3_stream_capture_id(void* stream, unsigned long long* id);

/*
 * Dense reconstruct: W (ic, oc) fp16 row-major from trellis (ic/16, oc/16, 16K).
 * Replaces ext.reconstruct(W, trellis, K, mcg, mul1)  [orcasaq2/ops.py:56,
 * orcasaq2/__init__.py:57].  W must be 16-byte aligned.  Bit-exact to the format.
 */
int exl3_reconstruct(void* W, const void* trellis, int ic, int oc, int K, int codebook, void* stream);

/*
 * Dense reconstruct, transposed: Wt (oc, ic) fp16 row-major, Wt[o][i] = W_q[i][o], from the
 * same trellis.  No entry point of the reference writes this layout: it is the reference's
 * reconstruct branch [orcasaq2/ops.py:54-59] made faster -- y = x W_q becomes a
 * transposed-B library GEMM (y = x Wt^T), the library's faster layout on MI355X.  Same
 * argument rules and bit-exactness as exl3_reconstruct.
 */
int exl3_reconstruct_t(void* Wt, const void* trellis, int ic, int oc, int K, int codebook, void* stream);

/*
 * Block-128 Walsh-Hadamard along the last dim of a (rows, cols) fp16 matrix:
 *   out = ((in * pre) . blockdiag(H128 / sqrt(128))) * post * scale
 * pre/post are fp16 (cols) vectors or NULL; in == out is allowed.
 * Replaces ext.had_r_128(in, out, pre, post, scale)  [orcasaq2/ops.py:54, 59].
 */
int exl3_had_r_128(const void* in, void* out, const void* pre, const void* post, float scale,
                   long rows, int cols, void* stream);

/*
 * Fused decode-GEMV, 1 <= rows <= 16:
 *   C (rows, oc) = fp16( H( fp16(H(A * suh)) . W_q ) * svh ),  A (rows, ic) fp16.
 * Replaces ext.exl3_gemm(A, trellis, C, suh, A_had, svh, -1, mcg, mul1, 0)
 * [orcasaq2/ops.py:46-49] for rows <= 16 (the A_had scratch is internal to the kernel).
 * rows 1..4 take one decode launch per codebook: a column group whose inputs are split over
 * several workgroups is added up in the workspace's accumulators and finished by the
 * workgroup that adds last (when a call's accumulators would exceed EXL3_GEMV_ACC_BYTES,
 * one small kernel after the launch adds the split partial sums instead); 5..16 rows take a
 * set-up kernel (every shard's transformed activations), then per codebook one decode
 * launch and one finishing launch.  Results do not depend on the order workgroups finish
 * in: the same inputs give the same bits on every call.
 */
size_t exl3_gemv_workspace_bytes(int rows, int ic, int oc);
int exl3_gemv(const void* A, const void* trellis, void* C, const void* suh, const void* svh,
              void* workspace, size_t ws_bytes, int rows, int ic, int oc, int K, int codebook,
              void* stream);

/*
 * Grouped GEMV: several shards that read the same activations A (rows, ic) -- the q/k/v
 * of qkv_proj or gate/up of gate_up_proj, each its own EXL3 tensor with its own K, suh
 * and svh -- in as few launches as there are distinct (K, codebook) pairs.  Shard s
 * writes C_s (rows, oc_s) with row stride ldc_s elements, so the shards can land
 * directly in the columns of one concatenated output.  Replaces the per-shard loop of
 * shard_gemm calls plus torch.cat at orcasaq2/config.py:237-243.  The workspace is the
 * sum of exl3_gemv_workspace_bytes over the shards.
 */
typedef struct exl3_shard {
    const void* trellis;
    const void* suh;
    const void* svh;
    void* C;
    long ldc;
    int oc;
    int K;
    int codebook;
} exl3_shard_t;

size_t exl3_gemv_grouped_workspace_bytes(const exl3_shard_t* shards, int nshards, int rows, int ic);
int exl3_gemv_grouped(const void* A, const exl3_shard_t* shards, int nshards, void* workspace,
                      size_t ws_bytes, int rows, int ic, void* stream);

/*
 * exl3_gemv_grouped without a workspace argument: it allocates nothing (no hipMalloc, no
 * library allocation), for callers that cannot allocate -- code under HIP-graph capture,
 * serving loops that forbid device allocation.  No counterpart in the reference.
 * The scratch is a file-scope device array of EXL3_STATIC_SCRATCH_BYTES (24 MiB), one per
 * GPU (zero-filled when the library is loaded, as a GEMV workspace's accumulators must
 * be), held until the process ends; a call whose exl3_gemv_grouped_workspace_bytes exceeds
 * it fails with EXL3_ERR_WORKSPACE (rows 1..4 fit every shape of the 27B model and its
 * 151936-wide lm_head; rows 5..16 fit every layer of that model and its lm_head).  All calls on one GPU
 * share the array and each leaves it ready for the next, so calls issued in order (one
 * stream, or graph replays in order) are safe; calls that may overlap in time race on it.
 */
#define EXL3_STATIC_SCRATCH_BYTES (24u << 20)
int exl3_gemv_grouped_static(const void* A, const exl3_shard_t* shards, int nshards, int rows, int ic,
                             void* stream);

/*
 * Prefill GEMM, any rows >= 1 (meant for rows > 16): same result as exl3_gemv, computed
 * as one Hadamard pass over A into the workspace plus one kernel that decodes trellis
 * tiles into fp16 MFMA operands (no dense W_q in HBM) and applies H and svh on output.
 * Replaces the reconstruct branch ext.had_r_128 -> ext.reconstruct -> ext.hgemm_recon ->
 * ext.had_r_128  [orcasaq2/ops.py:50-59].
 */
size_t exl3_gemm_workspace_bytes(int rows, int ic, int oc);
int exl3_gemm(const void* A, const void* trellis, void* C, const void* suh, const void* svh,
              void* workspace, size_t ws_bytes, int rows, int ic, int oc, int K, int codebook,
              void* stream);

/*
 * Grouped prefill GEMM: exl3_gemm for several shards that read the same A (the q/k/v of
 * qkv_proj, gate/up of gate_up_proj), with exl3_gemv_grouped's shard table and output
 * layout.  Per codebook one set-up kernel (every shard's Hadamard pass, the tile counters)
 * and one stream-K launch over all the shards' tiles, whatever their K (up to 384 rows;
 * above, one launch per K).  Replaces the per-shard loop of shard_gemm calls plus
 * torch.cat at orcasaq2/config.py:237-243 for 17 .. GEMM_MAX_ROWS rows.  The workspace is
 * exl3_gemm_grouped_workspace_bytes.
 */
size_t exl3_gemm_grouped_workspace_bytes(const exl3_shard_t* shards, int nshards, int rows, int ic);
int exl3_gemm_grouped(const void* A, const exl3_shard_t* shards, int nshards, void* workspace,
                      size_t ws_bytes, int rows, int ic, void* stream);

/*
 * int8 embedding gather: out[n, :] = dtype(table[ids[n], :]) * scales[ids[n]], computed
 * in the scale dtype (0 = fp16, 1 = bf16, 2 = fp32); table (vocab, dim) int8 with
 * dim % 4 == 0, scales (vocab) or (vocab, 1), ids int64 (n_ids), out (n_ids, dim).
 * Ids outside [0, vocab) give zero rows.
 * Replaces `q[ids].to(s.dtype) * s[ids]`  [orcasaq2/heads.py:61-67].
 */
int exl3_embed_int8_gather(const void* table, const void* scales, int scale_dtype, const void* ids,
                           void* out, long n_ids, int vocab, int dim, void* stream);

/*
 * Argmax / top-k epilogue of the output head: the k largest entries of each row of an fp16
 * matrix (the logits the K=6 lm_head's exl3_gemv writes), largest first, equal values by
 * smaller column; every NaN ranks above +inf (torch.argmax's order), -0 equals +0.  k = 1 is
 * the argmax of greedy decoding.  x (rows, ld) fp16, 16-byte aligned, ld % 8 == 0,
 * n <= ld columns used (each row may be read up to column ceil(n / 8) * 8 - 1);
 * 1 <= k <= EXL3_TOPK_MAX_K, k <= n <= EXL3_TOPK_MAX_N.  values (rows, k)
 * fp16 (the entries' own bits), indices (rows, k) int64.  workspace >=
 * exl3_topk_workspace_bytes(rows, n, k) bytes, 8-byte aligned.  Two kernels on the stream;
 * nothing allocated.
 * No counterpart in the reference: its lm_head is an ordinary EXL3 linear
 * [orcasaq2/config.py:128-132] whose logits vLLM's sampler reduces; this is that reduction on
 * the GEMV's stream.
 */
#define EXL3_TOPK_MAX_K 64
#define EXL3_TOPK_MAX_N (1 << 19)
size_t exl3_topk_workspace_bytes(int rows, int n, int k);
int exl3_topk(const void* x, int rows, int n, long ld, int k, void* values, void* indices, void* workspace,
              size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3HIP_H */
