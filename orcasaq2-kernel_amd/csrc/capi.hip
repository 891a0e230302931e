// extern "C" entry points of libexl3hip (declared in include/exl3hip.h): host-side
// argument checks, then dispatch to the kernel translation units.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_err[0] = 0; }

int check_launch(const char* what)
{
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(EXL3_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return EXL3_OK;
}

// Compute units of the current device, queried once per device (every plan asks on every
// call).
int device_cus()
{
    constexpr int MAXDEV = 64;
    static int cus_of[MAXDEV];
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) {
        (void)hipGetLastError();
        return 256;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (cus_of[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
            (void)hipGetLastError();
            cus = 256;
        }
        cus_of[dev] = cus;
    }
    return cus_of[dev];
}

static bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

static int check_codebook(const char* fn, int cb)
{
    if (cb == CB_MUL1)
        return set_error(EXL3_ERR_UNSUPPORTED, "%s: the mul1 codebook is not supported", fn);
    if (cb != CB_3INST && cb != CB_MCG) return set_error(EXL3_ERR_ARG, "%s: unknown codebook %d", fn, cb);
    return EXL3_OK;
}

static int check_linear(const char* fn, const void* trellis, const void* suh, const void* svh, int ic, int oc,
                        int K, int cb)
{
    if (!trellis || !suh || !svh) return set_error(EXL3_ERR_ARG, "%s: null trellis/suh/svh", fn);
    if (ic <= 0 || oc <= 0 || ic % 128 || oc % 128)
        return set_error(EXL3_ERR_ARG, "%s: ic=%d and oc=%d must be positive multiples of 128", fn, ic, oc);
    if (K < 1 || K > 8) return set_error(EXL3_ERR_ARG, "%s: K=%d is not in 1..8", fn, K);
    if (!aligned(trellis, 4) || !aligned(suh, 4) || !aligned(svh, 4))
        return set_error(EXL3_ERR_ARG, "%s: trellis/suh/svh must be 4-byte aligned", fn);
    return check_codebook(fn, cb);
}

}  // namespace exl3

using namespace exl3;

extern "C" {

const char* exl3_last_error(void) { return g_err; }

int exl3_abi_version(void) { return 7; }

int exl3_stream_capture_id(void* stream, unsigned long long* id)
{
    g_err[0] = 0;
    if (!id) return set_error(EXL3_ERR_ARG, "exl3_stream_capture_id: null id");
    *id = 0;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    const hipError_t e = hipStreamGetCaptureInfo(static_cast<hipStream_t>(stream), &st, &cid);
    if (e != hipSuccess)
        return set_error(EXL3_ERR_HIP, "exl3_stream_capture_id: %s", hipGetErrorString(e));
    if (st == hipStreamCaptureStatusActive) *id = cid ? cid : 1;
    return EXL3_OK;
}

int exl3_reconstruct(void* W, const void* trellis, int ic, int oc, int K, int codebook, void* stream)
{
    g_err[0] = 0;
    if (!W || !trellis) return set_error(EXL3_ERR_ARG, "exl3_reconstruct: null pointer");
    if (ic <= 0 || oc <= 0 || ic % 16 || oc % 16)
        return set_error(EXL3_ERR_ARG, "exl3_reconstruct: ic=%d and oc=%d must be positive multiples of 16", ic, oc);
    if (!aligned(W, 16) || !aligned(trellis, 4))
        return set_error(EXL3_ERR_ARG, "exl3_reconstruct: W must be 16-byte and trellis 4-byte aligned");
    int rc = check_codebook("exl3_reconstruct", codebook);
    if (rc) return rc;
    return reconstruct_dispatch(static_cast<uint16_t*>(W), static_cast<const uint32_t*>(trellis), ic, oc, K,
                                codebook, false, static_cast<hipStream_t>(stream));
}

int exl3_reconstruct_t(void* Wt, const void* trellis, int ic, int oc, int K, int codebook, void* stream)
{
    g_err[0] = 0;
    if (!Wt || !trellis) return set_error(EXL3_ERR_ARG, "exl3_reconstruct_t: null pointer");
    if (ic <= 0 || oc <= 0 || ic % 16 || oc % 16)
        return set_error(EXL3_ERR_ARG, "exl3_reconstruct_t: ic=%d and oc=%d must be positive multiples of 16", ic,
                         oc);
    if (!aligned(Wt, 16) || !aligned(trellis, 4))
        return set_error(EXL3_ERR_ARG, "exl3_reconstruct_t: Wt must be 16-byte and trellis 4-byte aligned");
    int rc = check_codebook("exl3_reconstruct_t", codebook);
    if (rc) return rc;
    return reconstruct_dispatch(static_cast<uint16_t*>(Wt), static_cast<const uint32_t*>(trellis), ic, oc, K,
                                codebook, true, static_cast<hipStream_t>(stream));
}

int exl3_had_r_128(const void* in, void* out, const void* pre, const void* post, float scale, long rows, int cols,
                   void* stream)
{
    g_err[0] = 0;
    if (!in || !out) return set_error(EXL3_ERR_ARG, "exl3_had_r_128: null in/out");
    if (rows < 0 || cols <= 0 || cols % 128)
        return set_error(EXL3_ERR_ARG, "exl3_had_r_128: rows=%ld, cols=%d (cols must be a multiple of 128)", rows,
                         cols);
    if (!aligned(in, 4) || !aligned(out, 4) || (pre && !aligned(pre, 4)) || (post && !aligned(post, 4)))
        return set_error(EXL3_ERR_ARG, "exl3_had_r_128: pointers must be 4-byte aligned");
    return had_dispatch(static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out),
                        static_cast<const uint16_t*>(pre), static_cast<const uint16_t*>(post), scale, rows, cols,
                        static_cast<hipStream_t>(stream));
}

size_t exl3_gemv_workspace_bytes(int rows, int ic, int oc)
{
    if (rows < 1 || ic < 128 || oc < 128) return 0;
    return GEMV_COUNTER_BYTES + GEMV_ACC_BYTES + gemv_workspace_bytes(rows, ic, oc);
}

size_t exl3_gemv_grouped_workspace_bytes(const exl3_shard_t* shards, int nshards, int rows, int ic)
{
    if (!shards || nshards < 1 || rows < 1 || ic < 128) return 0;
    size_t t = GEMV_COUNTER_BYTES + GEMV_ACC_BYTES;
    for (int i = 0; i < nshards; i++) {
        if (shards[i].oc < 128) return 0;
        t += gemv_workspace_bytes(rows, ic, shards[i].oc);
    }
    return t;
}

int exl3_gemv_grouped(const void* A, const exl3_shard_t* shards, int nshards, void* workspace, size_t ws_bytes,
                      int rows, int ic, void* stream)
{
    g_err[0] = 0;
    if (!A || !shards || nshards < 1 || nshards > EXL3_MAX_SHARDS)
        return set_error(EXL3_ERR_ARG, "exl3_gemv: need A and 1..%d shards (got %d)", EXL3_MAX_SHARDS, nshards);
    if (!workspace) return set_error(EXL3_ERR_ARG, "exl3_gemv: null workspace");
    if (!aligned(A, 4) || !aligned(workspace, 256))
        return set_error(EXL3_ERR_ARG, "exl3_gemv: A must be 4-byte and workspace 256-byte aligned");
    GemvShard d[EXL3_MAX_SHARDS];
    for (int i = 0; i < nshards; i++) {
        const exl3_shard_t& s = shards[i];
        int rc = check_linear("exl3_gemv", s.trellis, s.suh, s.svh, ic, s.oc, s.K, s.codebook);
        if (rc) return rc;
        if (!s.C || !aligned(s.C, 4) || s.ldc < s.oc || s.ldc % 2)
            return set_error(EXL3_ERR_ARG, "exl3_gemv: shard %d: C must be 4-byte aligned with even ldc >= oc", i);
        d[i] = GemvShard{static_cast<const uint32_t*>(s.trellis), static_cast<const uint16_t*>(s.suh),
                         static_cast<const uint16_t*>(s.svh), static_cast<uint16_t*>(s.C), ic, s.oc, s.K,
                         s.codebook, s.ldc};
    }
    return gemv_dispatch(static_cast<const uint16_t*>(A), d, nshards, rows, workspace, ws_bytes,
                         static_cast<hipStream_t>(stream));
}

int exl3_gemv(const void* A, const void* trellis, void* C, const void* suh, const void* svh, void* workspace,
              size_t ws_bytes, int rows, int ic, int oc, int K, int codebook, void* stream)
{
    exl3_shard_t s = {trellis, suh, svh, C, (long)oc, oc, K, codebook};
    return exl3_gemv_grouped(A, &s, 1, workspace, ws_bytes, rows, ic, stream);
}

size_t exl3_gemm_workspace_bytes(int rows, int ic, int oc)
{
    if (rows < 1 || ic < 128 || oc < 128) return 0;
    return gemm_workspace_bytes(rows, ic, oc);
}

int exl3_gemm(const void* A, const void* trellis, void* C, const void* suh, const void* svh, void* workspace,
              size_t ws_bytes, int rows, int ic, int oc, int K, int codebook, void* stream)
{
    g_err[0] = 0;
    int rc = check_linear("exl3_gemm", trellis, suh, svh, ic, oc, K, codebook);
    if (rc) return rc;
    if (!A || !C || !workspace) return set_error(EXL3_ERR_ARG, "exl3_gemm: null A/C/workspace");
    if (rows < 1) return set_error(EXL3_ERR_ARG, "exl3_gemm: rows=%d", rows);
    if (!aligned(A, 4) || !aligned(C, 4) || !aligned(workspace, 256))
        return set_error(EXL3_ERR_ARG, "exl3_gemm: A, C must be 4-byte and workspace 256-byte aligned");
    return gemm_dispatch(static_cast<const uint16_t*>(A), static_cast<const uint32_t*>(trellis),
                         static_cast<uint16_t*>(C), static_cast<const uint16_t*>(suh),
                         static_cast<const uint16_t*>(svh), workspace, ws_bytes, rows, ic, oc, K, codebook,
                         static_cast<hipStream_t>(stream));
}

size_t exl3_gemm_grouped_workspace_bytes(const exl3_shard_t* shards, int nshards, int rows, int ic)
{
    if (!shards || nshards < 1 || rows < 1 || ic < 128) return 0;
    size_t t = 0;
    for (int i = 0; i < nshards; i++) {
        if (shards[i].oc < 128) return 0;
        t += gemm_grouped_shard_bytes(rows, ic, shards[i].oc);
    }
    return t;
}

int exl3_gemm_grouped(const void* A, const exl3_shard_t* shards, int nshards, void* workspace, size_t ws_bytes,
                      int rows, int ic, void* stream)
{
    g_err[0] = 0;
    if (!A || !shards || nshards < 1 || nshards > EXL3_MAX_SHARDS)
        return set_error(EXL3_ERR_ARG, "exl3_gemm_grouped: need A and 1..%d shards (got %d)", EXL3_MAX_SHARDS,
                         nshards);
    if (!workspace) return set_error(EXL3_ERR_ARG, "exl3_gemm_grouped: null workspace");
    if (rows < 1) return set_error(EXL3_ERR_ARG, "exl3_gemm_grouped: rows=%d", rows);
    if (!aligned(A, 4) || !aligned(workspace, 256))
        return set_error(EXL3_ERR_ARG, "exl3_gemm_grouped: A must be 4-byte and workspace 256-byte aligned");
    const size_t need = exl3_gemm_grouped_workspace_bytes(shards, nshards, rows, ic);
    GemvShard d[EXL3_MAX_SHARDS];
    for (int i = 0; i < nshards; i++) {
        const exl3_shard_t& s = shards[i];
        int rc = check_linear("exl3_gemm_grouped", s.trellis, s.suh, s.svh, ic, s.oc, s.K, s.codebook);
        if (rc) return rc;
        if (!s.C || !aligned(s.C, 4) || s.ldc < s.oc || s.ldc % 2)
            return set_error(EXL3_ERR_ARG, "exl3_gemm_grouped: shard %d: C must be 4-byte aligned with even ldc >= oc",
                             i);
        d[i] = GemvShard{static_cast<const uint32_t*>(s.trellis), static_cast<const uint16_t*>(s.suh),
                         static_cast<const uint16_t*>(s.svh), static_cast<uint16_t*>(s.C), ic, s.oc, s.K,
                         s.codebook, s.ldc};
    }
    if (ws_bytes < need)
        return set_error(EXL3_ERR_WORKSPACE, "exl3_gemm_grouped: workspace of %zu bytes, %zu needed", ws_bytes, need);
    return gemm_grouped_dispatch(static_cast<const uint16_t*>(A), d, nshards, rows, static_cast<char*>(workspace),
                                 ws_bytes, static_cast<hipStream_t>(stream));
}

int exl3_embed_int8_gather(const void* table, const void* scales, int scale_dtype, const void* ids, void* out,
                           long n_ids, int vocab, int dim, void* stream)
{
    g_err[0] = 0;
    if (n_ids < 0 || vocab < 0 || dim <= 0 || dim % 4)
        return set_error(EXL3_ERR_ARG, "exl3_embed_int8_gather: n_ids=%ld vocab=%d dim=%d (dim %% 4 == 0)", n_ids,
                         vocab, dim);
    if (n_ids > 0 && (!table || !scales || !ids || !out))
        return set_error(EXL3_ERR_ARG, "exl3_embed_int8_gather: null pointer");
    if (scale_dtype < 0 || scale_dtype > 2)
        return set_error(EXL3_ERR_ARG, "exl3_embed_int8_gather: scale dtype %d", scale_dtype);
    if (!aligned(table, 4) || !aligned(ids, 8) || !aligned(out, scale_dtype == 2 ? 16 : 8) ||
        !aligned(scales, scale_dtype == 2 ? 4 : 2))
        return set_error(EXL3_ERR_ARG, "exl3_embed_int8_gather: misaligned pointer");
    return embed_dispatch(static_cast<const int8_t*>(table), scales, scale_dtype, static_cast<const int64_t*>(ids),
                          out, n_ids, vocab, dim, static_cast<hipStream_t>(stream));
}

size_t exl3_topk_workspace_bytes(int rows, int n, int k) { return topk_workspace_bytes(rows, n, k); }

int exl3_topk(const void* x, int rows, int n, long ld, int k, void* values, void* indices, void* workspace,
              size_t workspace_bytes, void* stream)
{
    g_err[0] = 0;
    if (rows < 0 || rows > 65535)
        return set_error(EXL3_ERR_ARG, "exl3_topk: rows=%d is not in 0..65535", rows);
    if (k < 1 || k > EXL3_TOPK_MAX_K || n < k || n > EXL3_TOPK_MAX_N)
        return set_error(EXL3_ERR_ARG, "exl3_topk: k=%d n=%d (need 1 <= k <= %d, k <= n <= %d)", k, n,
                         EXL3_TOPK_MAX_K, EXL3_TOPK_MAX_N);
    if (ld < n || ld % 8)
        return set_error(EXL3_ERR_ARG, "exl3_topk: ld=%ld (need ld >= n=%d, ld %% 8 == 0)", ld, n);
    if (rows == 0) return EXL3_OK;
    if (!x || !values || !indices || !workspace) return set_error(EXL3_ERR_ARG, "exl3_topk: null pointer");
    if (!aligned(x, 16) || !aligned(values, 2) || !aligned(indices, 8) || !aligned(workspace, 8))
        return set_error(EXL3_ERR_ARG, "exl3_topk: misaligned pointer (x 16, values 2, indices 8, workspace 8 bytes)");
    const size_t need = topk_workspace_bytes(rows, n, k);
    if (workspace_bytes < need)
        return set_error(EXL3_ERR_WORKSPACE, "exl3_topk: workspace %zu bytes < %zu needed", workspace_bytes, need);
    return topk_dispatch(static_cast<const uint16_t*>(x), rows, n, ld, k, static_cast<uint16_t*>(values),
                         static_cast<int64_t*>(indices), workspace, static_cast<hipStream_t>(stream));
}

}  // extern "C"
