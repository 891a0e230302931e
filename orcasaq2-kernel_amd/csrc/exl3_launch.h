// Host-side helpers shared by the kernel translation units: status codes and the
// thread-local error message behind exl3_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/exl3hip.h"

namespace exl3 {

// Records a printf-style message for exl3_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Empties that message (for a refusal the caller recovers from).
void clear_error();

// Returns EXL3_OK, or records the pending launch error of `what`.
int check_launch(const char* what);

// Compute units of the current device (queried once per device).
int device_cus();

int reconstruct_dispatch(uint16_t* W, const uint32_t* trellis, int ic, int oc, int K, int cb, bool transposed,
                         hipStream_t stream);
// zero / nzero: 32-bit words the first workgroup sets to 0 (a following launch's counters:
// one launch fewer than a fill kernel of their own), or none.
int had_dispatch(const uint16_t* in, uint16_t* out, const uint16_t* pre, const uint16_t* post,
                 float scale, long rows, int cols, hipStream_t stream, uint32_t* zero = nullptr, int nzero = 0);

struct GemvShard {
    const uint32_t* trellis;
    const uint16_t* suh;
    const uint16_t* svh;
    uint16_t* C;       // (rows, ldc) fp16; this shard writes columns [0, oc)
    int ic, oc, K, cb;
    long ldc;
};

// A GEMV workspace: a reserved 16 KiB head (no kernel reads or writes it), then the
// accumulator area of the 1..4-row kernel's split column groups (GEMV_ACC_BYTES; zero-filled
// before a workspace's first call, and every call leaves it zero-filled), then the per-shard
// partial-sum buffers of all GEMV paths (no required contents).
constexpr size_t GEMV_COUNTER_BYTES = 16384;
constexpr size_t GEMV_ACC_BYTES = EXL3_GEMV_ACC_BYTES;
size_t gemv_workspace_bytes(int rows, int ic, int oc);
size_t gemv1_slot_bytes(int ic, int oc, int rows);
bool gemv1_plan_fits(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* slots,
                     size_t slot_bytes);
int gemv1_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* slots,
                   size_t slot_bytes, char* acc, size_t acc_bytes, hipStream_t stream);
int gemv_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows,
                  void* workspace, size_t ws_bytes, hipStream_t stream);
size_t gemm_workspace_bytes(int rows, int ic, int oc);
int gemm_dispatch(const uint16_t* A, const uint32_t* trellis, uint16_t* C, const uint16_t* suh,
                  const uint16_t* svh, void* workspace, size_t ws_bytes, int rows, int ic, int oc,
                  int K, int cb, hipStream_t stream);
size_t gemm_sk_slot_bytes(int rows, int oc);
size_t gemv16_shard_bytes(int ic, int oc);
int gemv16_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* ws, size_t ws_bytes,
                    hipStream_t stream);
size_t gemm_grouped_shard_bytes(int rows, int ic, int oc);
int gemm_grouped_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows, char* ws,
                          size_t ws_bytes, hipStream_t stream, const char* what = "exl3_gemm_grouped");
int gemm_sk_cus();
// The launch's tile counters, the first sk_ntiles(rows, oc) words of ws, must be 0 when it
// starts (exl3_gemm's Hadamard pass clears them).
int gemm_sk_dispatch(const uint16_t* Ah, const uint32_t* trellis, uint16_t* C, const uint16_t* svh, char* ws,
                     size_t ws_bytes, int rows, int ic, int oc, int K, int cb, hipStream_t stream);
int embed_dispatch(const int8_t* table, const void* scales, int scale_dtype, const int64_t* ids,
                   void* out, long n_ids, int vocab, int dim, hipStream_t stream);

constexpr int TK_MAX_K = EXL3_TOPK_MAX_K;
constexpr int TK_MAX_N = EXL3_TOPK_MAX_N;
size_t topk_workspace_bytes(int rows, int n, int k);
int topk_dispatch(const uint16_t* x, int rows, int n, long ld, int k, uint16_t* values, int64_t* idx,
                  void* workspace, hipStream_t stream);

}  // namespace exl3
