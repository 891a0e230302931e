// Fused EXL3 decode-GEMV for 1..16 activation rows:
//   C = fp16( H( fp16(H(A * suh)) . W_q ) * svh )
// with W_q decoded from the packed trellis on the fly and never written anywhere.
// Replaces exllamav3_ext.exl3_gemm as called at orcasaq2/ops.py:46-49 (rows <= 144 there;
// this path takes rows <= 16 and the MFMA GEMM takes the rest).  This file routes a call by
// its row count:
//   * 1: gemv1.hip (persistent decode, MFMA multiply-accumulate);
//   * 2..4: gemv1.hip as well (its four-row template), unless its plan refuses the shards --
//     a workgroup range's activation tables would exceed a CU's LDS even at G1_GMAX
//     workgroups, which takes some 2.6e9 weights in one launch -- then gemv16.hip;
//   * 5..16: gemv16.hip (the batch-1 decode on 4 x 2-tile units, one MFMA serving all 16
//     rows; the cost hardly depends on the row count).
#include "exl3_launch.h"

#include <algorithm>

namespace exl3 {

constexpr int GV_MAX_ROWS = 16;
constexpr int GV_G1_MAX_ROWS = 4;   // the four-row template of gemv1.hip

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Per-shard share of a GEMV workspace (the reserved head area is added once per call).
// 2..4 rows: enough for either path, gemv1's slots or gemv16's fragments and slots.
size_t gemv_workspace_bytes(int rows, int ic, int oc)
{
    if (rows == 1) return align256(gemv1_slot_bytes(ic, oc, 1));
    if (rows <= GV_G1_MAX_ROWS) return align256(std::max(gemv1_slot_bytes(ic, oc, rows), gemv16_shard_bytes(ic, oc)));
    return align256(gemv16_shard_bytes(ic, oc));
}

int gemv_dispatch(const uint16_t* A, const GemvShard* shards, int nshards, int rows,
                  void* workspace, size_t ws_bytes, hipStream_t stream)
{
    if (rows < 1 || rows > GV_MAX_ROWS)
        return set_error(EXL3_ERR_ARG, "exl3_gemv: rows=%d is not in 1..%d", rows, GV_MAX_ROWS);
    size_t need = GEMV_COUNTER_BYTES + GEMV_ACC_BYTES;
    for (int i = 0; i < nshards; i++) need += gemv_workspace_bytes(rows, shards[i].ic, shards[i].oc);
    if (ws_bytes < need)
        return set_error(EXL3_ERR_WORKSPACE, "exl3_gemv: workspace of %zu bytes, %zu needed", ws_bytes, need);

    char* acc = static_cast<char*>(workspace) + GEMV_COUNTER_BYTES;
    char* ws = acc + GEMV_ACC_BYTES;
    const size_t wsb = need - GEMV_COUNTER_BYTES - GEMV_ACC_BYTES;
    if (rows == 1 || (rows <= GV_G1_MAX_ROWS && gemv1_plan_fits(A, shards, nshards, rows, ws, wsb)))
        return gemv1_dispatch(A, shards, nshards, rows, ws, wsb, acc, GEMV_ACC_BYTES, stream);
    return gemv16_dispatch(A, shards, nshards, rows, ws, wsb, stream);
}

}  // namespace exl3
