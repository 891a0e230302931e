// Prefill EXL3 GEMM (exl3_gemm):
//   C = fp16( H( fp16(H(A * suh)) . W_q ) * svh )
// Replaces the reconstruct branch of orcasaq2/ops.py:50-59 (had_r_128 -> reconstruct ->
// hgemm_recon -> had_r_128), and the fused exl3_gemm of orcasaq2/ops.py:46-49 for 17..144
// rows, with: one Hadamard pass over A into the workspace, then the stream-K kernel of
// gemm_sk.hip, which decodes trellis tiles straight into MFMA operands -- the dense W_q is
// never written to HBM -- and applies the output Hadamard and svh in its epilogue.  The tile
// height follows the row count (32, 48, 64, 96, 128 or 256 rows: gemm_sk.hip).
// Up to SK_PREP_MAX_ROWS rows (gemm_sk_plan.h) the activation pass is small and each launch
// mostly its fixed cost, so the call runs as the one-shard form of the grouped launch: one
// set-up kernel does the Hadamard pass and clears the tile counters, one launch fewer
// (measured on MI355X on the 27B shapes: 1-3 us faster per call at 17..144 rows, even at 384,
// slower from 1024 rows, where the 16-byte-lane Hadamard kernel moves the larger
// activations faster).  Above it: had_r_128 (whose first workgroup also clears the stream-K
// launch's tile counters, one launch fewer: down_proj at 2048 rows 394-402 -> 388-389 us in a
// same-box A/B) and the stream-K kernel.
#include "exl3_common.h"
#include "exl3_launch.h"
#include "gemm_sk_plan.h"

namespace exl3 {

size_t gemm_workspace_bytes(int rows, int ic, int oc)
{
    return gemm_sk_ah_bytes(rows, ic) + gemm_sk_slot_bytes(rows, oc);
}

int gemm_dispatch(const uint16_t* A, const uint32_t* trellis, uint16_t* C, const uint16_t* suh,
                  const uint16_t* svh, void* workspace, size_t ws_bytes, int rows, int ic, int oc,
                  int K, int cb, hipStream_t stream)
{
    const size_t need = gemm_workspace_bytes(rows, ic, oc);
    if (ws_bytes < need)
        return set_error(EXL3_ERR_WORKSPACE, "exl3_gemm: workspace of %zu bytes, %zu needed", ws_bytes, need);
    if (K < 1 || K > 8) return set_error(EXL3_ERR_ARG, "exl3_gemm: K=%d is not in 1..8", K);
    if (rows <= SK_PREP_MAX_ROWS) {
        // the same workspace layout: fp16(H(A * suh)) (rows x ic), then counters and slots
        const GemvShard d{trellis, suh, svh, C, ic, oc, K, cb, (long)oc};
        return gemm_grouped_dispatch(A, &d, 1, rows, static_cast<char*>(workspace), ws_bytes, stream, "exl3_gemm");
    }
    uint16_t* Ah = static_cast<uint16_t*>(workspace);
    const size_t ah = gemm_sk_ah_bytes(rows, ic);
    char* const sk_ws = static_cast<char*>(workspace) + ah;   // tile counters first, then slots
    int rc = had_dispatch(A, Ah, suh, nullptr, 1.0f, rows, ic, stream, reinterpret_cast<uint32_t*>(sk_ws),
                          sk_ntiles(rows, oc));
    if (rc != EXL3_OK) return rc;
    return gemm_sk_dispatch(Ah, trellis, C, svh, sk_ws, ws_bytes - ah, rows, ic, oc, K, cb, stream);
}

}  // namespace exl3
