// Prefill EXL3 GEMM (exl3_gemm):
//   C = fp16( H( fp16(H(A * suh)) . W_q ) * svh )
// Replaces the reconstruct branch of orcasaq2/ops.py:50-59 (had_r_128 -> reconstruct ->
// hgemm_recon -> had_r_128), and the fused exl3_gemm of orcasaq2/ops.py:46-49 for 17..144
// rows, with: one had_r_128 pass over A into the workspace, then the stream-K kernel of
// gemm_sk.hip, which decodes trellis tiles straight into LDS as MFMA operands -- the dense
// W_q is never written to HBM -- and applies the output Hadamard and svh in its epilogue.
// The tile height follows the row count (32, 48, 64, 96, 128 or 256 rows: gemm_sk.hip).
#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

static size_t gemm_ah_bytes(int rows, int ic) { return ((size_t)rows * ic * sizeof(uint16_t) + 255) & ~(size_t)255; }

size_t gemm_workspace_bytes(int rows, int ic, int oc)
{
    return gemm_ah_bytes(rows, ic) + gemm_sk_slot_bytes(rows, oc);
}

int gemm_dispatch(const uint16_t* A, const uint32_t* trellis, uint16_t* C, const uint16_t* suh,
                  const uint16_t* svh, void* workspace, size_t ws_bytes, int rows, int ic, int oc,
                  int K, int cb, hipStream_t stream)
{
    const size_t need = gemm_workspace_bytes(rows, ic, oc);
    if (ws_bytes < need)
        return set_error(EXL3_ERR_WORKSPACE, "exl3_gemm: workspace of %zu bytes, %zu needed", ws_bytes, need);
    if (K < 1 || K > 8) return set_error(EXL3_ERR_ARG, "exl3_gemm: K=%d is not in 1..8", K);
    uint16_t* Ah = static_cast<uint16_t*>(workspace);
    int rc = had_dispatch(A, Ah, suh, nullptr, 1.0f, rows, ic, stream);
    if (rc != EXL3_OK) return rc;
    const size_t ah = gemm_ah_bytes(rows, ic);
    return gemm_sk_dispatch(Ah, trellis, C, svh, static_cast<char*>(workspace) + ah, ws_bytes - ah, rows, ic, oc, K,
                            cb, stream);
}

}  // namespace exl3
