// exl3_gemv_grouped_static: the grouped GEMV with its workspace in a file-scope device array
// instead of a caller buffer, for callers that cannot allocate device memory (code under
// HIP-graph capture, serving loops that forbid hipMalloc).  It has no counterpart in the
// reference plugin.
//
// The array `scratch` is one per GPU (each device holds its own copy at its own address).
// Host code never passes the array's name to a kernel: that name is a host-side stand-in,
// not a device address.  The first call on a device resolves the device address with
// hipGetSymbolAddress (that device current) and keeps it; every later call uses the kept
// pointer.  The workspace has no required contents (include/exl3hip.h), so nothing is
// cleared.
//
// All calls on one GPU share its array: calls that may overlap in time (different streams
// without ordering between them, or graphs replayed concurrently) race on it.
#include <mutex>

#include "exl3_common.h"
#include "exl3_launch.h"

namespace exl3 {

static __device__ __align__(256) unsigned char scratch[EXL3_STATIC_SCRATCH_BYTES];

constexpr int NA_MAX_DEVICES = 64;
static void* g_scratch_ptr[NA_MAX_DEVICES];
static std::mutex g_scratch_mu;

// Device address of this device's `scratch`, resolved on the device's first call.
static int na_scratch(void** out)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(EXL3_ERR_HIP, "exl3_gemv_grouped_static: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= NA_MAX_DEVICES)
        return set_error(EXL3_ERR_ARG, "exl3_gemv_grouped_static: device %d (at most %d devices)", dev, NA_MAX_DEVICES);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(EXL3_ERR_HIP, "exl3_gemv_grouped_static: hipGetSymbolAddress(scratch): %s",
                             hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return EXL3_OK;
}

}  // namespace exl3

using namespace exl3;

extern "C" int exl3_gemv_grouped_static(const void* A, const exl3_shard_t* shards, int nshards, int rows, int ic,
                                        void* stream)
{
    if (!shards || nshards < 1 || nshards > EXL3_MAX_SHARDS)
        return set_error(EXL3_ERR_ARG, "exl3_gemv_grouped_static: need 1..%d shards (got %d)", EXL3_MAX_SHARDS,
                         nshards);
    const size_t need = exl3_gemv_grouped_workspace_bytes(shards, nshards, rows, ic);
    if (need == 0)
        return set_error(EXL3_ERR_ARG, "exl3_gemv_grouped_static: rows=%d, ic=%d or a shard's oc is out of range",
                         rows, ic);
    if (need > (size_t)EXL3_STATIC_SCRATCH_BYTES)
        return set_error(EXL3_ERR_WORKSPACE,
                         "exl3_gemv_grouped_static: this call needs %zu bytes of scratch, above the static "
                         "maximum of %zu (EXL3_STATIC_SCRATCH_BYTES); use exl3_gemv_grouped with a workspace",
                         need, (size_t)EXL3_STATIC_SCRATCH_BYTES);
    void* ws = nullptr;
    const int rc = na_scratch(&ws);
    if (rc != EXL3_OK) return rc;
    return exl3_gemv_grouped(A, shards, nshards, ws, (size_t)EXL3_STATIC_SCRATCH_BYTES, rows, ic, stream);
}
