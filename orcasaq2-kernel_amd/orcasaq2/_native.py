"""ctypes binding of libexl3hip.so (include/exl3hip.h) for torch tensors on the GPU.

This is the only place Python crosses into native code.  Each wrapper validates device,
dtype, contiguity and shapes on the host (raising RuntimeError, as the reference's
extension does, e.g. orcasaq2/ops.py:29-31), allocates outputs and workspaces through
torch's caching allocator, and enqueues on torch's current stream.  There is no fallback:
if the library is missing or a tensor is not on the GPU, the call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_NAME = "libexl3hip.so"
LIB_PATH = os.environ.get("ORCASAQ2_LIB", os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME))
ABI_VERSION = 7

CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2
GEMV_MAX_ROWS = 16
MAX_SHARDS = 64
TOPK_MAX_K = 64
TOPK_MAX_N = 1 << 19

_lib = None
_lock = threading.Lock()


class Shard(ctypes.Structure):
    """exl3_shard_t."""
    _fields_ = [("trellis", ctypes.c_void_p), ("suh", ctypes.c_void_p), ("svh", ctypes.c_void_p),
                ("C", ctypes.c_void_p), ("ldc", ctypes.c_long), ("oc", ctypes.c_int),
                ("K", ctypes.c_int), ("codebook", ctypes.c_int)]


_SIGS = {
    "exl3_last_error": (ctypes.c_char_p, []),
    "exl3_abi_version": (ctypes.c_int, []),
    "exl3_stream_capture_id": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_ulonglong)]),
    "exl3_reconstruct": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "exl3_reconstruct_t": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "exl3_had_r_128": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_float, ctypes.c_long, ctypes.c_int, ctypes.c_void_p]),
    "exl3_gemv_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "exl3_gemv": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "exl3_gemv_grouped_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Shard), ctypes.c_int,
                                                            ctypes.c_int, ctypes.c_int]),
    "exl3_gemv_grouped": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Shard), ctypes.c_int,
                                         ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_void_p]),
    "exl3_gemv_grouped_static": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Shard), ctypes.c_int,
                                                ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "exl3_gemm_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "exl3_gemm": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "exl3_gemm_grouped_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Shard), ctypes.c_int,
                                                            ctypes.c_int, ctypes.c_int]),
    "exl3_gemm_grouped": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Shard), ctypes.c_int,
                                         ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_void_p]),
    "exl3_embed_int8_gather": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                              ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long,
                                              ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "exl3_topk_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "exl3_topk": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_long, ctypes.c_int,
                                 ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                 ctypes.c_void_p]),
}

EXPORTED = tuple(_SIGS)


def lib() -> ctypes.CDLL:
    """Loads libexl3hip.so (after torch, so the HIP runtime torch mapped is reused)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"orcasaq2 needs its HIP library and {LIB_PATH} does not exist. Build it with\n"
                    "  python orcasaq2-kernel_amd/build_lib.py\n"
                    "(hipcc --offload-arch=gfx950; cross-compiles without a GPU).")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            v = L.exl3_abi_version()
            if v != ABI_VERSION:
                raise RuntimeError(f"orcasaq2: {LIB_PATH} has ABI {v}, this package wants {ABI_VERSION}")
            _lib = L
    return _lib


def _check(rc: int, fn: str) -> None:
    if rc != 0:
        msg = lib().exl3_last_error().decode(errors="replace")
        raise RuntimeError(f"{fn} failed ({rc}): {msg}")


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _need_gpu(fn: str, *ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"{fn}: tensors must be on the GPU (got {t.device}); "
                               "orcasaq2 has no CPU path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{fn}: tensors on different devices ({dev} and {t.device})")
    return dev


def _need(cond: bool, fn: str, msg: str) -> None:
    if not cond:
        raise RuntimeError(f"{fn}: {msg}")


def codebook_id(mcg: bool, mul1: bool) -> int:
    if mul1:
        raise RuntimeError("orcasaq2: the mul1 codebook is not supported by the HIP kernels")
    return CB_MCG if mcg else CB_3INST


def check_trellis(fn: str, trellis: torch.Tensor, ic: int, oc: int, K) -> int:
    """trellis must be int16 (ic/16, oc/16, 16K), contiguous (orcasaq2/ops.py:28-34)."""
    _need(trellis.dtype in (torch.int16, torch.uint16), fn, f"trellis must be int16, got {trellis.dtype}")
    _need(trellis.is_contiguous(), fn, "trellis must be contiguous")
    if not float(K).is_integer():
        raise RuntimeError(f"{fn}: K={K}: half-rate (mul1) trellis widths are not supported")
    K = int(K)
    _need(1 <= K <= 8, fn, f"K={K} is not in 1..8")
    _need(trellis.dim() == 3 and trellis.shape[0] * 16 == ic and trellis.shape[1] * 16 == oc, fn,
          f"trellis shape {tuple(trellis.shape)} does not match ic={ic}, oc={oc}")
    _need(trellis.shape[2] == 16 * K, fn, f"packed dimension 2 is incorrect size "
          f"({trellis.shape[2]} for K={K})")
    return K


def _vec16(fn: str, name: str, t: torch.Tensor, n: int) -> None:
    _need(t.dtype == torch.float16, fn, f"{name} must be fp16, got {t.dtype}")
    _need(t.is_contiguous() and t.numel() == n, fn, f"{name} must be contiguous with {n} elements")


# ---------------------------------------------------------------- workspaces

def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-call scratch from torch's caching allocator (no required contents); it stays
    alive on the stream it was allocated on until the kernels using it have run."""
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


# GEMV workspaces.  A workspace's accumulator area must be zero before its first call and
# every call leaves it zero (include/exl3hip.h), so workspaces are made zero-filled and one
# buffer serves every call issued in order on one stream.
#   _gemv_ws[(device, stream)]            made by an eager call.
#   _gemv_ws_cap[(device, stream)]        (capture id, workspace) made inside a graph capture
#                                         because the stream had no large-enough eager
#                                         workspace.  Its memory comes from that graph's pool,
#                                         which keeps it for as long as the graph lives, so the
#                                         entry serves that capture only and is simply replaced
#                                         by the next capture on the stream (the memory may
#                                         then go to tensors of later captures into the same
#                                         pool, which torch replays one graph at a time: the
#                                         zero-fill made during the capture is a node of that
#                                         graph, so each replay clears the area again before
#                                         its calls).
# An eager workspace that a captured graph uses is never freed (_gemv_ws_kept): the graph's
# replays keep writing to it after the eager side has moved on to a larger buffer, and an
# eager free would hand it to unrelated tensors.  That list grows only when a captured
# stream's eager workspace is outgrown, so it holds at most one buffer per size step a
# process takes, however many graphs it captures and destroys.
_gemv_ws: dict = {}
_gemv_ws_cap: dict = {}
_gemv_ws_captured: set = set()
_gemv_ws_kept: list = []


def capture_id(device: torch.device) -> int:
    """0 when the current stream of `device` is not being captured, else the capture's id."""
    cid = ctypes.c_ulonglong(0)
    _check(lib().exl3_stream_capture_id(_stream(device), ctypes.byref(cid)), "exl3_stream_capture_id")
    return int(cid.value)


def _new_gemv_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    return torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)


def gemv_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """The GEMV workspace for a call on the current stream of `device` (see above).  Calls on
    one stream run in order, so they can share one; another stream gets its own, and so does
    a graph capture that finds no eager workspace of the size it needs on its stream."""
    stream = torch.cuda.current_stream(device).cuda_stream
    dev = device.index if device.index is not None else torch.cuda.current_device()
    key = (dev, stream)
    ws = _gemv_ws.get(key)
    cid = capture_id(device) if torch.cuda.is_current_stream_capturing() else 0
    if cid:
        if ws is None or ws.numel() < nbytes:
            ent = _gemv_ws_cap.get(key)
            if ent is None or ent[0] != cid or ent[1].numel() < nbytes:
                ent = (cid, _new_gemv_workspace(device, nbytes))
                _gemv_ws_cap[key] = ent
            return ent[1]
        if ws.data_ptr() not in _gemv_ws_captured:
            _gemv_ws_captured.add(ws.data_ptr())
            _gemv_ws_kept.append(ws)
        return ws
    if ws is None or ws.numel() < nbytes:
        ws = _new_gemv_workspace(device, nbytes)
        _gemv_ws[key] = ws
    return ws


# ---------------------------------------------------------------- entry points

def reconstruct(trellis: torch.Tensor, K, codebook: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """W_q (ic, oc) fp16 from trellis (ic/16, oc/16, 16K) -- ext.reconstruct (orcasaq2/ops.py:56)."""
    fn = "exl3_reconstruct"
    dev = _need_gpu(fn, trellis, out)
    ic, oc = trellis.shape[0] * 16, trellis.shape[1] * 16
    K = check_trellis(fn, trellis, ic, oc, K)
    if out is None:
        out = torch.empty((ic, oc), dtype=torch.float16, device=dev)
    _need(out.dtype == torch.float16 and out.is_contiguous() and tuple(out.shape) == (ic, oc), fn,
          "out must be contiguous fp16 (ic, oc)")
    _check(lib().exl3_reconstruct(_ptr(out), _ptr(trellis), ic, oc, K, codebook, _stream(dev)), fn)
    return out


def reconstruct_t(trellis: torch.Tensor, K, codebook: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """W_q^T (oc, ic) fp16 from the same trellis: the reconstruct branch's operand for a
    transposed-B library GEMM (orcasaq2/ops.py:54-59 multiplies by W_q)."""
    fn = "exl3_reconstruct_t"
    dev = _need_gpu(fn, trellis, out)
    ic, oc = trellis.shape[0] * 16, trellis.shape[1] * 16
    K = check_trellis(fn, trellis, ic, oc, K)
    if out is None:
        out = torch.empty((oc, ic), dtype=torch.float16, device=dev)
    _need(out.dtype == torch.float16 and out.is_contiguous() and tuple(out.shape) == (oc, ic), fn,
          "out must be contiguous fp16 (oc, ic)")
    _check(lib().exl3_reconstruct_t(_ptr(out), _ptr(trellis), ic, oc, K, codebook, _stream(dev)), fn)
    return out


def had_r_128(x: torch.Tensor, out: torch.Tensor | None = None, pre: torch.Tensor | None = None,
              post: torch.Tensor | None = None, scale: float = 1.0) -> torch.Tensor:
    """Row-wise block-128 Hadamard with optional pre/post scales -- ext.had_r_128
    (orcasaq2/ops.py:54, 59).  out may be x (in place)."""
    fn = "exl3_had_r_128"
    dev = _need_gpu(fn, x, out, pre, post)
    _need(x.dtype == torch.float16 and x.is_contiguous(), fn, "x must be contiguous fp16")
    cols = x.shape[-1]
    _need(cols % 128 == 0, fn, f"last dim {cols} is not a multiple of 128")
    rows = x.numel() // cols if cols else 0
    if out is None:
        out = torch.empty_like(x)
    _need(out.dtype == torch.float16 and out.is_contiguous() and out.shape == x.shape, fn,
          "out must match x")
    for name, v in (("pre", pre), ("post", post)):
        if v is not None:
            _vec16(fn, name, v, cols)
    _check(lib().exl3_had_r_128(_ptr(x), _ptr(out), _ptr(pre), _ptr(post), float(scale), rows, cols,
                                _stream(dev)), fn)
    return out


def _shard_table(fn: str, x: torch.Tensor, shards: list[dict], out: torch.Tensor | None, dev):
    """(out, exl3_shard_t array) of a grouped call: the shards' outputs side by side in out
    (rows, sum oc), shard s writing its columns with row stride sum oc."""
    rows, ic = x.shape
    _need(1 <= len(shards) <= MAX_SHARDS, fn, f"{len(shards)} shards")
    total = sum(int(s["oc"]) for s in shards)
    if out is None:
        out = torch.empty((rows, total), dtype=torch.float16, device=dev)
    _need(out.dtype == torch.float16 and out.is_contiguous() and tuple(out.shape) == (rows, total), fn,
          f"out must be contiguous fp16 ({rows}, {total})")
    arr = (Shard * len(shards))()
    col = 0
    for i, s in enumerate(shards):
        oc = int(s["oc"])
        K = check_trellis(fn, s["trellis"], ic, oc, s["K"])
        _vec16(fn, "suh", s["suh"], ic)
        _vec16(fn, "svh", s["svh"], oc)
        arr[i] = Shard(s["trellis"].data_ptr(), s["suh"].data_ptr(), s["svh"].data_ptr(),
                       out.data_ptr() + 2 * col, total, oc, K, int(s["codebook"]))
        col += oc
    return out, arr


def gemv_grouped(x: torch.Tensor, shards: list[dict], out: torch.Tensor | None = None) -> torch.Tensor:
    """Fused decode-GEMV of 1..16 rows through one or more shards that share x; returns
    (rows, sum oc) with the shards' outputs side by side (the concat of
    orcasaq2/config.py:243 written in place).  Each shard: dict(trellis, suh, svh, oc, K,
    codebook)."""
    fn = "exl3_gemv"
    _need(x.dim() == 2, fn, "x must be (rows, ic)")
    rows, ic = x.shape
    dev = _need_gpu(fn, x, out, *[s["trellis"] for s in shards])
    _need(x.dtype == torch.float16 and x.is_contiguous(), fn, "x must be contiguous fp16")
    _need(1 <= rows <= GEMV_MAX_ROWS, fn, f"rows={rows} is not in 1..{GEMV_MAX_ROWS}")
    out, arr = _shard_table(fn, x, shards, out, dev)
    L = lib()
    nbytes = L.exl3_gemv_grouped_workspace_bytes(arr, len(shards), rows, ic)
    ws = gemv_workspace(dev, nbytes)
    _check(L.exl3_gemv_grouped(_ptr(x), arr, len(shards), _ptr(ws), ws.numel(), rows, ic, _stream(dev)), fn)
    return out


def gemv(x, trellis, suh, svh, K, codebook, out=None) -> torch.Tensor:
    """ext.exl3_gemm for rows <= 16 (orcasaq2/ops.py:46-49)."""
    oc = svh.numel()
    return gemv_grouped(x, [dict(trellis=trellis, suh=suh, svh=svh, oc=oc, K=K, codebook=codebook)], out)


def gemm(x: torch.Tensor, trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, K, codebook: int,
         out: torch.Tensor | None = None) -> torch.Tensor:
    """Prefill path: Hadamard of x into a scratch, fused decode-into-MFMA GEMM with the
    output Hadamard in its epilogue (replaces orcasaq2/ops.py:50-59)."""
    fn = "exl3_gemm"
    _need(x.dim() == 2, fn, "x must be (rows, ic)")
    rows, ic = x.shape
    oc = svh.numel()
    dev = _need_gpu(fn, x, trellis, suh, svh, out)
    _need(x.dtype == torch.float16 and x.is_contiguous(), fn, "x must be contiguous fp16")
    K = check_trellis(fn, trellis, ic, oc, K)
    _vec16(fn, "suh", suh, ic)
    _vec16(fn, "svh", svh, oc)
    if out is None:
        out = torch.empty((rows, oc), dtype=torch.float16, device=dev)
    _need(out.dtype == torch.float16 and out.is_contiguous() and tuple(out.shape) == (rows, oc), fn,
          "out must be contiguous fp16 (rows, oc)")
    if rows == 0:
        return out
    L = lib()
    nbytes = L.exl3_gemm_workspace_bytes(rows, ic, oc)
    ws = workspace(dev, nbytes)
    _check(L.exl3_gemm(_ptr(x), _ptr(trellis), _ptr(out), _ptr(suh), _ptr(svh), _ptr(ws), nbytes, rows, ic,
                       oc, K, codebook, _stream(dev)), fn)
    return out


_SCALE_DTYPES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def gemm_grouped(x: torch.Tensor, shards: list[dict], out: torch.Tensor | None = None) -> torch.Tensor:
    """Prefill of several shards that share x in one stream-K launch per codebook: returns
    (rows, sum oc) with the shards' outputs side by side (the concat of
    orcasaq2/config.py:243 written in place).  Each shard: dict(trellis, suh, svh, oc, K,
    codebook)."""
    fn = "exl3_gemm_grouped"
    _need(x.dim() == 2, fn, "x must be (rows, ic)")
    rows, ic = x.shape
    dev = _need_gpu(fn, x, out, *[s["trellis"] for s in shards])
    _need(x.dtype == torch.float16 and x.is_contiguous(), fn, "x must be contiguous fp16")
    out, arr = _shard_table(fn, x, shards, out, dev)
    if rows == 0:
        return out
    L = lib()
    nbytes = L.exl3_gemm_grouped_workspace_bytes(arr, len(shards), rows, ic)
    ws = workspace(dev, nbytes)
    _check(L.exl3_gemm_grouped(_ptr(x), arr, len(shards), _ptr(ws), nbytes, rows, ic, _stream(dev)), fn)
    return out


def embed_int8(table: torch.Tensor, scales: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
    """table[ids].to(scales.dtype) * scales[ids] (orcasaq2/heads.py:66-67); output shape
    ids.shape + (dim,)."""
    fn = "exl3_embed_int8_gather"
    dev = _need_gpu(fn, table, scales, ids)
    _need(table.dtype == torch.int8 and table.dim() == 2 and table.is_contiguous(), fn,
          "table must be contiguous int8 (vocab, dim)")
    vocab, dim = table.shape
    _need(dim % 4 == 0, fn, f"dim={dim} must be a multiple of 4")
    _need(scales.dtype in _SCALE_DTYPES, fn, f"scales dtype {scales.dtype}")
    _need(scales.is_contiguous() and scales.numel() == vocab, fn, "scales must be contiguous (vocab) or (vocab, 1)")
    idx = ids.reshape(-1)
    if idx.dtype != torch.int64 or not idx.is_contiguous():
        idx = idx.to(torch.int64).contiguous()
    out = torch.empty((idx.numel(), dim), dtype=scales.dtype, device=dev)
    _check(lib().exl3_embed_int8_gather(_ptr(table), _ptr(scales), _SCALE_DTYPES[scales.dtype], _ptr(idx),
                                        _ptr(out), idx.numel(), vocab, dim, _stream(dev)), fn)
    return out.reshape(*ids.shape, dim)


def topk(x: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The k largest entries of each row of fp16 x (..., n), e.g. the output head's logits:
    values (..., k) fp16, largest first, equal values by smaller column, every NaN above
    +inf and -0 equal to +0, and their columns (..., k) int64 (exl3_topk).  k = 1 is greedy
    decoding's argmax.  A row layout the kernel cannot read (column stride != 1, row stride
    not a multiple of 8, base not 16-byte aligned) is first copied to one it can."""
    fn = "exl3_topk"
    dev = _need_gpu(fn, x)
    _need(x.dtype == torch.float16, fn, f"x must be fp16, got {x.dtype}")
    _need(x.dim() >= 1 and x.shape[-1] >= 1, fn, f"x must have a non-empty last dim, got {tuple(x.shape)}")
    n = x.shape[-1]
    _need(1 <= k <= TOPK_MAX_K and k <= n <= TOPK_MAX_N, fn,
          f"k={k} n={n} (need 1 <= k <= {TOPK_MAX_K}, k <= n <= {TOPK_MAX_N})")
    x2 = x.reshape(-1, n)
    rows = x2.shape[0]
    _need(rows <= 65535, fn, f"{rows} rows (at most 65535)")
    ld = x2.stride(0) if rows > 1 else (n + 7) // 8 * 8
    readable = x2.stride(-1) == 1 and ld % 8 == 0 and ld >= n and x2.data_ptr() % 16 == 0
    if readable:
        # the kernel may read each row up to the next multiple of 8 columns, which must lie
        # inside x's storage for the last row too
        end = x2.storage_offset() + (rows - 1) * ld + (n + 7) // 8 * 8
        readable = end <= x2.untyped_storage().nbytes() // 2
    if not readable:
        ld = (n + 7) // 8 * 8
        xp = torch.empty((rows, ld), dtype=torch.float16, device=dev)
        xp[:, :n].copy_(x2)
        x2 = xp
    values = torch.empty((rows, k), dtype=torch.float16, device=dev)
    idx = torch.empty((rows, k), dtype=torch.int64, device=dev)
    L = lib()
    ws = workspace(dev, L.exl3_topk_workspace_bytes(rows, n, k))
    _check(L.exl3_topk(_ptr(x2), rows, n, ld, k, _ptr(values), _ptr(idx), _ptr(ws), ws.numel(), _stream(dev)), fn)
    return values.reshape(*x.shape[:-1], k), idx.reshape(*x.shape[:-1], k)


def argmax(x: torch.Tensor) -> torch.Tensor:
    """Column of each row's largest entry of fp16 x (..., n) (the first one of equal maxima,
    as torch.argmax): topk with k = 1."""
    return topk(x, 1)[1][..., 0]
