"""CPU oracle for the EXL3 trellis linear path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker (or, for cpu_baseline, as the timed CPU restatement of
the reference's path).  The product (orcasaq2/ and libexl3hip.so) never calls it.

The integer/byte work (trellis decode) is the C restatement in exl3_oracle.c, loaded
with ctypes and built by the Makefile next to it.  The floating-point algebra is numpy
fp64, restating the reference:

  * H = Sylvester H128 / sqrt(128) along the last dim ..... orcasaq2/__init__.py:33-46
  * dense deploy weight (diag(suh) H W_q H diag(svh))^T .... orcasaq2/__init__.py:49-61
  * fused order y = H(H(x * suh) W_q) * svh, fp16 A_had .... orcasaq2/ops.py:44-59
  * activations cast to fp16, concat of shards ............ orcasaq2/config.py:232-245
  * int8 embedding: q[ids] * s[ids] ........................ orcasaq2/heads.py:61-67
  * top-k / argmax of the head's logits ..................... no reference counterpart (vLLM's
    sampler reduces the logits of orcasaq2/config.py:128-132); restates torch.argmax's order
    (first maximal column, NaN above every number, -0 == +0) with ties by smaller column
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libexl3oracle.so")
_lib = None
_lock = threading.Lock()

CB_3INST = 0
CB_MCG = 1


def build(force: bool = False) -> str:
    """Compile exl3_oracle.c with the Makefile in this directory; returns the .so path."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []), check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    with _lock:
        if _lib is None:
            build()
            L = ctypes.CDLL(_LIB_PATH)
            u16p = ctypes.POINTER(ctypes.c_uint16)
            f64p = ctypes.POINTER(ctypes.c_double)
            L.exl3o_half_to_float.restype = ctypes.c_float
            L.exl3o_half_to_float.argtypes = [ctypes.c_uint16]
            L.exl3o_double_to_half.restype = ctypes.c_uint16
            L.exl3o_double_to_half.argtypes = [ctypes.c_double]
            L.exl3o_state.restype = ctypes.c_uint32
            L.exl3o_state.argtypes = [u16p, ctypes.c_int, ctypes.c_int]
            L.exl3o_perm.restype = ctypes.c_int
            L.exl3o_perm.argtypes = [ctypes.c_int]
            L.exl3o_codebook.restype = ctypes.c_uint16
            L.exl3o_codebook.argtypes = [ctypes.c_uint32, ctypes.c_int]
            L.exl3o_codebook_table.restype = None
            L.exl3o_codebook_table.argtypes = [u16p, ctypes.c_int]
            L.exl3o_decode_tile.restype = None
            L.exl3o_decode_tile.argtypes = [u16p, u16p, ctypes.c_int, ctypes.c_int]
            L.exl3o_reconstruct.restype = None
            L.exl3o_reconstruct.argtypes = [u16p, u16p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_int]
            L.exl3o_had128.restype = None
            L.exl3o_had128.argtypes = [f64p, ctypes.c_long, ctypes.c_int]
            _lib = L
    return _lib


def _u16p(a: np.ndarray):
    assert a.dtype == np.uint16 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


def as_u16(a) -> np.ndarray:
    """int16/uint16 array or torch tensor -> contiguous uint16 numpy view of the bits."""
    if hasattr(a, "detach"):
        a = a.detach().cpu().contiguous().numpy()
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16 or a.dtype == np.int16:
        return a.view(np.uint16)
    assert a.dtype == np.uint16, a.dtype
    return a


# ---------------------------------------------------------------- decode

def codebook_table(cb: int = CB_3INST) -> np.ndarray:
    out = np.empty(65536, np.uint16)
    lib().exl3o_codebook_table(_u16p(out), cb)
    return out


def codebook_value(s: int, cb: int = CB_3INST) -> int:
    return int(lib().exl3o_codebook(s, cb))


def states(tile, K: int) -> np.ndarray:
    """All 256 states of one tile (16K words)."""
    t = as_u16(tile).reshape(-1)
    assert t.size == 16 * K
    return np.array([lib().exl3o_state(_u16p(t), K, i) for i in range(256)], np.uint32)


def perm() -> np.ndarray:
    """perm[t] = row*16 + col of stream position t inside a 16x16 tile."""
    return np.array([lib().exl3o_perm(t) for t in range(256)], np.int64)


def decode_tile(tile, K: int, cb: int = CB_3INST) -> np.ndarray:
    t = as_u16(tile).reshape(-1)
    out = np.empty(256, np.uint16)
    lib().exl3o_decode_tile(_u16p(out), _u16p(t), K, cb)
    return out.reshape(16, 16)


def reconstruct(trellis, K: int | None = None, cb: int = CB_3INST, nthreads: int = 0) -> np.ndarray:
    """W_q (ic, oc) as uint16 fp16 bits, from trellis (ic/16, oc/16, 16K)."""
    tr = as_u16(trellis)
    assert tr.ndim == 3
    if K is None:
        K = tr.shape[2] // 16
    assert tr.shape[2] == 16 * K
    ic, oc = tr.shape[0] * 16, tr.shape[1] * 16
    W = np.empty((ic, oc), np.uint16)
    lib().exl3o_reconstruct(_u16p(W), _u16p(tr), ic, oc, K, cb, nthreads)
    return W


def reconstruct_f16(trellis, K=None, cb=CB_3INST, nthreads=0) -> np.ndarray:
    return reconstruct(trellis, K, cb, nthreads).view(np.float16)


# ---------------------------------------------------------------- fp algebra (fp64)

def double_to_half(d: float) -> int:
    return int(lib().exl3o_double_to_half(float(d)))


def had_matrix(n: int = 128) -> np.ndarray:
    """Sylvester H_n / sqrt(n) (orcasaq2/__init__.py:33-40)."""
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h / np.sqrt(n)


def had128(x: np.ndarray) -> np.ndarray:
    """Blockwise H128 along the last dim, fp64, via the C fast transform."""
    a = np.array(x, dtype=np.float64, copy=True, order="C")
    cols = a.shape[-1]
    assert cols % 128 == 0
    rows = a.size // cols
    lib().exl3o_had128(a.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), rows, cols)
    return a


def had_r_128(x, pre=None, post=None, scale: float = 1.0) -> np.ndarray:
    """fp64 value of ((x * pre) H) * post * scale, blockwise along the last dim
    (the ext.had_r_128 call at orcasaq2/ops.py:54,59)."""
    a = np.asarray(x, dtype=np.float64)
    if pre is not None:
        a = a * np.asarray(pre, dtype=np.float64)
    a = had128(a)
    if post is not None:
        a = a * np.asarray(post, dtype=np.float64)
    return a * scale


def a_had(x, suh) -> np.ndarray:
    """fp16(H(x * suh)): the fp16 activation scratch of the fused path (orcasaq2/ops.py:49)."""
    return had_r_128(np.asarray(x, np.float16), np.asarray(suh, np.float16)).astype(np.float16)


def shard_gemm_ref(x, trellis, suh, svh, K=None, cb=CB_3INST, W=None) -> np.ndarray:
    """fp64 y = H(fp16(H(x*suh)) @ W_q) * svh  (orcasaq2/ops.py:44-59).  x (rows, ic) fp16."""
    x = np.asarray(x, np.float16)
    if W is None:
        W = reconstruct_f16(trellis, K, cb)
    ah = a_had(x, suh).astype(np.float64)
    y = ah @ W.astype(np.float64)
    return had_r_128(y, post=np.asarray(svh, np.float16))


def deploy_weight(W_q_f16, suh, svh) -> np.ndarray:
    """(diag(suh) H W_q H diag(svh))^T in fp64 (orcasaq2/__init__.py:58-61 before .half())."""
    w = np.asarray(W_q_f16, np.float64)
    w = had128(w.T).T * np.asarray(suh, np.float64)[:, None]
    w = had128(w) * np.asarray(svh, np.float64)[None, :]
    return w.T.copy()


def rel_err_rows(y, y_ref) -> np.ndarray:
    """Per-row ||y - y_ref||_2 / ||y_ref||_2."""
    y = np.asarray(y, np.float64).reshape(-1, np.shape(y_ref)[-1])
    r = np.asarray(y_ref, np.float64).reshape(y.shape)
    return np.linalg.norm(y - r, axis=1) / np.maximum(np.linalg.norm(r, axis=1), 1e-300)


def embed_int8_ref(q, s, ids) -> np.ndarray:
    """q[ids].astype(s.dtype) * s[ids] (orcasaq2/heads.py:66-67), computed in the scale dtype."""
    q = np.asarray(q)
    s = np.asarray(s).reshape(-1, 1)
    ids = np.asarray(ids).reshape(-1)
    return (q[ids].astype(np.float32) * s[ids].astype(np.float32)).astype(s.dtype)


def fp16_order_key(x) -> np.ndarray:
    """Unsigned order key of fp16 values: larger for larger values, -0 and +0 alike, every
    NaN above +inf (torch.argmax's order)."""
    h = np.asarray(x, np.float16).view(np.uint16).astype(np.int64)
    mag = h & 0x7FFF
    key = np.where(h & 0x8000, (~h) & 0xFFFF, h | 0x8000)
    key = np.where(mag == 0, 0x8000, key)
    return np.where(mag > 0x7C00, 0xFFFF, key)


def topk_rows(x, k: int):
    """The k largest entries of each row of fp16 x (rows, n): values (rows, k) fp16 (the
    entries' own bits) largest first, equal values by smaller column, and their columns
    (rows, k) int64."""
    x = np.asarray(x, np.float16).reshape(-1, np.shape(x)[-1])
    key = fp16_order_key(x)
    cols = np.arange(x.shape[1])
    idx = np.empty((x.shape[0], k), np.int64)
    for r in range(x.shape[0]):
        idx[r] = np.lexsort((cols, -key[r]))[:k]     # primary: key descending; then column
    return np.take_along_axis(x, idx, axis=1), idx
