"""The EXL3 shard GEMM as PyTorch custom ops (same names and schema as the reference's
orcasaq2/ops.py:37-66), backed by the gfx950 HIP library through its C ABI.

A custom op keeps the shard opaque to Dynamo -- one graph node with a known output shape
(the register_fake below) -- so a torch.compile'd model compiles around it, and its
kernels only enqueue on the current stream, so it can be captured in a HIP graph.

Dispatch on the number of activation rows (reference: orcasaq2/ops.py:25, 46-59):
  * rows <= 16            fused decode-GEMV (exl3_gemv): packed words streamed from HBM and
                          decoded in registers, never stored; rows 1..4: one persistent kernel
                          (MFMA multiply-accumulate; a column group split over workgroups is
                          summed in fixed point in the workspace and finished by the workgroup
                          whose add completes it); rows 5..16, and 2..4-row shards too large for
                          that kernel's tables: the same decode on 4 x 2-tile units, one MFMA
                          serving all rows; output Hadamard and svh at the end;
  * 16 < rows <= GEMM_MAX_ROWS
                          fused decode-GEMM (exl3_gemm): Hadamard pass over x, then stream-K
                          tiles decoded straight into MFMA operands, output Hadamard in the
                          epilogue; a fused layer's shards together (shards_gemm) -- except a
                          single shard with 4096 <= ic < 8192 above 64 rows where the
                          reconstruct branch measured faster (_fused_gemm_faster);
  * rows > GEMM_MAX_ROWS  the reference's reconstruct branch: had_r_128(x, suh), dense W_q
                          (decoded transposed, (oc, ic)) into a scratch freed on exit, library
                          fp16 transposed-B GEMM, had_r_128(y, svh) -- except, while the row
                          knob is at its default, 8192+ inputs up to WIDE_FUSED_MAX_ROWS rows
                          (faster fused but at 2048 rows, kept fused there for no dense W_q)
                          and 4096..8191 inputs with at least twice as many outputs in
                          WIDE_OUT_FUSED_ROWS, where the fused kernel measured faster
                          (_fused_gemm_faster); a fused layer whose shards all route fused
                          runs them as one grouped launch (shards_gemm).
The op is registered for the "cuda" device type (ROCm) only: there is no CPU path.
"""

import os

import torch
from torch import Tensor

from . import _native

# Rows at or below which the fused kernels are used (the reference's default and env knob,
# orcasaq2/ops.py:22-25).  Above it the dense W_q is rebuilt once and a library GEMM runs --
# except, while the knob is left at its default, for the shapes where the fused kernel
# measured faster (_fused_gemm_faster).  Setting the knob makes it the hard switch of the
# reference.
GEMM_MAX_ROWS = int(os.environ.get("ORCA_EXL3_GEMM_MAX_ROWS", "144"))
GEMM_MAX_ROWS_SET = "ORCA_EXL3_GEMM_MAX_ROWS" in os.environ
WIDE_FUSED_MAX_ROWS = 2560           # 8192+ inputs: fused up to here
WIDE_OUT_FUSED_ROWS = (1536, 3072)   # 4096..8191 inputs, oc >= 2 ic: fused in (lo, hi] too
GEMV_MAX_ROWS = _native.GEMV_MAX_ROWS


def exl3_K(trellis: Tensor):
    """Bits per weight = trellis.shape[-1] / 16 (16-weight steps per tile row).  Integers
    stay int; the mul1 half rates (1.5/2.5/3.5: 24/40/56 words per tile) stay float, as in
    orcasaq2/ops.py:28-34.  The HIP kernels accept integer K in 1..8 only."""
    k = trellis.shape[-1] / 16
    return int(k) if float(k).is_integer() else k


def _fused_gemm_faster(rows: int, ic: int, oc: int) -> bool:
    """Whether the fused decode-GEMM beats the reconstruct branch for one shard of `rows` >
    GEMV_MAX_ROWS rows.  Measured on MI355X at settled clocks (us per call, HIP graph, fused /
    reconstruct branch; the branch's library GEMM is far from monotone in the row count):
      17408 -> 5120:  144: 116 / 176, 256: 118 / 225, 1024: 221 / 308, 1536: 308 / 430,
                      2048: 388 / 370, 2560: 499 / 652, 3072: 589 / 487, 4096: 732 / 701;
      5120 -> 17408:  64: 60 / 77, 128: 80 / 83, 144: 112 / 95, 384: 143 / 120,
                      1024: 220 / 232, 1536: 300 / 285, 2048: 390 / 478, 2560: 478 / 569,
                      3072: 592 / 644, 4096: 742 / 685;
      5120 -> 6144:   40: 39 / 45, 64: 46 / 46, 80: 60 / 49, 144: 71 / 52, 2048: 166 / 142.
    So: 8192+ inputs fused up to WIDE_FUSED_MAX_ROWS -- at 2048 rows too, 5% slower than the
    reconstruct branch but with no dense W_q (the branch writes and reads a 2 ic oc-byte
    transient, 178 MB for down_proj) and no library GEMM;
    4096..8191 inputs fused up to 64 rows, and with oc >= 2 ic up to 128 rows and within
    WIDE_OUT_FUSED_ROWS; narrower inputs (unmeasured below 4096) fused up to GEMM_MAX_ROWS."""
    if ic >= 8192:
        return rows <= WIDE_FUSED_MAX_ROWS
    if ic < 4096:
        return True
    if oc >= 2 * ic:
        lo, hi = WIDE_OUT_FUSED_ROWS
        return rows <= 128 or lo < rows <= hi
    return rows <= 64


def _fused_route(rows: int, ic: int, oc: int) -> bool:
    """The fused decode-GEMM for rows > GEMV_MAX_ROWS: within GEMM_MAX_ROWS where it measured
    faster; beyond it, while the knob is at its default, for inputs of 4096 or more where it
    measured faster (narrower inputs keep the reference's switch)."""
    if rows <= GEMM_MAX_ROWS:
        return _fused_gemm_faster(rows, ic, oc)
    return not GEMM_MAX_ROWS_SET and ic >= 4096 and _fused_gemm_faster(rows, ic, oc)


def _shard_gemm_impl(x: Tensor, trellis: Tensor, suh: Tensor, svh: Tensor, oc: int, k: float,
                     mcg: bool, mul1: bool) -> Tensor:
    cb = _native.codebook_id(mcg, mul1)
    if float(k).is_integer():
        k = int(k)
    rows, ic = x.shape
    if rows == 0:
        return x.new_empty((0, oc), dtype=torch.half)
    if rows <= GEMV_MAX_ROWS:
        return _native.gemv(x, trellis, suh, svh, k, cb)
    if _fused_route(rows, ic, oc):
        return _native.gemm(x, trellis, suh, svh, k, cb)
    return _reconstruct_branch(x, trellis, suh, svh, k, cb)


def _reconstruct_branch(x: Tensor, trellis: Tensor, suh: Tensor, svh: Tensor, k, cb: int) -> Tensor:
    """The reference's prefill branch (orcasaq2/ops.py:50-59): had_r_128, reconstruct, a dense
    GEMM, had_r_128.  The dense W_q lives only for the duration of the call, decoded as W_q^T
    (oc, ic) so the library runs its transposed-B GEMM (measured 15-20% faster than x @ W_q at
    512-4096 rows on MI355X)."""
    xh = _native.had_r_128(x, pre=suh)
    wt = _native.reconstruct_t(trellis, k, cb)
    y = torch.nn.functional.linear(xh, wt)
    del wt, xh
    return _native.had_r_128(y, out=y, post=svh)


@torch.library.custom_op("orcasaq2::shard_gemm", mutates_args=(), device_types="cuda")
def shard_gemm(x: Tensor, trellis: Tensor, suh: Tensor, svh: Tensor,
               oc: int, k: float, mcg: bool, mul1: bool) -> Tensor:
    return _shard_gemm_impl(x, trellis, suh, svh, oc, k, mcg, mul1)


@shard_gemm.register_fake
def _shard_gemm_fake(x: Tensor, trellis: Tensor, suh: Tensor, svh: Tensor,
                     oc: int, k: float, mcg: bool, mul1: bool) -> Tensor:
    return x.new_empty((x.shape[0], oc), dtype=torch.half)


@torch.library.custom_op("orcasaq2::shards_gemv", mutates_args=(), device_types="cuda")
def shards_gemv(x: Tensor, trellis: list[Tensor], suh: list[Tensor], svh: list[Tensor],
                oc: list[int], k: list[float], mcg: list[bool], mul1: list[bool]) -> Tensor:
    """All shards of a fused layer (q/k/v, gate/up) for rows <= 16 in as few launches as
    there are distinct (K, codebook); outputs are written side by side, which is the
    per-shard loop + torch.cat of orcasaq2/config.py:237-243 without the copy."""
    shards = [dict(trellis=t, suh=a, svh=b, oc=o, K=kk, codebook=_native.codebook_id(m, m1))
              for t, a, b, o, kk, m, m1 in zip(trellis, suh, svh, oc, k, mcg, mul1)]
    return _native.gemv_grouped(x, shards)


@shards_gemv.register_fake
def _shards_gemv_fake(x, trellis, suh, svh, oc, k, mcg, mul1) -> Tensor:
    return x.new_empty((x.shape[0], sum(oc)), dtype=torch.half)


@torch.library.custom_op("orcasaq2::shards_gemm", mutates_args=(), device_types="cuda")
def shards_gemm(x: Tensor, trellis: list[Tensor], suh: list[Tensor], svh: list[Tensor],
                oc: list[int], k: list[float], mcg: list[bool], mul1: list[bool]) -> Tensor:
    """All shards of a fused layer for rows > 16 (up to GEMM_MAX_ROWS, and above it when every
    shard routes fused): one set-up kernel (each shard's Hadamard pass) and one stream-K
    launch per codebook (per K with 256-row tiles) for all of them, outputs side by side --
    the per-shard shard_gemm loop + torch.cat of orcasaq2/config.py:237-243 with one launch
    tail instead of one per shard."""
    shards = [dict(trellis=t, suh=a, svh=b, oc=o, K=kk, codebook=_native.codebook_id(m, m1))
              for t, a, b, o, kk, m, m1 in zip(trellis, suh, svh, oc, k, mcg, mul1)]
    return _native.gemm_grouped(x, shards)


@shards_gemm.register_fake
def _shards_gemm_fake(x, trellis, suh, svh, oc, k, mcg, mul1) -> Tensor:
    return x.new_empty((x.shape[0], sum(oc)), dtype=torch.half)
