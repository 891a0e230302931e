"""exl3_gemv_grouped_static, the GEMV entry point that allocates nothing (its scratch is a
file-scope device array of the library), called through the C ABI against
exl3_gemv_grouped with a caller workspace on the same inputs.

The kernels are the same and their split reductions are exact (fixed-point sums at 1..4
rows) or run in a fixed order (5..16 rows), so the two outputs must agree bit for bit; each
call is also checked against the fp64 oracle at the GEMV bar (per-row relative L2 error <=
1e-3).  Two calls in a row on one stream, the second smaller, cover the reuse of the array
(its accumulator area, zero when the library loads, is left zero by every call) at 1, 4 and
16 rows; 16 rows on a lm_head-width shard covers the largest scratch the array holds; a
captured-and-replayed call covers a caller that cannot allocate because it is under graph
capture.  The size limit is a host check, tested without a GPU call.
"""
import ctypes

import numpy as np
import pytest
import torch

from orcasaq2 import synthetic as syn

REL_TOL = 1e-3
P = ctypes.c_void_p


def _table(native, shards, out, total):
    arr = (native.Shard * len(shards))()
    col = 0
    for i, s in enumerate(shards):
        arr[i] = native.Shard(s["trellis"].data_ptr(), s["suh"].data_ptr(), s["svh"].data_ptr(),
                              out.data_ptr() + 2 * col, total, s["oc"], s["K"], 0)
        col += s["oc"]
    return arr


def _case(ic, ocs_ks, rows, seed):
    lins = [syn.linear(ic, oc, K, seed=seed + i) for i, (oc, K) in enumerate(ocs_ks)]
    x = syn.activations(rows, ic, torch.Generator().manual_seed(seed))
    return lins, x


def _run_both(native, lins, x):
    """(static output, workspace output) of one grouped call on the current stream."""
    dev = torch.device("cuda", 0)
    L = native.lib()
    d = [{k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in l.items()} for l in lins]
    rows, ic = x.shape
    total = sum(l["oc"] for l in lins)
    xd = x.to(dev)
    stream = P(torch.cuda.current_stream(dev).cuda_stream)
    y_static = torch.full((rows, total), float("nan"), dtype=torch.float16, device=dev)
    arr = _table(native, d, y_static, total)
    rc = L.exl3_gemv_grouped_static(P(xd.data_ptr()), arr, len(d), rows, ic, stream)
    assert rc == 0, L.exl3_last_error().decode()
    y_ws = torch.full((rows, total), float("nan"), dtype=torch.float16, device=dev)
    arr2 = _table(native, d, y_ws, total)
    nbytes = L.exl3_gemv_grouped_workspace_bytes(arr2, len(d), rows, ic)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    rc = L.exl3_gemv_grouped(P(xd.data_ptr()), arr2, len(d), P(ws.data_ptr()), nbytes, rows, ic, stream)
    assert rc == 0, L.exl3_last_error().decode()
    torch.cuda.synchronize()
    return y_static, y_ws, d, xd


def _check_oracle(oracle, y, x, lins):
    col = 0
    for l in lins:
        ref = oracle.shard_gemm_ref(x.numpy(), l["trellis"], l["suh"].numpy(), l["svh"].numpy(), l["K"], 0)
        err = oracle.rel_err_rows(y[:, col:col + l["oc"]].cpu().numpy(), ref)
        assert err.max() <= REL_TOL, (l["oc"], l["K"], err.max())
        col += l["oc"]


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 4, 16])
def test_static_matches_workspace_twice_second_smaller(native, oracle, rows):
    # first: the 27B qkv (three shards, K = 4, 5, 5); second: one small shard
    for ic, ocs_ks, seed in ((syn.HIDDEN, [(syn.Q_OUT, 4), (syn.KV_OUT, 5), (syn.KV_OUT, 5)], 11),
                             (1024, [(512, 3)], 12)):
        lins, x = _case(ic, ocs_ks, rows, seed)
        print(f"static gemv: rows={rows} ic={ic} shards={ocs_ks}", flush=True)
        y_static, y_ws, _, _ = _run_both(native, lins, x)
        assert not torch.isnan(y_static).any()
        assert torch.equal(y_static, y_ws)
        _check_oracle(oracle, y_static, x, lins)


@pytest.mark.gpu
def test_static_lm_head_width_at_16_rows(native, oracle):
    """The K=6 lm_head shape (5120 -> 151936) at 16 rows: the 5..16-row path's fragments and
    slots for 1187 column groups, the most scratch a 27B call asks of the array.  Static and
    workspace outputs agree bit for bit; two column groups are checked against the oracle."""
    dev = torch.device("cuda", 0)
    L = native.lib()
    g = torch.Generator(device=dev).manual_seed(31)
    lin = syn.linear_gpu(syn.HIDDEN, syn.VOCAB, 6, g, dev)
    x = syn.activations(16, syn.HIDDEN, torch.Generator().manual_seed(31))
    xd = x.to(dev)
    stream = P(torch.cuda.current_stream(dev).cuda_stream)
    print("static gemv: rows=16 lm_head 5120->151936 K=6", flush=True)
    y_static = torch.full((16, syn.VOCAB), float("nan"), dtype=torch.float16, device=dev)
    arr = _table(native, [lin], y_static, syn.VOCAB)
    assert L.exl3_gemv_grouped_workspace_bytes(arr, 1, 16, syn.HIDDEN) <= (24 << 20)
    rc = L.exl3_gemv_grouped_static(P(xd.data_ptr()), arr, 1, 16, syn.HIDDEN, stream)
    assert rc == 0, L.exl3_last_error().decode()
    y_ws = torch.full_like(y_static, float("nan"))
    arr2 = _table(native, [lin], y_ws, syn.VOCAB)
    nbytes = L.exl3_gemv_grouped_workspace_bytes(arr2, 1, 16, syn.HIDDEN)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    rc = L.exl3_gemv_grouped(P(xd.data_ptr()), arr2, 1, P(ws.data_ptr()), nbytes, 16, syn.HIDDEN, stream)
    assert rc == 0, L.exl3_last_error().decode()
    torch.cuda.synchronize()
    assert not torch.isnan(y_static).any()
    assert torch.equal(y_static, y_ws)
    for cg in (0, 1000):
        sl = slice(cg * 128, (cg + 1) * 128)
        t = lin["trellis"][:, cg * 8:(cg + 1) * 8].contiguous().cpu()
        ref = oracle.shard_gemm_ref(x.numpy(), t, lin["suh"].cpu().numpy(), lin["svh"][sl].cpu().numpy(), 6, 0)
        err = oracle.rel_err_rows(y_static[:, sl].cpu().numpy(), ref)
        assert err.max() <= REL_TOL, (cg, err.max())


@pytest.mark.gpu
def test_static_under_graph_capture(native, oracle):
    """Captured on a side stream and replayed three times, eager calls of another size in
    between: every replay equals the eager workspace result."""
    dev = torch.device("cuda", 0)
    L = native.lib()
    lins, x = _case(syn.INTERMEDIATE, [(syn.HIDDEN, 5)], 1, 21)
    print("static gemv under capture: down_proj 17408->5120 K=5", flush=True)
    ref_static, ref_ws, d, xd = _run_both(native, lins, x)
    assert torch.equal(ref_static, ref_ws)
    other, xo = _case(2048, [(1024, 2)], 1, 22)
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    y = torch.zeros_like(ref_static)
    arr = _table(native, d, y, syn.HIDDEN)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            rc = L.exl3_gemv_grouped_static(P(xd.data_ptr()), arr, 1, 1, syn.INTERMEDIATE,
                                            P(s.cuda_stream))
            assert rc == 0, L.exl3_last_error().decode()
    torch.cuda.current_stream(dev).wait_stream(s)
    for _ in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref_ws)
        o_static, o_ws, _, _ = _run_both(native, other, xo)   # eager work on the same array between replays
        assert torch.equal(o_static, o_ws)
    _check_oracle(oracle, y, x, lins)


def test_static_rejects_calls_above_its_scratch(native):
    """Host check only (no GPU call): a grouped call whose workspace exceeds the array."""
    L = native.lib()
    arr = (native.Shard * 4)()
    for i in range(4):
        arr[i] = native.Shard(0x10000, 0x10000, 0x10000, 0x10000, 4 * syn.INTERMEDIATE, syn.INTERMEDIATE, 4, 0)
    need = L.exl3_gemv_grouped_workspace_bytes(arr, 4, 16, syn.HIDDEN)
    assert need > 24 << 20
    rc = L.exl3_gemv_grouped_static(P(0x10000), arr, 4, 16, syn.HIDDEN, None)
    assert rc == 3
    msg = L.exl3_last_error().decode()
    assert "static" in msg and str(need) in msg
    assert L.exl3_gemv_grouped_static(P(0x10000), arr, 0, 1, syn.HIDDEN, None) == 1
