"""GPU parity of the whole config-4 token the benchmark times: the seeded 64-layer
Qwen-27B-shaped linear stack of orcasaq2.synthetic.stack_gpu (the bench's own tensors), the
int8 embedding gather in front, the K=6 lm_head and its argmax behind.

The token is the bench's (bench.py stack_bench): each projection reads what the one before it
produced (o_proj the q columns of qkv, gate/up the o_proj output, down_proj the gate columns,
the next layer the down_proj output, the lm_head the last one), here with one output buffer
per layer so every projection's input is still there afterwards.  It is captured once into a
HIP graph and replayed once; then all 64 x 7 projections are checked on two 128-output column
groups each (the first and one drawn per projection) against the fp64 oracle on the input
that projection actually read, the lm_head on four column groups, the gather bit for bit and
the argmax against torch.argmax of the logits.  A second replay must reproduce the first.

Bar: per-row relative L2 error <= 1e-3 (orcasaq2/ops.py:44-59 restated in oracle/oracle.py;
apply's shard order and concat, orcasaq2/config.py:228-245).
"""
import random

import numpy as np
import pytest
import torch

from orcasaq2 import synthetic as syn

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
D = torch.device("cuda", 0)


def _check_groups(oracle, y, x, lin, groups, what):
    """y (1, oc) against the oracle on column groups `groups` of lin (on the GPU)."""
    xs = np.asarray(x.detach().cpu().numpy(), np.float16)
    suh = lin["suh"].cpu().numpy()
    for cg in groups:
        sl = slice(cg * 128, (cg + 1) * 128)
        t = lin["trellis"][:, cg * 8:(cg + 1) * 8].contiguous().cpu()
        ref = oracle.shard_gemm_ref(xs, t, suh, lin["svh"][sl].cpu().numpy(), lin["K"], 0)
        err = oracle.rel_err_rows(y[:, sl].detach().cpu().numpy(), ref)
        assert err.max() <= REL_TOL, (what, cg, float(err.max()))


def test_config4_full_stack_token(native, oracle):
    st = syn.stack_gpu(D)
    layers, head, table, scales = st["layers"], st["head"], st["table"], st["scales"]
    n = len(layers)
    assert n == syn.LAYERS
    H, Q, KV, I = syn.HIDDEN, syn.Q_OUT, syn.KV_OUT, syn.INTERMEDIATE
    ids = torch.tensor([12345], device=D)
    ids0 = ids.clone()
    h0 = torch.empty(1, H, dtype=torch.half, device=D)
    y_qkv = [torch.empty(1, Q + 2 * KV, dtype=torch.half, device=D) for _ in range(n)]
    y_o = [torch.empty(1, H, dtype=torch.half, device=D) for _ in range(n)]
    y_gu = [torch.empty(1, 2 * I, dtype=torch.half, device=D) for _ in range(n)]
    y_d = [torch.empty(1, H, dtype=torch.half, device=D) for _ in range(n)]
    logits = torch.empty(1, syn.VOCAB, dtype=torch.half, device=D)
    nxt = torch.empty(1, dtype=torch.long, device=D)

    def token():
        h0.copy_(native.embed_int8(table, scales, ids))
        h = h0
        for li, L in enumerate(layers):
            native.gemv_grouped(h, [L["q"], L["k"], L["v"]], out=y_qkv[li])
            native.gemv_grouped(y_qkv[li][:, :Q], [L["o"]], out=y_o[li])
            native.gemv_grouped(y_o[li], [L["gate"], L["up"]], out=y_gu[li])
            native.gemv_grouped(y_gu[li][:, :I], [L["down"]], out=y_d[li])
            h = y_d[li]
        native.gemv_grouped(h, [head], out=logits)
        nxt.copy_(native.argmax(logits))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        token()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        token()
    outs = [h0, logits] + y_qkv + y_o + y_gu + y_d
    for t in outs:
        t.fill_(float("nan"))
    torch.cuda.synchronize()
    print("config-4 stack: first replay", flush=True)
    with torch.cuda.stream(s):
        graph.replay()
    torch.cuda.synchronize()
    first = [t.clone() for t in outs] + [nxt.clone()]

    assert torch.equal(h0, table[ids0].half() * scales[ids0])
    rng = random.Random(4)

    def groups(oc):
        return (0, rng.randrange(1, oc // 128))

    x = h0
    for li, L in enumerate(layers):
        col = 0
        for name in ("q", "k", "v"):
            oc = L[name]["oc"]
            _check_groups(oracle, y_qkv[li][:, col:col + oc], x, L[name], groups(oc), (li, name))
            col += oc
        _check_groups(oracle, y_o[li], y_qkv[li][:, :Q], L["o"], groups(H), (li, "o"))
        _check_groups(oracle, y_gu[li][:, :I], y_o[li], L["gate"], groups(I), (li, "gate"))
        _check_groups(oracle, y_gu[li][:, I:], y_o[li], L["up"], groups(I), (li, "up"))
        _check_groups(oracle, y_d[li], y_gu[li][:, :I], L["down"], groups(H), (li, "down"))
        x = y_d[li]
    _check_groups(oracle, logits, x, head, (0, 1, 593, syn.VOCAB // 128 - 1), "lm_head")
    assert bool(torch.isfinite(logits).all())
    assert torch.equal(nxt, torch.argmax(logits, dim=1))

    print("config-4 stack: second replay", flush=True)
    with torch.cuda.stream(s):
        graph.replay()
    torch.cuda.synchronize()
    for a, b in zip(first, outs + [nxt]):
        assert torch.equal(a, b)
    del graph, st, layers, head, table
    torch.cuda.empty_cache()
