"""GPU parity of the top-k / argmax epilogue (exl3_topk through _native.topk) against the
oracle's restatement (oracle.topk_rows: largest first, equal values by smaller column, NaN
above every number, -0 == +0), bit-exact in values and columns.

Shapes: the K=6 lm_head's vocabulary (151936) at 1, 3 and 16 rows; four stage-1 chunks of
4096 exactly (16384), one column past them, a last chunk holding fewer than k columns; tiny rows
(n = k, n = 1); the 2^19-column bound; a strided view read in place (ld > n) and rows the
wrapper first copies (n % 8 != 0).  Values: normal logits (many fp16 ties at this size),
rows drawn from a handful of values (ties everywhere, also across chunk boundaries), all-equal
rows, +-0, +-inf and NaN.  Then the epilogue behind the real K=6 lm_head GEMV, and inside a
captured HIP graph replayed with new logits between replays.
"""
import numpy as np
import pytest
import torch

from orcasaq2 import synthetic as syn

pytestmark = pytest.mark.gpu

D = torch.device("cuda", 0)


def check(native, oracle, x, k):
    v, i = native.topk(x, k)
    torch.cuda.synchronize()
    xr = x.detach().cpu().numpy().reshape(-1, x.shape[-1])
    wv, wi = oracle.topk_rows(xr, k)
    gv = v.cpu().numpy().reshape(-1, k)
    gi = i.cpu().numpy().reshape(-1, k)
    assert gi.dtype == np.int64 and gv.dtype == np.float16
    bad = np.argwhere(gi != wi)
    assert bad.size == 0, f"k={k} n={x.shape[-1]}: first mismatch at {bad[0]}: got {gi[tuple(bad[0])]} want {wi[tuple(bad[0])]}"
    assert np.array_equal(gv.view(np.uint16), wv.view(np.uint16))


def logits(rows, n, seed, scale=3.0):
    g = torch.Generator(device=D).manual_seed(seed)
    return (torch.randn(rows, n, generator=g, device=D) * scale).half()


@pytest.mark.parametrize("rows", [1, 3, 16])
@pytest.mark.parametrize("k", [1, 2, 7, 64])
def test_topk_vocab_rows(native, oracle, rows, k):
    print(f"topk vocab rows={rows} k={k}", flush=True)
    check(native, oracle, logits(rows, syn.VOCAB, 11 + rows + k), k)


@pytest.mark.parametrize("n,k", [(16384, 64), (16385, 64), (16384 + 3, 64), (32768 + 40, 64), (100, 7),
                                 (64, 64), (8, 8), (1, 1), (9, 3), (1 << 19, 64), (1 << 19, 1)])
def test_topk_chunk_edges_and_bounds(native, oracle, n, k):
    print(f"topk n={n} k={k}", flush=True)
    check(native, oracle, logits(2, n, n + k), k)


def test_topk_ties_everywhere_and_special_values(native, oracle):
    rng = np.random.default_rng(17)
    n = 3 * 16384 + 77
    pool = np.array([-2.0, -0.0, 0.0, 1.0, 3.0], np.float16)
    x = rng.choice(pool, size=(6, n))
    x[1] = 3.0                                    # one value: the first k columns
    x[2, [5, 16383, 16384, 40000]] = np.inf       # inf across chunk boundaries
    x[3, [70, 16390, 49000]] = np.nan             # NaN ranks first, by column
    x[4] = np.nan
    x[5] = -np.inf
    x[5, 16384 * 2 + 3] = -65504.0
    xt = torch.from_numpy(x).to(D)
    for k in (1, 5, 64):
        print(f"topk ties k={k}", flush=True)
        check(native, oracle, xt, k)


def test_topk_argmax_is_torch_argmax(native):
    x = logits(4, syn.VOCAB, 5)
    x[2, 1000:1010] = 30.0                        # tied maxima: the first one
    assert torch.equal(native.argmax(x), torch.argmax(x, dim=1))


def test_topk_reads_views_and_copies_unreadable_rows(native, oracle):
    big = logits(3, 20000 + 24, 7)
    view = big[:, :20000]                        # ld = 20024 (a multiple of 8), read in place
    check(native, oracle, view, 16)
    odd = logits(3, 20001, 8)                    # n % 8 != 0: copied to a padded layout first
    check(native, oracle, odd, 16)
    check(native, oracle, odd[:, 1:], 16)        # base not 16-byte aligned
    check(native, oracle, logits(2, 5, 3, 2)[1:2], 3)


def test_topk_behind_the_k6_lm_head(native, oracle):
    lin = syn.linear(5120, syn.VOCAB, 6, seed=29)
    trellis, suh, svh = (lin[k].to(D) for k in ("trellis", "suh", "svh"))
    g = torch.Generator().manual_seed(31)
    for rows in (1, 4):
        print(f"lm_head + topk rows={rows}", flush=True)
        x = syn.activations(rows, 5120, g).to(D)
        y = native.gemv(x, trellis, suh, svh, 6, native.CB_3INST)
        check(native, oracle, y, 1)
        check(native, oracle, y, 50)
        assert torch.equal(native.argmax(y), torch.argmax(y, dim=1))


def test_topk_in_a_captured_graph(native, oracle):
    x = logits(2, syn.VOCAB, 40)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        native.topk(x, 8)                        # warm-up on the capture stream
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=s):
        v, i = native.topk(x, 8)
    for rep in range(3):
        x.copy_(logits(2, syn.VOCAB, 41 + rep))
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        wv, wi = oracle.topk_rows(x.cpu().numpy(), 8)
        assert np.array_equal(i.cpu().numpy(), wi), rep
        assert np.array_equal(v.cpu().numpy().view(np.uint16), wv.view(np.uint16)), rep
        ev, ei = native.topk(x, 8)               # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(ei, i)


def test_lm_head_topk_through_the_plugin_surface(native, oracle):
    """A ParallelLMHead quantized at head_bits=6 (the linear method), loaded through its
    placeholders; lm_head_topk gives the argmax / top-k of the fp16 logits its apply casts
    to the activation dtype."""
    from orcasaq2.config import Exl3Config
    from orcasaq2._vllm_compat import ParallelLMHead
    from orcasaq2.heads import lm_head_topk
    vocab, hidden = 4096 + 128, 512
    cfg = Exl3Config.from_config({"bits": 4, "head_bits": 6})
    head = ParallelLMHead(vocab, hidden, params_dtype=torch.bfloat16, quant_config=cfg, prefix="lm_head")
    lin = syn.linear(hidden, vocab, 6, seed=77)
    for name in ("trellis", "suh", "svh"):
        p = getattr(head, name)
        p.weight_loader(p, lin[name].to(D))
    head.quant_method.process_weights_after_loading(head)
    x = syn.activations(3, hidden, torch.Generator().manual_seed(78)).to(torch.bfloat16).to(D)
    logits16 = head.quant_method.apply_fp16(head, x)
    assert logits16.dtype == torch.float16 and logits16.shape == (3, vocab)
    assert torch.equal(head.quant_method.apply(head, x), logits16.to(torch.bfloat16))
    for k in (1, 10):
        v, i = lm_head_topk(head, x, k)
        wv, wi = oracle.topk_rows(logits16.cpu().numpy(), k)
        assert np.array_equal(i.cpu().numpy(), wi)
        assert np.array_equal(v.cpu().numpy().view(np.uint16), wv.view(np.uint16))
