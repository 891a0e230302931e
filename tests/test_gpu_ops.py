"""GPU tests of the drop-in surface: the orcasaq2::shard_gemm / shards_gemv / shards_gemm custom ops
(all three row branches), HIP-graph capture and replay, torch.compile around the op,
and Exl3LinearMethod.apply through a stand-in vLLM layer."""
import numpy as np
import pytest
import torch

import orcasaq2  # noqa: F401
from orcasaq2 import ops as O
from orcasaq2 import synthetic as syn

pytestmark = pytest.mark.gpu

D = torch.device("cuda", 0)


def on(lin):
    return {k: (v.to(D) if isinstance(v, torch.Tensor) else v) for k, v in lin.items()}


def ref(oracle, x, lin, cb=0):
    return oracle.shard_gemm_ref(x.cpu().numpy(), lin["trellis"], lin["suh"].numpy(), lin["svh"].numpy(),
                                 lin["K"], cb)


@pytest.mark.parametrize("rows", [1, 16, 17, 144, 145, 400])
def test_shard_gemm_branches(native, oracle, rows):
    """1 and 16 rows: fused GEMV; 17 and 144: fused GEMM (ic = 512 keeps it); 145 and 400:
    the reconstruct branch."""
    lin = syn.linear(512, 256, 4, seed=rows)
    x = syn.activations(rows, 512, torch.Generator().manual_seed(rows))
    d = on(lin)
    y = torch.ops.orcasaq2.shard_gemm(x.to(D), d["trellis"], d["suh"], d["svh"], 256, 4.0, False, False)
    assert y.dtype == torch.half and y.shape == (rows, 256)
    assert oracle.rel_err_rows(y.cpu().numpy(), ref(oracle, x, lin)).max() <= 1e-3


def test_shard_gemm_rejects_mul1_and_half_rates(native):
    lin = on(syn.linear(256, 256, 4, seed=1))
    x = torch.zeros(1, 256, dtype=torch.half, device=D)
    with pytest.raises(RuntimeError, match="mul1"):
        torch.ops.orcasaq2.shard_gemm(x, lin["trellis"], lin["suh"], lin["svh"], 256, 4.0, False, True)
    bad = torch.zeros(16, 16, 56, dtype=torch.int16, device=D)
    with pytest.raises(RuntimeError, match="half-rate|packed dimension"):
        torch.ops.orcasaq2.shard_gemm(x, bad, lin["suh"], lin["svh"], 256, 3.5, False, False)


def test_shard_gemm_wrong_width_message(native):
    lin = on(syn.linear(256, 256, 4, seed=1))
    x = torch.zeros(1, 256, dtype=torch.half, device=D)
    with pytest.raises(RuntimeError, match="packed dimension 2 is incorrect size"):
        torch.ops.orcasaq2.shard_gemm(x, lin["trellis"], lin["suh"], lin["svh"], 256, 3.0, False, False)


@pytest.mark.parametrize("rows,oc", [(80, 1024), (144, 1024), (120, 10240)])
def test_shard_gemm_routing_by_shape(native, oracle, rows, oc):
    """5120-input shards above 64 rows: the reconstruct branch where it measured faster (oc <
    2 ic, or more than 128 rows), the fused GEMM for wide outputs up to 128 rows; both match
    the oracle."""
    ic = 5120
    assert O._fused_gemm_faster(rows, ic, oc) == (oc >= 2 * ic and rows <= 128)   # within GEMM_MAX_ROWS
    lin = syn.linear(ic, oc, 3, seed=rows + oc)
    x = syn.activations(rows, ic, torch.Generator().manual_seed(rows))
    d = on(lin)
    y = torch.ops.orcasaq2.shard_gemm(x.to(D), d["trellis"], d["suh"], d["svh"], oc, 3.0, False, False)
    assert oracle.rel_err_rows(y.cpu().numpy(), ref(oracle, x, lin)).max() <= 1e-3


@pytest.mark.parametrize("rows", [512, 2048, 3072])
def test_shard_gemm_down_proj_prefill_op_route(native, oracle, rows):
    """The op on config 3's shape, down_proj 17408 -> 5120 at K=4, at 512 and 2048 rows
    (above GEMM_MAX_ROWS: the fused GEMM for wide inputs) and 3072 rows (the reconstruct
    branch, measured faster there): whichever route the op takes, sampled rows match the
    oracle."""
    lin = syn.linear(17408, 5120, 4, seed=3)
    x = syn.activations(rows, 17408, torch.Generator().manual_seed(rows + 33))
    d = on(lin)
    fused = O._fused_route(rows, 17408, 5120)
    if not O.GEMM_MAX_ROWS_SET:
        assert fused == (rows <= O.WIDE_FUSED_MAX_ROWS)
    print(f"shard_gemm down_proj rows={rows} fused={fused}", flush=True)
    y = torch.ops.orcasaq2.shard_gemm(x.to(D), d["trellis"], d["suh"], d["svh"], 5120, 4.0, False, False)
    assert y.shape == (rows, 5120) and y.dtype == torch.half
    W = oracle.reconstruct_f16(lin["trellis"], 4, 0)
    idx = torch.tensor([0, 1, 63, 64, rows // 2, rows - 1])
    want = oracle.shard_gemm_ref(x[idx].numpy(), lin["trellis"], lin["suh"].numpy(), lin["svh"].numpy(), 4, 0, W=W)
    assert oracle.rel_err_rows(y[idx.to(D)].cpu().numpy(), want).max() <= 1e-3


def _two_shard_step(rows, ic=1024):
    lins = [syn.linear(ic, oc, K, seed=i) for i, (oc, K) in enumerate([(512, 4), (256, 5)])]
    ds = [on(l) for l in lins]

    def step(x):
        a = torch.ops.orcasaq2.shard_gemm(x, ds[0]["trellis"], ds[0]["suh"], ds[0]["svh"], 512, 4.0, False, False)
        grouped = torch.ops.orcasaq2.shards_gemv if x.shape[0] <= 16 else torch.ops.orcasaq2.shards_gemm
        b = grouped(x, [d["trellis"] for d in ds], [d["suh"] for d in ds], [d["svh"] for d in ds], [512, 256],
                    [4.0, 5.0], [False, False], [False, False])
        return a, b
    return step


@pytest.mark.parametrize("rows", [1, 2, 9, 40])
def test_hip_graph_capture_replays(native, oracle, rows):
    """The op and the grouped op captured into a HIP graph on a stream that ran them eagerly
    first (so the capture uses that stream's eager GEMV workspace), replayed four times with
    eager work between replays, against eager results: 1 row (persistent decode launch that
    finishes its split column groups through the accumulator area), 2 rows (four-row
    template), 9 rows (the 5..16-row
    kernel: set-up, one decode launch over both K, finish), 40 rows (prefill: 48-row stream-K tiles, counters zeroed by the
    set-up kernels inside the graph)."""
    step = _two_shard_step(rows)
    x = syn.activations(rows, 1024, torch.Generator().manual_seed(1)).to(D)
    eager = step(x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(x)  # creates this stream's workspace outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = step(x)
    for i in range(4):
        x.copy_(syn.activations(rows, 1024, torch.Generator().manual_seed(1)).to(D))
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[0], eager[0]) and torch.equal(out[1], eager[1]), i
        with torch.cuda.stream(s):
            step(x)  # eager work on the same stream between replays
        torch.cuda.synchronize()


def test_graphs_share_workspace_and_survive_its_growth(native):
    """Two graphs captured on one stream share its eager workspace; an eager 16-row call on
    that stream then needs a larger workspace (the old one must stay alive for the graphs);
    the graphs are replayed in reverse capture order, each against eager results."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    steps = {r: _two_shard_step(r) for r in (1, 3)}
    xs = {r: syn.activations(r, 1024, torch.Generator().manual_seed(10 + r)).to(D) for r in (1, 3)}
    eager = {r: steps[r](xs[r]) for r in (1, 3)}
    graphs, outs = {}, {}
    with torch.cuda.stream(s):
        steps[1](xs[1])
        torch.cuda.synchronize()
        for r in (1, 3):
            graphs[r] = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graphs[r], stream=s):
                outs[r] = steps[r](xs[r])
    torch.cuda.synchronize()
    x16 = syn.activations(16, 1024, torch.Generator().manual_seed(16)).to(D)
    with torch.cuda.stream(s):
        big = _two_shard_step(16)(x16)
    torch.cuda.synchronize()
    for rep in range(3):
        for r in (3, 1):
            with torch.cuda.stream(s):
                graphs[r].replay()
            torch.cuda.synchronize()
            assert torch.equal(outs[r][0], eager[r][0]) and torch.equal(outs[r][1], eager[r][1]), (rep, r)
        with torch.cuda.stream(s):
            again = _two_shard_step(16)(x16)
        torch.cuda.synchronize()
        assert torch.equal(again[0], big[0]) and torch.equal(again[1], big[1]), rep


def test_capture_without_eager_warmup(native):
    """A capture on a stream that never ran the op eagerly: the workspace is made inside the
    capture (from the graph's memory pool) and is private to that graph; eager calls on the
    same stream afterwards get their own, and both stay correct in any order."""
    step = _two_shard_step(1)
    x = syn.activations(1, 1024, torch.Generator().manual_seed(21)).to(D)
    eager = step(x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = step(x)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        e1 = step(x)   # eager before the graph was ever replayed
    torch.cuda.synchronize()
    assert torch.equal(e1[0], eager[0]) and torch.equal(e1[1], eager[1])
    for i in range(3):
        with torch.cuda.stream(s):
            g.replay()
            e2 = step(x)
        torch.cuda.synchronize()
        assert torch.equal(out[0], eager[0]) and torch.equal(out[1], eager[1]), i
        assert torch.equal(e2[0], eager[0]) and torch.equal(e2[1], eager[1]), i


def test_many_captures_keep_bounded_workspace_bookkeeping(native):
    """Graph after graph captured on fresh streams (no eager workspace there, so each capture
    makes its own from its graph's pool): the library keeps one capture entry per stream and
    keeps no capture workspace alive itself (the graphs' pools do), and every graph still
    replays to the eager result after all the later captures and their destruction."""
    step = _two_shard_step(1)
    x = syn.activations(1, 1024, torch.Generator().manual_seed(22)).to(D)
    eager = step(x)
    kept0 = len(native._gemv_ws_kept)
    graphs = []
    for i in range(12):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = step(x)
        graphs.append((g, s, out))
        if i % 3 == 2:
            graphs.pop(0)            # a graph destroyed along the way
    torch.cuda.synchronize()
    assert len(native._gemv_ws_kept) == kept0
    assert all(isinstance(e, tuple) and len(e) == 2 for e in native._gemv_ws_cap.values())
    for g, s, out in graphs:
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[0], eager[0]) and torch.equal(out[1], eager[1])


def test_torch_compile_treats_op_as_opaque(native):
    lin = on(syn.linear(256, 256, 3, seed=4))
    x = syn.activations(1, 256, torch.Generator().manual_seed(4)).to(D)

    def f(x):
        y = torch.ops.orcasaq2.shard_gemm(x * 1.0, lin["trellis"], lin["suh"], lin["svh"], 256, 3.0, False, False)
        return y.float().sum(-1)

    want = f(x)
    got = torch.compile(f, backend="eager", fullgraph=True)(x)
    assert torch.equal(want, got)


def test_linear_method_apply_fused_layers(native, oracle):
    """qkv_proj-style layer: shards captured by slot, processed, applied (grouped decode-GEMV
    at <= 16 rows, grouped GEMM to 144, per-shard ops + cat above for these narrow inputs),
    bias added, dtype restored."""
    from orcasaq2.config import Exl3Config, Exl3LinearMethod
    from orcasaq2._vllm_compat import LinearBase
    cfg = Exl3Config.from_config({"bits": 4})
    spec = [("q", 512, 4), ("k", 128, 5), ("v", 128, 5)]
    lins = {sid: syn.linear(256, oc, K, seed=i) for i, (sid, oc, K) in enumerate(spec)}
    layer = LinearBase(256, 768, bias=True, params_dtype=torch.bfloat16, quant_config=cfg,
                       prefix="model.layers.0.self_attn.qkv_proj", output_partition_sizes=[512, 128, 128])
    assert isinstance(layer.quant_method, Exl3LinearMethod)
    for sid in ("v", "q", "k"):  # arrival order must not matter
        for name in ("trellis", "suh", "svh"):
            p = getattr(layer, name)
            p.weight_loader(p, lins[sid][name].to(D), sid)
    layer.bias.data = torch.randn(768).to(torch.bfloat16)
    layer.quant_method.process_weights_after_loading(layer)
    layer.bias.data = layer.bias.data.to(D)
    for rows in (1, 5, 40, 144, 200):
        x = syn.activations(rows, 256, torch.Generator().manual_seed(rows)).to(torch.bfloat16)
        y = layer(x.to(D))
        assert y.dtype == torch.bfloat16 and y.shape == (rows, 768)
        xh = x.half()
        col = 0
        for sid, oc, K in spec:
            want = ref(oracle, xh, lins[sid]) + layer.bias.float().cpu().numpy()[col:col + oc]
            got = y[:, col:col + oc].float().cpu().numpy()
            err = np.linalg.norm(got - want, axis=1) / np.linalg.norm(want, axis=1)
            assert err.max() < 1e-2, (sid, rows, err.max())  # bf16 output rounding
            col += oc


def test_linear_method_apply_grouped_above_gemm_max_rows(native, oracle):
    """A gate_up-style layer (4096 inputs, two 8192-output shards, K = 3 and 4) at 2048 rows:
    above GEMM_MAX_ROWS every shard routes to the fused GEMM (oc >= 2 ic inside
    WIDE_OUT_FUSED_ROWS), so apply runs them as one grouped launch -- bit for bit the
    grouped op's output -- and sampled rows of both shards match the oracle."""
    from orcasaq2.config import Exl3Config
    from orcasaq2._vllm_compat import LinearBase
    if O.GEMM_MAX_ROWS_SET:
        pytest.skip("the row knob is set: the reference's hard switch applies")
    rows, ic = 2048, 4096
    spec = [(0, 8192, 3), (1, 8192, 4)]
    assert all(O._fused_route(rows, ic, oc) for _, oc, _ in spec)
    lins = {sid: syn.linear(ic, oc, K, seed=40 + sid) for sid, oc, K in spec}
    cfg = Exl3Config.from_config({"bits": 4})
    layer = LinearBase(ic, 2 * 8192, bias=False, params_dtype=torch.float16, quant_config=cfg,
                       prefix="model.layers.0.mlp.gate_up_proj", output_partition_sizes=[8192, 8192])
    for sid, _, _ in spec:
        for name in ("trellis", "suh", "svh"):
            p = getattr(layer, name)
            p.weight_loader(p, lins[sid][name].to(D), sid)
    layer.quant_method.process_weights_after_loading(layer)
    x = syn.activations(rows, ic, torch.Generator().manual_seed(41))
    print(f"apply gate_up-like 4096 -> 2 x 8192 rows={rows}", flush=True)
    y = layer(x.to(D))
    sh = layer.exl3_shards
    yg = torch.ops.orcasaq2.shards_gemm(x.to(D), [s.trellis for s in sh], [s.suh for s in sh], [s.svh for s in sh],
                                        [s.oc for s in sh], [float(s.K) for s in sh], [False, False], [False, False])
    assert torch.equal(y, yg)
    idx = torch.tensor([0, 1, 255, 256, 1027, rows - 1])
    col = 0
    for sid, oc, K in spec:
        l = lins[sid]
        W = oracle.reconstruct_f16(l["trellis"], K, 0)
        want = oracle.shard_gemm_ref(x[idx].numpy(), l["trellis"], l["suh"].numpy(), l["svh"].numpy(), K, 0, W=W)
        got = y[idx.to(D), col:col + oc].cpu().numpy()
        assert oracle.rel_err_rows(got, want).max() <= 1e-3, sid
        col += oc


def test_embedding_method_int8_on_gpu(native):
    from orcasaq2.config import Exl3Config
    from orcasaq2._vllm_compat import VocabParallelEmbedding
    cfg = Exl3Config.from_config({})
    emb = VocabParallelEmbedding(1000, 64, params_dtype=torch.bfloat16, quant_config=cfg)
    g = torch.Generator().manual_seed(3)
    q = torch.randint(-128, 128, (1000, 64), generator=g, dtype=torch.int8)
    s = torch.rand(1000, generator=g) * 0.01
    emb.qweight.weight_loader(emb.qweight, q.to(D))
    emb.scales.weight_loader(emb.scales, s.to(D))
    emb.quant_method.process_weights_after_loading(emb)
    ids = torch.tensor([3, 999, 0, 3], device=D)
    out = emb(ids)
    want = q[ids.cpu()].to(torch.bfloat16) * s.to(torch.bfloat16).reshape(-1, 1)[ids.cpu()]
    assert torch.equal(out.cpu(), want)


def test_reconstruct_weight_dense_equivalence(native, oracle):
    """F.linear(x, reconstruct_weight(...)) matches the fused op (orcasaq2/__init__.py:49-61
    against orcasaq2/ops.py:53-59)."""
    from orcasaq2 import reconstruct_weight
    lin = syn.linear(256, 384, 4, seed=12)
    d = on(lin)
    W = reconstruct_weight(d["trellis"], d["suh"], d["svh"], None, None)
    assert W.shape == (384, 256) and W.dtype == torch.half
    x = syn.activations(3, 256, torch.Generator().manual_seed(12)).to(D)
    y_dense = torch.nn.functional.linear(x.float(), W.float())
    y = torch.ops.orcasaq2.shard_gemm(x, d["trellis"], d["suh"], d["svh"], 384, 4.0, False, False)
    err = torch.linalg.norm(y.float() - y_dense, dim=1) / torch.linalg.norm(y_dense, dim=1)
    assert err.max().item() < 2e-3


def test_reconstruct_weight_matches_oracle_deploy_weight(native, oracle):
    """reconstruct_weight (HIP W_q + fp32 Hadamard/sign algebra, orcasaq2/__init__.py:49-61)
    against the oracle's fp64 deploy weight on the oracle's own W_q: every element within
    half an fp16 ulp of the fp64 value plus the fp32 algebra's absolute rounding (two
    128-term Hadamard sums: at most ~2^-18 of the largest element; 2^-16 allowed), so a
    wrong sign, index or transposition -- an error of the order of the elements -- fails."""
    from orcasaq2 import reconstruct_weight
    for K, cb, (ic, oc) in ((4, 0, (256, 384)), (3, 1, (384, 128)), (5, 0, (5120, 1024))):
        lin = syn.linear(ic, oc, K, seed=40 + K)
        d = on(lin)
        mcg = torch.ones(1, device=D) if cb else None
        W = reconstruct_weight(d["trellis"], d["suh"], d["svh"], mcg, None).cpu().numpy().astype(np.float64)
        ref = oracle.deploy_weight(oracle.reconstruct_f16(lin["trellis"], K, cb), lin["suh"].numpy(),
                                   lin["svh"].numpy())
        assert W.shape == ref.shape == (oc, ic)
        ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
        bound = 0.5 * ulp + 2.0 ** -16 * np.abs(ref).max()
        assert (np.abs(W - ref) <= bound).all(), (K, cb, np.max(np.abs(W - ref) / bound))


def test_min_capability_passes_vllms_check_on_this_gpu():
    """vLLM refuses a quantization method when the device capability, major * 10 + minor,
    is below get_min_capability() (reference orcasaq2/config.py:107-109 returns 80).  On
    ROCm torch reports gfx9 parts as (9, x): gfx950 is (9, 5), so 95 >= 80 passes."""
    from orcasaq2.config import Exl3Config
    major, minor = torch.cuda.get_device_capability(0)
    assert major * 10 + minor >= Exl3Config.get_min_capability(), (major, minor)
    assert "gfx9" in torch.cuda.get_device_properties(0).gcnArchName


def test_concurrent_streams_keep_their_own_workspaces(native):
    """Three streams (default priority) run the ops at 1, 9 and 40 rows at the same time, each
    calling repeatedly on its own stream: every stream gets its own GEMV workspace, and every
    result equals the one computed alone on the default stream."""
    steps = {rows: _two_shard_step(rows) for rows in (1, 9, 40)}
    xs = {rows: syn.activations(rows, 1024, torch.Generator().manual_seed(90 + rows)).to(D) for rows in steps}
    want = {rows: steps[rows](xs[rows]) for rows in steps}
    torch.cuda.synchronize()
    streams = {rows: torch.cuda.Stream() for rows in steps}
    for s in streams.values():
        s.wait_stream(torch.cuda.current_stream())
    got = {rows: [] for rows in steps}
    for it in range(6):                                   # interleaved issue on the three streams
        for rows, s in streams.items():
            with torch.cuda.stream(s):
                got[rows].append(steps[rows](xs[rows]))
    torch.cuda.synchronize()
    for rows in steps:
        for a, b in got[rows]:
            assert torch.equal(a, want[rows][0]) and torch.equal(b, want[rows][1]), rows
    keys = [k for k in native._gemv_ws if k[1] in {s.cuda_stream for s in streams.values()}]
    assert len({native._gemv_ws[k].data_ptr() for k in keys}) == len(keys)   # no workspace shared
