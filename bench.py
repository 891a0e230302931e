"""Benchmark of the MI355X EXL3 trellis linear path (BASELINE.json metric):
bs=1 fused EXL3 GEMV, packed-weight GB/s and fraction of HBM peak.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-stack]

Workload: down_proj 17408 -> 5120 at batch 1 through the fused
decode-GEMV at K = 2, 3, 4 and 5 bits.  One step = one GEMV at each K.  Every GEMV reads a
different copy of the weights (more than 512 MB of distinct packed words per K), so the
256 MB Infinity Cache cannot serve a repeat: the bytes come from HBM.  Inputs are
resident in HBM before the timed region starts.

The timed steps are replayed from a HIP graph (captured once, the way decode serving
replays its steps), so host launch overhead is not part of the measurement; the
warm-up steps are a graph replay too.
`value` = total packed trellis bytes / total time over the timed steps.
`roofline` = the dominant GEMV (the K whose call moves the most bytes; one call = one
gemv1_kernel<K> launch, which also finishes its split column groups): algorithmic bytes per call
(ic*oc*K/8) / its mean duration from HIP events recorded on the replay stream around a
graph of the same steps, against 8 TB/s.  `traffic` = HBM bytes per call measured with
rocprofv3 FETCH_SIZE + WRITE_SIZE and scaled by the same counters' reading for a plain
copy of known size (profiles/gemv_traffic.json; `python bench.py --copy-calib` is the
calibration workload).
`cpu_baseline` = the reference's CPU path restated by the oracle (trellis decode in C, the
reconstruct_weight Hadamard/sign algebra in fp32 torch, F.linear), timed on this host's
cores on one step of the same workload.
`tok_s_equiv` / `stack` = config 4 measured: the whole 64-layer linear stack + lm_head +
its argmax epilogue + the embedding gather of the argmax token, one batch-1 greedy token as
one HIP graph, replayed (attention excluded).

    python bench.py --workload config2   # grouped qkv / gate_up GEMVs at batch 1, 4, 16
    python bench.py --workload config3   # M=2048 prefill GEMM (TFLOP/s, MFMA share) + reconstruct
    python bench.py --workload config4   # the 64-layer batch-1 linear stack alone (tok/s-equivalent)
    python bench.py --workload lmhead    # the K=6 lm_head GEMV at 1, 2, 3, 4, 8, 16 rows
    python bench.py --workload prefill   # 17..768-row prefill: fused vs reconstruct branch, grouped layers
    python bench.py --workload ceiling   # what bounds batch 1: loads / decode / MFMA alone, instruction costs
print their own JSON line instead of the headline line.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "orcasaq2-kernel_amd"))
sys.path.insert(0, ROOT)

METRIC = "bs=1 fused EXL3 GEMV packed-weight GB/s (% HBM peak) + 27B tok/s-equiv"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFS = 2500.0   # dense fp16 MFMA, MI355X
ROTATE_BYTES = 600 * 2 ** 20


def copy_calib(args) -> None:
    """Plain device copy of 256 MiB, repeated: the known-size workload that calibrates the
    FETCH_SIZE / WRITE_SIZE counters (each copy reads and writes exactly 268435456 bytes)."""
    import torch
    dev = torch.device("cuda", 0)
    a = torch.empty(1 << 28, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    for _ in range(max(args.steps, 1)):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calib_bytes": 1 << 28, "copies": max(args.steps, 1)}), flush=True)


def load_traffic(dom_K: int, nbytes: int):
    """HBM bytes per GEMV call from the committed counter calibration, or None."""
    path = os.path.join(ROOT, "profiles", "gemv_traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        e = t["per_K"][str(dom_K)]
        return int(e["hbm_bytes_per_call"])
    except (OSError, KeyError, ValueError):
        return None


def gpu_bench(args) -> dict:
    """Config 1 on the GPU.  Each step is captured once into a HIP graph (the way decode
    serving replays its steps) so host launch overhead is outside the measurement: W
    warm-up steps are one graph replay, the K timed steps another, bracketed by
    synchronisation.  Per-K figures come from one graph per K (the K timed steps' calls of
    that K), replayed PER_K_REPS times back to back between HIP events on the capture stream,
    so the one launch of a graph from the host is spread over that many replays instead of
    weighing on one replay's calls."""
    import torch
    from orcasaq2 import _native
    from orcasaq2 import synthetic as syn

    dev = torch.device("cuda", 0)
    ic, oc = syn.INTERMEDIATE, syn.HIDDEN
    Ks = (args.only_K,) if args.only_K else (2, 3, 4, 5)
    g = torch.Generator(device=dev).manual_seed(1)
    copies = {}
    for K in Ks:
        nbytes = syn.packed_bytes(ic, oc, K)
        n = max(2, math.ceil(ROTATE_BYTES / nbytes))
        lst = []
        for _ in range(n):
            t = torch.randint(-32768, 32768, (ic // 16, oc // 16, 16 * K), generator=g, device=dev,
                              dtype=torch.int32).to(torch.int16)
            suh = (torch.randint(0, 2, (ic,), generator=g, device=dev) * 2 - 1).half()
            svh = ((torch.randn(oc, generator=g, device=dev).abs() / math.sqrt(ic)).half()
                   * (torch.randint(0, 2, (oc,), generator=g, device=dev) * 2 - 1).half())
            lst.append((t, suh, svh))
        copies[K] = lst
    x = torch.randn(1, ic, generator=g, device=dev).half()
    outs = {K: torch.empty(1, oc, dtype=torch.half, device=dev) for K in Ks}

    def gemv(K, step):
        t, suh, svh = copies[K][step % len(copies[K])]
        _native.gemv(x, t, suh, svh, K, 0, out=outs[K])

    def run_steps(first, count, only=None):
        for i in range(first, first + count):
            for K in (only or Ks):
                gemv(K, i)

    # eager calls first: they allocate the persistent workspace outside any capture
    run_steps(0, 2)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(dev)

    def capture(first, count, only=None):
        graph = torch.cuda.CUDAGraph()
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            run_steps(first, 1, only)   # settles this stream's workspace before capture
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=side):
                run_steps(first, count, only)
        torch.cuda.synchronize()
        return graph

    g_warm = capture(0, max(args.warmup, 1))
    g_timed = capture(args.warmup, args.steps)
    _settle(g_warm.replay, side)          # clocks out of their idle state (not timed)
    g_warm.replay()                       # the W warm-up steps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g_timed.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    per_k = {}
    for K in Ks:
        gk = capture(args.warmup, args.steps, only=(K,))
        _settle(gk.replay, side)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(side)
        with torch.cuda.stream(side):
            for _ in range(PER_K_REPS):
                gk.replay()
        e1.record(side)
        torch.cuda.synchronize()
        mean = e0.elapsed_time(e1) * 1e-3 / (args.steps * PER_K_REPS)
        nbytes = syn.packed_bytes(ic, oc, K)
        per_k[K] = dict(bytes=nbytes, mean_us=mean * 1e6, gbs=nbytes / mean / 1e9,
                        frac=nbytes / mean / 1e9 / HBM_PEAK_GBS, total_s=mean * args.steps)
        del gk
    total_bytes = sum(per_k[K]["bytes"] for K in Ks) * args.steps
    value = total_bytes / wall / 1e9
    # the call that moves the most of the step's bytes (K=5 in the default run); the calls'
    # times are within noise of each other, so the longest one changes from run to run
    dom = max(Ks, key=lambda K: per_k[K]["bytes"])
    return dict(value=value, wall=wall, per_k=per_k, dom=dom,
                device=torch.cuda.get_device_name(dev))


def _rand_linear(ic, oc, K, g, dev):
    """One synthetic EXL3 tensor set made on the GPU (orcasaq2.synthetic.linear_gpu)."""
    from orcasaq2 import synthetic as syn
    return syn.linear_gpu(ic, oc, K, g, dev)


def _graph(dev, fn, settle=True):
    """Capture fn() into a HIP graph on a side stream (one eager call first settles the
    stream's persistent GEMV workspace outside the capture)."""
    import torch
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        if settle:
            fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            fn()
    torch.cuda.synchronize()
    return graph, side


SETTLE_S = 0.25     # seconds of sustained GPU work before any timed region
PER_K_REPS = 5      # back-to-back replays of each per-K graph between its HIP events


def _settle(replay, side, seconds: float = SETTLE_S) -> None:
    """Runs replay() (one graph replay, or one eager step) on `side` until `seconds` of GPU time
    have passed.  The GPU's clocks rise from their idle state only over the first tens of
    milliseconds of sustained work: measured on MI355X from idle, a down_proj K=5 GEMV call
    takes 19.6-20.3 us in the first ~3 ms and 16.4-17.0 us from ~20 ms on, the M=2048 prefill
    GEMM 456-514 us at first and ~400 us from ~35 ms on.  A serving GPU runs busy, so the
    timed regions start from those steady clocks; the settle is never part of a timing."""
    import torch
    spent, n = 0.0, 1
    while spent < seconds:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(side)
        with torch.cuda.stream(side):
            for _ in range(n):
                replay()
        e1.record(side)
        torch.cuda.synchronize()
        spent += e0.elapsed_time(e1) * 1e-3
        # small batches: right after one batch of some hundreds of replays, the next replay
        # measured ~3x its steady time (the runtime's own cost, not the GPU's)
        n = min(2 * n, 16)


def _time_graph(graph, side, reps: int) -> float:
    """Seconds per replay: replays until the clocks have settled (_settle), then `reps`
    replays between HIP events recorded on the replay stream."""
    import torch
    _settle(graph.replay, side)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(side)
    with torch.cuda.stream(side):
        for _ in range(reps):
            graph.replay()
    e1.record(side)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / reps


def prefill_bench(reps: int) -> dict:
    """Prefill at 17..4096 rows, the 27B layer shapes: per shape and row count the fused
    stream-K GEMM (exl3_gemm) against the op's reconstruct branch (had_r_128, reconstruct
    to (oc, ic), library fp16 transposed-B GEMM, had_r_128); per fused layer (qkv, gate_up)
    the grouped launch (exl3_gemm_grouped) against the per-shard fused GEMMs + cat and the
    per-shard reconstruct branch + cat.  us per call, each call one HIP-graph replay."""
    import torch
    from orcasaq2 import _native
    import orcasaq2.ops  # noqa: F401

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(5)

    def t_of(fn):
        graph, side = _graph(dev, fn)
        return round(_time_graph(graph, side, reps) * 1e6, 1)

    import orcasaq2.ops as ops

    def recon(x, d):
        return ops._reconstruct_branch(x, d["trellis"], d["suh"], d["svh"], d["K"], 0)

    out = {"single": {}, "grouped": {}}
    for name, ic, oc, K in (("down 17408->5120 K4", 17408, 5120, 4), ("gate 5120->17408 K3", 5120, 17408, 3),
                            ("q 5120->6144 K4", 5120, 6144, 4)):
        d = _rand_linear(ic, oc, K, g, dev)
        row = {}
        for M in (17, 40, 64, 80, 128, 144, 256, 384, 768, 1024, 1536, 2048, 2560, 3072, 4096):
            x = torch.randn(M, ic, generator=g, device=dev).half()
            y = torch.empty(M, oc, dtype=torch.half, device=dev)
            row[M] = {"fused": t_of(lambda: _native.gemm(x, d["trellis"], d["suh"], d["svh"], K, 0, out=y)),
                      "reconstruct_branch": t_of(lambda: recon(x, d))}
        out["single"][name] = row
    for name, spec in (("qkv (q 6144 K4, k/v 1024 K5)", [(6144, 4), (1024, 5), (1024, 5)]),
                       ("gate_up (2 x 17408 K3)", [(17408, 3), (17408, 3)])):
        sh = [_rand_linear(5120, o, k, g, dev) for o, k in spec]
        row = {}
        for M in (17, 64, 144, 2048):
            x = torch.randn(M, 5120, generator=g, device=dev).half()
            row[M] = {"grouped": t_of(lambda: _native.gemm_grouped(x, sh)),
                      "per_shard_fused_cat": t_of(lambda: torch.cat(
                          [_native.gemm(x, d["trellis"], d["suh"], d["svh"], d["K"], 0) for d in sh], dim=1)),
                      "per_shard_reconstruct_cat": t_of(lambda: torch.cat([recon(x, d) for d in sh], dim=1))}
        out["grouped"][name] = row
    return out


def stack_bench(tokens: int = 20) -> dict:
    """Config 4: the linear stack of a 64-layer Qwen-27B-shaped decoder at batch-1 decode,
    one token = the int8 embedding gather, per layer the grouped q/k/v GEMV, o_proj, the
    grouped gate/up GEMV and down_proj (K from the seeded {2,3,4,5} draw), then the K=6
    lm_head.  Attention, norms, residuals and the activation function are excluded
    but every projection reads what the one before it produced, so
    nothing runs before its input exists: o_proj reads the q columns of qkv (the width of
    the attention output it stands for), gate/up read o_proj's output, down_proj reads the
    gate columns, the next layer reads down_proj's output, the lm_head the last one
    (orcasaq2.synthetic.stack_gpu builds the tensors).  The token is captured once into a
    HIP graph and replayed `tokens` times."""
    import torch
    from orcasaq2 import _native
    from orcasaq2 import synthetic as syn

    dev = torch.device("cuda", 0)
    st = syn.stack_gpu(dev)
    layers, head, table, scales, nbytes = st["layers"], st["head"], st["table"], st["scales"], st["nbytes"]
    ids = torch.tensor([12345], device=dev)
    y_qkv = torch.empty(1, syn.Q_OUT + 2 * syn.KV_OUT, dtype=torch.half, device=dev)
    y_o = torch.empty(1, syn.HIDDEN, dtype=torch.half, device=dev)
    y_gu = torch.empty(1, 2 * syn.INTERMEDIATE, dtype=torch.half, device=dev)
    y_h = torch.empty(1, syn.HIDDEN, dtype=torch.half, device=dev)
    logits = torch.empty(1, syn.VOCAB, dtype=torch.half, device=dev)
    q_cols = y_qkv[:, :syn.Q_OUT]           # one row: a contiguous view
    gate_cols = y_gu[:, :syn.INTERMEDIATE]

    def token():
        h = _native.embed_int8(table, scales, ids)
        for L in layers:
            _native.gemv_grouped(h, [L["q"], L["k"], L["v"]], out=y_qkv)
            _native.gemv_grouped(q_cols, [L["o"]], out=y_o)
            _native.gemv_grouped(y_o, [L["gate"], L["up"]], out=y_gu)
            _native.gemv_grouped(gate_cols, [L["down"]], out=y_h)
            h = y_h
        _native.gemv_grouped(h, [head], out=logits)
        ids.copy_(_native.argmax(logits))       # greedy: the next token's embedding row

    graph, side = _graph(dev, token)
    sec = _time_graph(graph, side, tokens)
    finite = bool(torch.isfinite(logits).all().item())
    rms = float(logits.float().pow(2).mean().sqrt().item())
    del graph
    # the argmax / top-k epilogue alone on the same logits: 20 calls per graph, so a replay's
    # launch cost is spread over them
    epilogue = {}
    for name, k in (("argmax", 1), ("top64", 64)):
        def calls(k=k):
            for _ in range(20):
                _native.topk(logits, k)
        g2, side2 = _graph(dev, calls)
        epilogue[name] = round(_time_graph(g2, side2, 20) * 1e6 / 20, 2)
        del g2
    return {"tok_s": round(1.0 / sec, 2), "ms_per_token": round(sec * 1e3, 4), "bytes_per_token": nbytes,
            "GB/s": round(nbytes / sec / 1e9, 1), "frac": round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4),
            "tokens": tokens, "logits_finite": finite, "logits_rms": round(rms, 4),
            "epilogue_us": epilogue,
            "what": "config4 measured: 64-layer Qwen-27B-shaped linear stack + K=6 lm_head + argmax epilogue "
                    "+ int8 embedding gather of the argmax token, batch 1, each projection chained on the "
                    "previous output, one HIP-graph-launched token replayed; attention/KV/norms/activation "
                    "excluded"}


def config2_bench(reps: int) -> dict:
    """Config 2: grouped q/k/v (K 4/5/5) and gate/up (K 3/3) GEMVs at batch 1, 4 and 16,
    each call on a different weight copy (> 512 MB rotated per projection group)."""
    import torch
    from orcasaq2 import _native
    from orcasaq2 import synthetic as syn

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(2)
    H = syn.HIDDEN
    groups = {"qkv": [(syn.Q_OUT, 4), (syn.KV_OUT, 5), (syn.KV_OUT, 5)],
              "gate_up": [(syn.INTERMEDIATE, 3), (syn.INTERMEDIATE, 3)]}
    out = {}
    for name, spec in groups.items():
        gbytes = sum(syn.packed_bytes(H, oc, K) for oc, K in spec)
        n = max(2, math.ceil(ROTATE_BYTES / gbytes))
        copies = [[_rand_linear(H, oc, K, g, dev) for oc, K in spec] for _ in range(n)]
        total = sum(oc for oc, _ in spec)
        for rows in (1, 4, 16):
            x = torch.randn(rows, H, generator=g, device=dev).half()
            y = torch.empty(rows, total, dtype=torch.half, device=dev)

            def run():
                for c in copies:
                    _native.gemv_grouped(x, c, out=y)

            graph, side = _graph(dev, run)
            sec = _time_graph(graph, side, max(1, reps // n)) / n
            del graph
            out[f"{name}_b{rows}"] = {"us_per_call": round(sec * 1e6, 3), "packed_bytes": gbytes,
                                      "GB/s": round(gbytes / sec / 1e9, 1),
                                      "frac": round(gbytes / sec / 1e9 / HBM_PEAK_GBS, 4)}
        del copies
    return out


def lmhead_bench(reps: int) -> dict:
    """The K=6 lm_head (5120 -> 151936, 583 MB packed) as one GEMV at 1, 2, 3, 4, 8 and 16
    rows: 1..4 rows on the four-row decode kernel (with 2..4 rows its workgroup ranges' tables
    leave fewer than three workgroups per CU resident, so the launch takes more workgroups
    than stay resident), 5..16 on gemv16.  Each call reads a different weight copy."""
    import torch
    from orcasaq2 import _native
    from orcasaq2 import synthetic as syn

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(6)
    H, V, K = syn.HIDDEN, syn.VOCAB, 6
    nbytes = syn.packed_bytes(H, V, K)
    n = max(2, math.ceil(ROTATE_BYTES / nbytes))
    copies = [_rand_linear(H, V, K, g, dev) for _ in range(n)]
    out = {}
    for rows in (1, 2, 3, 4, 8, 16):
        x = torch.randn(rows, H, generator=g, device=dev).half()
        y = torch.empty(rows, V, dtype=torch.half, device=dev)

        def run():
            for c in copies:
                _native.gemv(x, c["trellis"], c["suh"], c["svh"], K, 0, out=y)

        graph, side = _graph(dev, run)
        sec = _time_graph(graph, side, max(1, reps // n)) / n
        del graph
        out[f"b{rows}"] = {"us_per_call": round(sec * 1e6, 3), "packed_bytes": nbytes,
                           "GB/s": round(nbytes / sec / 1e9, 1),
                           "frac": round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4)}
    del copies
    return out


def config3_bench(reps: int) -> dict:
    """Config 3: prefill GEMM of M=2048 rows through down_proj (17408 -> 5120, K=4), and a
    standalone reconstruct of the same weight to fp16, as (ic, oc) and as (oc, ic)."""
    import torch
    from orcasaq2 import _native
    from orcasaq2 import synthetic as syn

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(3)
    ic, oc, K, M = syn.INTERMEDIATE, syn.HIDDEN, 4, 2048
    lin = _rand_linear(ic, oc, K, g, dev)
    x = torch.randn(M, ic, generator=g, device=dev).half()
    y = torch.empty(M, oc, dtype=torch.half, device=dev)
    W = torch.empty(ic, oc, dtype=torch.half, device=dev)
    Wt = torch.empty(oc, ic, dtype=torch.half, device=dev)

    def gemm():
        _native.gemm(x, lin["trellis"], lin["suh"], lin["svh"], K, 0, out=y)

    def recon():
        _native.reconstruct(lin["trellis"], K, 0, out=W)

    def recon_t():
        _native.reconstruct_t(lin["trellis"], K, 0, out=Wt)

    import orcasaq2.ops as ops

    def op():
        # the reference's path for M > GEMM_MAX_ROWS: had_r_128 -> reconstruct (transposed) ->
        # library fp16 GEMM -> had_r_128 (orcasaq2/ops.py:50-59 of the reference); the op
        # itself routes this shape through exl3_gemm (the line above)
        ops._reconstruct_branch(x, lin["trellis"], lin["suh"], lin["svh"], K, 0)

    gg, side = _graph(dev, gemm)
    t_gemm = _time_graph(gg, side, reps)
    gr, side_r = _graph(dev, recon)
    t_rec = _time_graph(gr, side_r, reps)
    grt, side_rt = _graph(dev, recon_t)
    t_rect = _time_graph(grt, side_rt, reps)
    op()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream(dev)
    _settle(op, cur)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        op()
    e1.record()
    torch.cuda.synchronize()
    t_op = e0.elapsed_time(e1) * 1e-3 / reps
    flops = 2 * M * ic * oc
    rbytes = syn.packed_bytes(ic, oc, K) + 2 * ic * oc
    return {"gemm": {"us_per_call": round(t_gemm * 1e6, 2), "flop": flops,
                     "TFLOP/s": round(flops / t_gemm / 1e12, 2),
                     "mfma_util": round(flops / t_gemm / 1e12 / MFMA_F16_PEAK_TFS, 4),
                     "peak_TFLOP/s": MFMA_F16_PEAK_TFS,
                     "what": "exl3_gemm: had_r_128 pass + fused decode-into-MFMA kernel"},
            "op_route": "exl3_gemm" if ops._fused_route(M, ic, oc) else "reconstruct_branch",
            "reconstruct_branch": {"us_per_call": round(t_op * 1e6, 2),
                                   "TFLOP/s": round(flops / t_op / 1e12, 2),
                                   "mfma_util": round(flops / t_op / 1e12 / MFMA_F16_PEAK_TFS, 4),
                                   "what": "the reference's prefill branch at M=2048 (eager): had_r_128, "
                                           "reconstruct to (oc, ic), library fp16 transposed-B GEMM, "
                                           "had_r_128"},
            "reconstruct": {"us_per_call": round(t_rec * 1e6, 2), "bytes": rbytes,
                            "GB/s": round(rbytes / t_rec / 1e9, 1),
                            "frac": round(rbytes / t_rec / 1e9 / HBM_PEAK_GBS, 4)},
            "reconstruct_t": {"us_per_call": round(t_rect * 1e6, 2), "bytes": rbytes,
                              "GB/s": round(rbytes / t_rect / 1e9, 1),
                              "frac": round(rbytes / t_rect / 1e9 / HBM_PEAK_GBS, 4)}}


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(runs: int = 5) -> dict:
    """The reference's CPU path, timed on this host (median of `runs` after one warm-up run):

    * value (all os.cpu_count() threads): oracle trellis decode -> reconstruct_weight's fp32
      Hadamard/sign algebra (reference orcasaq2/__init__.py:49-61) -> F.linear
      (orcasaq2/config.py:230), one batch-1 GEMV at each K = 2, 3, 4, 5 of down_proj
      (17408 -> 5120) restricted to its first 512 output columns (a bounded sample; the
      rate is per packed byte, so it does not depend on the column count);
    * the same path on one thread (first 128 columns);
    * the activation-side ordering of the same math (orcasaq2/ops.py:53-59: H(x*suh), the
      decoded W_q, H(y)*svh) on all threads;
    * config 0: the full 5120 -> 5120 K=4 layer, batch 1, the reference ordering, all threads.
    """
    import torch
    from oracle import oracle as O
    from orcasaq2 import _t128
    from orcasaq2 import synthetic as syn

    threads = os.cpu_count() or 1
    x17 = syn.activations(1, syn.INTERMEDIATE, torch.Generator().manual_seed(11))

    def sample(ic, oc_cols, K, seed):
        lin = syn.linear(ic, syn.HIDDEN, K, seed=seed)
        return dict(trellis=lin["trellis"][:, :oc_cols // 16].contiguous(), suh=lin["suh"],
                    svh=lin["svh"][:oc_cols].contiguous(), K=K, ic=ic, oc=oc_cols)

    def weight_side(x, d, nthreads):
        """decode, H.W_q.H algebra on the weight, then the product; seconds per phase."""
        a = time.perf_counter()
        wq = torch.from_numpy(O.reconstruct_f16(d["trellis"], d["K"], 0, nthreads=nthreads))
        b = time.perf_counter()
        w = wq.float()
        w = _t128(w.t()).t() * d["suh"].float().unsqueeze(1)
        w = _t128(w) * d["svh"].float().unsqueeze(0)
        w = w.t().contiguous().half()
        c = time.perf_counter()
        y = torch.nn.functional.linear(x, w)
        e = time.perf_counter()
        assert y.shape == (1, d["oc"])
        return b - a, c - b, e - c

    def act_side(x, d, nthreads):
        a = time.perf_counter()
        wq = torch.from_numpy(O.reconstruct_f16(d["trellis"], d["K"], 0, nthreads=nthreads))
        b = time.perf_counter()
        xh = _t128(x.float() * d["suh"].float()).half()
        y = (xh.float() @ wq.float()).half()
        y = (_t128(y.float()) * d["svh"].float()).half()
        c = time.perf_counter()
        assert y.shape == (1, d["oc"])
        return b - a, c - b, 0.0

    def median_rate(fn, ds, x, nthreads):
        torch.set_num_threads(nthreads)
        nbytes = sum(syn.packed_bytes(d["ic"], d["oc"], d["K"]) for d in ds)
        for d in ds:                          # warm-up run
            fn(x, d, nthreads)
        totals, phases = [], []
        for _ in range(runs):
            p = [fn(x, d, nthreads) for d in ds]
            phases.append([sum(v[i] for v in p) for i in range(3)])
            totals.append(sum(phases[-1]))
        med = statistics.median(totals)
        ph = phases[totals.index(sorted(totals)[len(totals) // 2])]
        return nbytes / med / 1e9, med, ph, nbytes

    wide = [sample(syn.INTERMEDIATE, 512, K, seed=K) for K in (2, 3, 4, 5)]
    narrow = [dict(d, trellis=d["trellis"][:, :8].contiguous(), svh=d["svh"][:128].contiguous(), oc=128)
              for d in wide]
    v_all, t_all, ph_all, nb_all = median_rate(weight_side, wide, x17, threads)
    v_one, t_one, ph_one, nb_one = median_rate(weight_side, narrow, x17, 1)
    v_act, t_act, ph_act, _ = median_rate(act_side, wide, x17, threads)
    c0 = syn.linear(syn.HIDDEN, syn.HIDDEN, 4, seed=0)
    c0 = dict(c0, K=4)
    x0 = syn.activations(1, syn.HIDDEN, torch.Generator().manual_seed(0))
    v_c0, t_c0, _, nb_c0 = median_rate(weight_side, [c0], x0, threads)
    return {"value": round(v_all, 5), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"reference CPU path (oracle C decode + reconstruct_weight fp32 Hadamard algebra + "
                      f"F.linear), one batch-1 GEMV at each K=2,3,4,5 of down_proj 17408->5120 restricted "
                      f"to its first 512 outputs ({nb_all / 1e6:.1f} MB packed), median of {runs} runs on "
                      f"{threads} threads: {t_all:.2f} s per run (decode {ph_all[0]:.2f}, hadamard "
                      f"{ph_all[1]:.2f}, matmul {ph_all[2]:.3f}); CPU: {_cpu_model()}",
            "one_thread": {"value": round(v_one, 5), "unit": "GB/s", "s_per_run": round(t_one, 3),
                           "sample": f"same path, first 128 outputs ({nb_one / 1e6:.2f} MB packed), 1 thread"},
            "activation_side": {"value": round(v_act, 5), "unit": "GB/s", "s_per_run": round(t_act, 3),
                                "sample": "orcasaq2/ops.py:53-59 ordering (H(x*suh), decoded W_q, "
                                          f"H(y)*svh), same sample, {threads} threads; decode "
                                          f"{ph_act[0]:.2f} s, rest {ph_act[1]:.3f} s"},
            "config0": {"value": round(v_c0, 5), "unit": "GB/s", "s_per_run": round(t_c0, 3),
                        "sample": f"5120->5120 K=4 batch 1 ({nb_c0 / 1e6:.1f} MB packed), reference ordering, "
                                  f"{threads} threads"}}


CEILING_OPS = {1: "v_add_u32", 2: "v_bitop3_b32", 3: "v_lshrrev_b32", 4: "v_mul_lo_u32", 5: "v_bfe_u32",
               6: "v_alignbit_b32", 7: "v_add_u32_sdwa", 8: "v_perm_b32", 9: "v_lshlrev_b32", 10: "v_mov_b32_dpp",
               11: "v_mad_u64_u32", 12: "v_mfma_f32_4x4x4_16b_f16", 13: "v_mfma_f32_16x16x32_f16",
               14: "4x4x4 MFMA waves beside v_mul_lo_u32 waves", 15: "16x16x32 MFMA waves beside v_mul_lo_u32 waves"}


def ceiling_bench(reps: int) -> dict:
    """What bounds the batch-1 GEMV (down_proj 17408 -> 5120): the measurement kernels of
    libexl3ceiling.so walk the same units, workgroup ranges, wave runs and load ring as
    gemv1_kernel but stop short of parts of its work (empty grid / loads only / loads +
    three-instruction decode / loads + decode + the 16 MFMAs per unit with activations from a
    constant LDS table), timed per call in HIP graphs over rotating weight copies exactly like
    config 1, beside a plain coalesced dwordx4 stream of the same bytes (what HBM gives a
    read of this size at all) and the product GEMV itself; then the issue cost of the decode's instructions
    and of the MFMA forms (8 independent chains per wave, 8 waves per SIMD)."""
    import ctypes
    import torch
    from orcasaq2 import _native
    path = os.path.join(ROOT, "orcasaq2-kernel_amd", "orcasaq2", "libexl3ceiling.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (python orcasaq2-kernel_amd/build_lib.py)")
    M = ctypes.CDLL(path)
    M.exl3m_stream.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                               ctypes.c_void_p, ctypes.c_void_p]
    M.exl3m_ops.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    M.exl3m_plain.argtypes = [ctypes.c_void_p, ctypes.c_long, ctypes.c_void_p, ctypes.c_void_p]
    M.exl3m_sink_bytes.restype = ctypes.c_long
    M.exl3m_stream_workgroups.argtypes = [ctypes.c_int, ctypes.c_int]
    M.exl3m_sink_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
    dev = torch.device("cuda", 0)
    ic, oc, calls = 17408, 5120, 30
    sink = torch.empty(M.exl3m_sink_bytes(ic, oc), dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev).manual_seed(7)
    out, names = {}, ["empty grid", "loads only", "loads + decode", "loads + decode + MFMA (constant activations)",
                      "same with 16x16x32 MFMAs"]
    for K in (2, 3, 4, 5):
        nbytes = ic * oc * K // 8
        copies = [_rand_linear(ic, oc, K, g, dev) for _ in range(max(2, math.ceil(ROTATE_BYTES / nbytes)))]
        x = torch.randn(1, ic, generator=g, device=dev).half()
        y = torch.empty(1, oc, dtype=torch.half, device=dev)
        row = {"bytes": nbytes}
        for mode in range(5):
            def run(mode=mode):
                st = torch.cuda.current_stream(dev).cuda_stream
                for i in range(calls):
                    rc = M.exl3m_stream(mode, copies[i % len(copies)]["trellis"].data_ptr(), ic, oc, K,
                                        sink.data_ptr(), st)
                    if rc != 0:
                        raise RuntimeError(f"exl3m_stream mode {mode} K={K}: {rc}")
            gr, side = _graph(dev, run, settle=False)
            us = _time_graph(gr, side, reps) / calls * 1e6
            row[names[mode]] = {"us": round(us, 2), "GB/s": round(nbytes / us / 1e3, 1)}

        def plain():
            st = torch.cuda.current_stream(dev).cuda_stream
            for i in range(calls):
                rc = M.exl3m_plain(copies[i % len(copies)]["trellis"].data_ptr(), nbytes, sink.data_ptr(), st)
                if rc != 0:
                    raise RuntimeError(f"exl3m_plain K={K}: {rc}")
        gr, side = _graph(dev, plain, settle=False)
        us = _time_graph(gr, side, reps) / calls * 1e6
        row["plain dwordx4 stream of the same bytes"] = {"us": round(us, 2), "GB/s": round(nbytes / us / 1e3, 1)}

        def prod():
            for i in range(calls):
                d = copies[i % len(copies)]
                _native.gemv(x, d["trellis"], d["suh"], d["svh"], K, 0, out=y)
        gr, side = _graph(dev, prod)
        us = _time_graph(gr, side, reps) / calls * 1e6
        row["product gemv1_kernel"] = {"us": round(us, 2), "GB/s": round(nbytes / us / 1e3, 1)}
        out[f"K={K}"] = row
        del copies
        torch.cuda.empty_cache()
    iters, ops = 500, {}
    waves_per_simd = 8
    for op, name in CEILING_OPS.items():
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st = torch.cuda.current_stream(dev).cuda_stream
        M.exl3m_ops(op, 10, sink.data_ptr(), st)
        best = 1e9
        for _ in range(3):
            e0.record()
            if M.exl3m_ops(op, iters, sink.data_ptr(), st) != 0:
                raise RuntimeError(f"exl3m_ops {op}")
            e1.record()
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e-3)
        ns = best * 1e9 / (waves_per_simd * iters * 32)
        ops[name] = {"ns_per_wave_instr_per_simd": round(ns, 3), "cycles_at_2.1GHz": round(ns * 2.1, 2)}
    return {"shape": "down_proj 17408->5120, batch 1, one shard per call, 30 calls per graph over rotating copies",
            "per_call": out, "instruction_issue": ops}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only-K", type=int, default=0, help="time a single K (profiling runs)")
    ap.add_argument("--copy-calib", action="store_true", help="run the counter-calibration copy and exit")
    ap.add_argument("--workload", default="config1",
                    choices=("config1", "config2", "config3", "config4", "lmhead", "prefill", "ceiling"),
                    help="config1 = the headline line (+ the config-4 stack); config2/config3/config4 "
                         "print their own measurement line")
    ap.add_argument("--no-stack", action="store_true", help="skip the config-4 stack measurement")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the EXL3 linear path has no "
              "multi-GPU code); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.copy_calib:
        copy_calib(args)
        return
    if args.workload in ("config2", "config3", "config4", "lmhead", "prefill", "ceiling"):
        import torch
        res = (config2_bench(args.steps * 5) if args.workload == "config2" else
               lmhead_bench(args.steps * 5) if args.workload == "lmhead" else
               ceiling_bench(args.steps) if args.workload == "ceiling" else
               config3_bench(args.steps) if args.workload == "config3" else
               prefill_bench(args.steps) if args.workload == "prefill" else stack_bench(args.steps))
        print(json.dumps({"workload": args.workload, "results": res,
                          "device": torch.cuda.get_device_name(0)}), flush=True)
        return
    r = gpu_bench(args)
    dom = r["per_k"][r["dom"]]
    traffic = load_traffic(r["dom"], dom["bytes"])
    out = {
        "metric": METRIC,
        "value": round(r["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["wall"] / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "config1: down_proj 17408->5120, batch 1, fused decode-GEMV at K=2,3,4,5 "
                               "(3INST codebook), weights rotated over >512 MB per K",
                   "hbm_frac": round(r["value"] / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(dom["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["frac"], 4), "traffic": traffic,
                     "kernel": f"exl3_gemv K={r['dom']}: gemv1_kernel<{r['dom']}, 0, true, 1> (one call = one decode "
                               "launch; its split column groups are finished inside it)",
                     "bytes_per_launch": dom["bytes"], "mean_launch_us": round(dom["mean_us"], 3)},
        "per_K": {str(K): {"GB/s": round(v["gbs"], 1), "frac": round(v["frac"], 4),
                           "mean_us": round(v["mean_us"], 3)} for K, v in r["per_k"].items()},
        "device": r["device"],
    }
    if not args.no_stack and not args.only_K:
        st = stack_bench()
        out["tok_s_equiv"] = st["tok_s"]
        out["stack"] = st
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
