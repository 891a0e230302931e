"""Benchmark of the MI355X EXL3 trellis linear path (BASELINE.json metric):
bs=1 fused EXL3 GEMV, packed-weight GB/s and fraction of HBM peak.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--workload config1]

Workload: down_proj 17408 -> 5120 at batch 1 through the fused
decode-GEMV at K = 2, 3, 4 and 5 bits.  One step = one GEMV at each K.  Every GEMV reads a
different copy of the weights (more than 512 MB of distinct packed words per K), so the
256 MB Infinity Cache cannot serve a repeat: the bytes come from HBM.  Inputs are
resident in HBM before the timed region starts.

The timed steps are replayed from a HIP graph (captured once, the way decode serving
replays its steps), so host launch overhead is not part of the measurement; the
warm-up steps are a graph replay too.
`value` = total packed trellis bytes / total time over the timed steps.
`roofline` = the dominant GEMV (the K whose calls take the most time; one call = one
gemv1_kernel<K> launch): algorithmic bytes per call (ic*oc*K/8) / its mean duration from
HIP events recorded on the replay stream around a graph of the same steps, against
8 TB/s.  `traffic` = HBM bytes per call measured with
rocprofv3 FETCH_SIZE + WRITE_SIZE and scaled by the same counters' reading for a plain
copy of known size (profiles/gemv_traffic.json; `python bench.py --copy-calib` is the
calibration workload).
`cpu_baseline` = the reference's CPU path restated by the oracle (trellis decode in C, the
reconstruct_weight Hadamard/sign algebra in fp32 torch, F.linear), timed on this host's
cores on one step of the same workload.
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
ROTATE_BYTES = 600 * 2 ** 20
STACK_BYTES_PER_TOKEN = None  # filled from the seeded config-4 draw


def stack_token_bytes() -> int:
    from orcasaq2 import synthetic as syn
    shapes = syn.stack_shapes()
    total = 0
    for layer in syn.stack_bits():
        for name, K in layer.items():
            ic, oc = shapes[name]
            total += syn.packed_bytes(ic, oc, K)
    total += syn.packed_bytes(syn.HIDDEN, syn.VOCAB, 6)  # K=6 lm_head
    total += syn.HIDDEN + 2                            # int8 embedding row + its scale
    return total


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
    synchronisation.  Per-K figures come from one graph per K, timed with HIP events on
    the capture stream."""
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
    g_warm.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g_timed.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    per_k = {}
    for K in Ks:
        gk = capture(args.warmup, args.steps, only=(K,))
        gk.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(side)
        with torch.cuda.stream(side):
            gk.replay()
        e1.record(side)
        torch.cuda.synchronize()
        mean = e0.elapsed_time(e1) * 1e-3 / args.steps
        nbytes = syn.packed_bytes(ic, oc, K)
        per_k[K] = dict(bytes=nbytes, mean_us=mean * 1e6, gbs=nbytes / mean / 1e9,
                        frac=nbytes / mean / 1e9 / HBM_PEAK_GBS, total_s=mean * args.steps)
        del gk
    total_bytes = sum(per_k[K]["bytes"] for K in Ks) * args.steps
    value = total_bytes / wall / 1e9
    dom = max(Ks, key=lambda K: per_k[K]["total_s"])
    tok_bytes = stack_token_bytes()
    return dict(value=value, wall=wall, per_k=per_k, dom=dom, tok_bytes=tok_bytes,
                device=torch.cuda.get_device_name(dev))


def cpu_baseline(max_seconds: float = 30.0) -> dict:
    """The reference's CPU path on one step of the workload (K = 2, 3, 4, 5 GEMVs):
    oracle trellis decode -> reconstruct_weight's fp32 Hadamard/sign algebra
    (orcasaq2/__init__.py:58-61) -> F.linear (orcasaq2/config.py:230)."""
    import torch
    from oracle import oracle as O
    from orcasaq2 import _t128
    from orcasaq2 import synthetic as syn

    # this host's share of cores for one GPU (the GPU boxes grant 16 per GPU)
    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    ic, oc = syn.INTERMEDIATE, syn.HIDDEN
    x = syn.activations(1, ic, torch.Generator().manual_seed(11))
    t_dec = t_had = t_mm = 0.0
    nbytes = 0
    t_start = time.perf_counter()
    for K in (2, 3, 4, 5):
        lin = syn.linear(ic, oc, K, seed=K)
        a = time.perf_counter()
        wq = torch.from_numpy(O.reconstruct_f16(lin["trellis"], K, 0, nthreads=threads))
        b = time.perf_counter()
        w = wq.float()
        w = _t128(w.t()).t() * lin["suh"].float().unsqueeze(1)
        w = _t128(w) * lin["svh"].float().unsqueeze(0)
        w = w.t().contiguous().half()
        c = time.perf_counter()
        y = torch.nn.functional.linear(x, w)
        d = time.perf_counter()
        assert y.shape == (1, oc)
        t_dec += b - a
        t_had += c - b
        t_mm += d - c
        nbytes += syn.packed_bytes(ic, oc, K)
        if time.perf_counter() - t_start > max_seconds:
            break
    total = t_dec + t_had + t_mm
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": nbytes / total / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"one step of the workload ({nbytes / 1e6:.1f} MB packed: down_proj at "
                      "K=2,3,4,5): oracle C decode (OpenMP) + fp32 torch Hadamard algebra + "
                      f"fp16 F.linear; decode {t_dec:.2f}s, hadamard {t_had:.2f}s, "
                      f"matmul {t_mm:.2f}s; CPU: {cpu}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only-K", type=int, default=0, help="time a single K (profiling runs)")
    ap.add_argument("--copy-calib", action="store_true", help="run the counter-calibration copy and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the EXL3 linear path has no "
              "multi-GPU code); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.copy_calib:
        copy_calib(args)
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
                     "kernel": f"exl3_gemv K={r['dom']}: gemv1_kernel<{r['dom']}, 0> (one launch per call)",
                     "bytes_per_launch": dom["bytes"], "mean_launch_us": round(dom["mean_us"], 3)},
        "per_K": {str(K): {"GB/s": round(v["gbs"], 1), "frac": round(v["frac"], 4),
                           "mean_us": round(v["mean_us"], 3)} for K, v in r["per_k"].items()},
        "tok_s_equiv": round(r["value"] * 1e9 / r["tok_bytes"], 1),
        "tok_s_equiv_note": "config-1 aggregate GB/s / config-4 packed bytes per token "
                            f"({r['tok_bytes']} B); attention and KV excluded",
        "device": r["device"],
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
