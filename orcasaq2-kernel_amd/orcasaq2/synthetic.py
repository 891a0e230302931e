"""Seed-fixed synthetic EXL3 tensors and activations of the benchmark configurations.

All generation runs on the CPU with torch.Generator(seed), so the CPU baseline and the
GPU see identical bytes:
  * trellis: uniform random 16-bit words, int16 (ic/16, oc/16, 16K);
  * suh: random +-1 fp16 (ic);
  * svh: random +-1 times fp16(|N(0,1)| / sqrt(ic)) (oc) -- the per-output-channel scale
    folded into svh (the EXL3 tensor set has no separate scale tensor);
  * x: N(0,1) fp16 (rows, ic).
"""
from __future__ import annotations

import math
import random

import torch

HIDDEN = 5120
INTERMEDIATE = 17408
Q_OUT = 6144
KV_OUT = 1024
VOCAB = 151936
LAYERS = 64


def trellis(ic: int, oc: int, K: int, gen: torch.Generator) -> torch.Tensor:
    w = torch.randint(0, 65536, (ic // 16, oc // 16, 16 * K), generator=gen, dtype=torch.int32)
    return w.to(torch.int16)  # two's-complement wrap keeps the uint16 bit pattern


def signs(n: int, gen: torch.Generator) -> torch.Tensor:
    return (torch.randint(0, 2, (n,), generator=gen) * 2 - 1).to(torch.float16)


def svh(ic: int, oc: int, gen: torch.Generator) -> torch.Tensor:
    mag = (torch.randn(oc, generator=gen).abs() / math.sqrt(ic)).to(torch.float16)
    return mag * signs(oc, gen)


def activations(rows: int, ic: int, gen: torch.Generator) -> torch.Tensor:
    return torch.randn(rows, ic, generator=gen).to(torch.float16)


def linear(ic: int, oc: int, K: int, seed: int) -> dict:
    """One EXL3 tensor set: dict(trellis, suh, svh, ic, oc, K) on the CPU."""
    g = torch.Generator().manual_seed(seed)
    t = trellis(ic, oc, K, g)
    return dict(trellis=t, suh=signs(ic, g), svh=svh(ic, oc, g), ic=ic, oc=oc, K=K)


def stack_bits(seed: int = 4, layers: int = LAYERS) -> list[dict[str, int]]:
    """Per-projection K for the 64-layer Qwen-27B-shaped stack, drawn uniformly from
    {2, 3, 4, 5} with a fixed seed."""
    rng = random.Random(seed)
    names = ("q", "k", "v", "o", "gate", "up", "down")
    return [{n: rng.choice((2, 3, 4, 5)) for n in names} for _ in range(layers)]


def stack_shapes() -> dict[str, tuple[int, int]]:
    """(ic, oc) of each projection of one decoder layer."""
    return {"q": (HIDDEN, Q_OUT), "k": (HIDDEN, KV_OUT), "v": (HIDDEN, KV_OUT),
            "o": (Q_OUT, HIDDEN), "gate": (HIDDEN, INTERMEDIATE), "up": (HIDDEN, INTERMEDIATE),
            "down": (INTERMEDIATE, HIDDEN)}


def packed_bytes(ic: int, oc: int, K: int) -> int:
    return ic * oc * K // 8


# ---------------------------------------------------------------- device-side generation

CODEBOOK_RMS = 1.2437   # RMS of the 3INST codebook's 2^16 values


def linear_gpu(ic: int, oc: int, K: int, gen: torch.Generator, dev: torch.device) -> dict:
    """One synthetic EXL3 tensor set made on the GPU with a device generator (the same
    distributions as linear(): uniform 16-bit trellis words, +-1 suh, +-|N(0,1)|/sqrt(ic)
    svh) -- for the benchmark's many large tensors, which CPU generation would make slow."""
    t = torch.randint(-32768, 32768, (ic // 16, oc // 16, 16 * K), generator=gen, device=dev,
                      dtype=torch.int32).to(torch.int16)
    suh = (torch.randint(0, 2, (ic,), generator=gen, device=dev) * 2 - 1).half()
    sv = ((torch.randn(oc, generator=gen, device=dev).abs() / math.sqrt(ic)).half()
          * (torch.randint(0, 2, (oc,), generator=gen, device=dev) * 2 - 1).half())
    return dict(trellis=t, suh=suh, svh=sv, ic=ic, oc=oc, K=K, codebook=0)


def stack_gpu(dev: torch.device, seed: int = 4) -> dict:
    """Config 4 on the GPU: the 64-layer Qwen-27B-shaped linear stack (K per projection from
    stack_bits()), the K=6 lm_head, and the int8 embedding table with its fp16 row scales.
    The svh scales are divided by the codebook RMS, so each projection keeps its input's RMS
    and 257 chained projections stay finite in fp16.  Returns dict(layers, head, table,
    scales, nbytes) with nbytes = packed trellis bytes of a token plus one embedding row."""
    g = torch.Generator(device=dev).manual_seed(seed)
    shapes = stack_shapes()

    def lin(ic, oc, K):
        d = linear_gpu(ic, oc, K, g, dev)
        d["svh"] = (d["svh"].float() / CODEBOOK_RMS).half()
        return d

    layers, nbytes = [], 0
    for bits in stack_bits():
        layers.append({n: lin(*shapes[n], bits[n]) for n in shapes})
        nbytes += sum(packed_bytes(*shapes[n], bits[n]) for n in shapes)
    head = lin(HIDDEN, VOCAB, 6)
    nbytes += packed_bytes(HIDDEN, VOCAB, 6)
    table = torch.randint(-128, 128, (VOCAB, HIDDEN), generator=g, device=dev, dtype=torch.int8)
    scales = (torch.rand(VOCAB, 1, generator=g, device=dev) * 0.02 + 0.001).half()
    nbytes += HIDDEN + 2
    return dict(layers=layers, head=head, table=table, scales=scales, nbytes=nbytes)
