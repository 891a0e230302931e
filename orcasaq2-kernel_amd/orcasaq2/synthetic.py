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
