"""GPU parity on seeded random shapes, through the grouped C-ABI entry points: a fused layer
of 1..5 shards over one input width (128..2048), each shard with its own output width
(128..2048), K (1..8) and codebook (3INST or MCG), at rows drawn from 1..4 (the 1..4-row
kernel), 5..16 (gemv16) and 17..300 (the stream-K GEMM).  The CPU address replay covers the
kernels' index arithmetic on many more shapes; this sweep checks the numbers on the GPU.
Every case prints its parameters before it runs.  Bar: per-row relative L2 error <= 1e-3
against the fp64 oracle on the same fp16 inputs, for every shard's columns.
"""
import random

import pytest
import torch

from orcasaq2 import synthetic as syn

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
D = torch.device("cuda", 0)


def draw(rnd, rows_lo, rows_hi):
    ic = 128 * rnd.randint(1, 16)
    n = rnd.randint(1, 5)
    shards = [(128 * rnd.randint(1, 16), rnd.randint(1, 8), rnd.randint(0, 1)) for _ in range(n)]
    return rnd.randint(rows_lo, rows_hi), ic, shards


def run_case(native, oracle, case, rows, ic, shards, grouped):
    print(f"case {case}: rows={rows} ic={ic} shards(oc,K,cb)={shards}", flush=True)
    lins = [syn.linear(ic, oc, K, seed=1000 * case + i) for i, (oc, K, cb) in enumerate(shards)]
    x = syn.activations(rows, ic, torch.Generator().manual_seed(case))
    specs = [dict(trellis=l["trellis"].to(D), suh=l["suh"].to(D), svh=l["svh"].to(D), oc=l["oc"], K=l["K"],
                  codebook=cb) for l, (_, _, cb) in zip(lins, shards)]
    y = grouped(x.to(D), specs)
    torch.cuda.synchronize()
    col = 0
    for l, (oc, K, cb) in zip(lins, shards):
        ref = oracle.shard_gemm_ref(x.numpy(), l["trellis"], l["suh"].numpy(), l["svh"].numpy(), K, cb)
        err = oracle.rel_err_rows(y[:, col:col + oc].float().cpu().numpy(), ref)
        assert err.max() <= REL_TOL, (case, rows, ic, shards, err.max())
        col += oc


@pytest.mark.parametrize("case", range(30))
def test_random_gemv_1_to_4_rows(native, oracle, case):
    rows, ic, shards = draw(random.Random(7100 + case), 1, 4)
    run_case(native, oracle, 7100 + case, rows, ic, shards, native.gemv_grouped)


@pytest.mark.parametrize("case", range(25))
def test_random_gemv_5_to_16_rows(native, oracle, case):
    rows, ic, shards = draw(random.Random(7200 + case), 5, 16)
    run_case(native, oracle, 7200 + case, rows, ic, shards, native.gemv_grouped)


@pytest.mark.parametrize("case", range(20))
def test_random_gemm_17_to_300_rows(native, oracle, case):
    rows, ic, shards = draw(random.Random(7300 + case), 17, 300)
    run_case(native, oracle, 7300 + case, rows, ic, shards, native.gemm_grouped)
