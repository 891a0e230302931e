"""Committed fixtures (tests/golden/exl3_golden.npz, made by tests/golden/make_golden.py)
against the oracle on the CPU and the HIP library on the GPU."""
import hashlib
import os

import numpy as np
import pytest
import torch

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "exl3_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)  # allow_pickle defaults to False


@pytest.mark.parametrize("cb", [0, 1])
def test_oracle_codebook_matches_fixture(oracle, gold, cb):
    t = oracle.codebook_table(cb)
    assert hashlib.sha256(t.tobytes()).digest() == gold[f"cb{cb}_sha256"].tobytes()
    assert np.array_equal(t[gold[f"cb{cb}_idx"]], gold[f"cb{cb}_val"])


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1])
def test_oracle_reconstruct_matches_fixture(oracle, gold, K, cb):
    assert np.array_equal(oracle.reconstruct(gold[f"rec_K{K}_cb{cb}_trellis"], K, cb), gold[f"rec_K{K}_cb{cb}_W"])


def test_oracle_linear_matches_fixture(oracle, gold):
    y = oracle.shard_gemm_ref(gold["lin_x"], gold["lin_trellis"], gold["lin_suh"], gold["lin_svh"], int(gold["lin_K"]))
    assert np.array_equal(y, gold["lin_y"])


@pytest.mark.gpu
@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1])
def test_hip_reconstruct_matches_fixture(native, gold, K, cb):
    tr = torch.from_numpy(gold[f"rec_K{K}_cb{cb}_trellis"].view(np.int16)).cuda()
    W = native.reconstruct(tr, K, cb)
    assert np.array_equal(W.cpu().view(torch.int16).numpy().view(np.uint16), gold[f"rec_K{K}_cb{cb}_W"])


@pytest.mark.gpu
def test_hip_linear_matches_fixture(native, gold):
    d = torch.device("cuda", 0)
    tr = torch.from_numpy(gold["lin_trellis"].view(np.int16)).to(d)
    args = [torch.from_numpy(gold[k]).to(d) for k in ("lin_x", "lin_suh", "lin_svh")]
    y = native.gemv(args[0], tr, args[1], args[2], int(gold["lin_K"]), 0).cpu().numpy().astype(np.float64)
    ref = gold["lin_y"]
    err = np.linalg.norm(y - ref, axis=1) / np.linalg.norm(ref, axis=1)
    assert err.max() <= 1e-3
