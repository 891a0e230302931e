"""Writes tests/golden/exl3_golden.npz: small fixed vectors of the EXL3 trellis path.

The reference ships no golden vectors for this path (its trellis arithmetic lives in the
absent exllamav3 extension), so these fixtures come from this build's CPU oracle after it
passed the pins in tests/test_oracle.py.  They freeze the format decisions (bit order,
state window, placement, codebooks) so any later change to oracle or kernels that moves a
single bit is caught, and they give the GPU tests an input/output pair that needs no
oracle run.  Regenerate with:  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402


def main():
    rng = np.random.default_rng(20261201)
    out = {}
    for cb in (O.CB_3INST, O.CB_MCG):
        t = O.codebook_table(cb)
        out[f"cb{cb}_sha256"] = np.frombuffer(hashlib.sha256(t.tobytes()).digest(), np.uint8)
        idx = np.sort(rng.choice(65536, 512, replace=False)).astype(np.uint32)
        out[f"cb{cb}_idx"] = idx
        out[f"cb{cb}_val"] = t[idx]
    for K in range(1, 9):
        for cb in (O.CB_3INST, O.CB_MCG):
            tr = rng.integers(0, 65536, (2, 3, 16 * K)).astype(np.uint16)
            out[f"rec_K{K}_cb{cb}_trellis"] = tr
            out[f"rec_K{K}_cb{cb}_W"] = O.reconstruct(tr, K, cb)
    # one 128 x 256 linear, 4 rows, K = 3, 3INST
    ic, oc, K, rows = 128, 256, 3, 4
    tr = rng.integers(0, 65536, (ic // 16, oc // 16, 16 * K)).astype(np.uint16)
    suh = rng.choice([-1.0, 1.0], ic).astype(np.float16)
    svh = (rng.choice([-1.0, 1.0], oc) * np.abs(rng.standard_normal(oc)) / np.sqrt(ic)).astype(np.float16)
    x = rng.standard_normal((rows, ic)).astype(np.float16)
    out["lin_trellis"] = tr
    out["lin_suh"] = suh
    out["lin_svh"] = svh
    out["lin_x"] = x
    out["lin_K"] = np.array(K)
    out["lin_y"] = O.shard_gemm_ref(x, tr, suh, svh, K, O.CB_3INST)
    np.savez_compressed(os.path.join(HERE, "exl3_golden.npz"), **out)
    print("wrote", os.path.join(HERE, "exl3_golden.npz"))


if __name__ == "__main__":
    main()
