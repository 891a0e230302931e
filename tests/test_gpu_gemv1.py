"""GPU parity of the 1..4-row decode-GEMV (gemv1.hip), mostly at one activation row, through
the C ABI.

The batch-1 kernel cuts a launch's tile-row units into equal contiguous ranges, one per
workgroup, so one column group can be split over several workgroups and one workgroup can
touch several column groups (and shards).  These cases cover: a column group inside one
workgroup, split over several, workgroups spanning 2-3 column groups and a shard
boundary, waves left without units, every K and both codebooks, grouped shards with mixed
K, the workspace's reserved head left untouched and its accumulator area left zero after
calls of every kind (split column groups are summed there and finished by the workgroup whose
add completes the count), one column group split over some 500 workgroups, determinism, and
the config-4
lm_head shape (5120 -> 151936, K = 6) checked on sampled column groups, at 1 row and at
2..4 rows (the four-row template on more workgroups than stay resident); and a shard too
large for the four-row template's LDS, which 2..4-row calls hand to gemv16.  Bar: per-row
relative L2 error <= 1e-3 against the fp64 oracle on the same fp16 inputs.
"""
import numpy as np
import pytest
import torch

from orcasaq2 import synthetic as syn

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


def dev():
    return torch.device("cuda", 0)


def to_gpu(d):
    return {k: (v.to(dev()) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


def check(y, x, lin, cb, oracle):
    ref = oracle.shard_gemm_ref(x.numpy(), lin["trellis"], lin["suh"].numpy(), lin["svh"].numpy(), lin["K"], cb)
    err = oracle.rel_err_rows(y.detach().cpu().numpy(), ref)
    assert err.max() <= REL_TOL, err.max()


@pytest.mark.parametrize("ic,oc", [(128, 128), (256, 1024), (1024, 128), (640, 3200), (5120, 1024),
                                   (2048, 2048)])
@pytest.mark.parametrize("K", [2, 3, 4, 5])
def test_gemv1_shapes(native, oracle, ic, oc, K):
    lin = syn.linear(ic, oc, K, seed=ic + oc + K)
    x = syn.activations(1, ic, torch.Generator().manual_seed(K))
    d = to_gpu(lin)
    y = native.gemv(x.to(dev()), d["trellis"], d["suh"], d["svh"], K, 0)
    check(y, x, lin, 0, oracle)


@pytest.mark.parametrize("K", [1, 6, 7, 8])
@pytest.mark.parametrize("cb", [0, 1])
def test_gemv1_other_K_and_mcg(native, oracle, K, cb):
    lin = syn.linear(768, 1536, K, seed=50 + K)
    x = syn.activations(1, 768, torch.Generator().manual_seed(K + 10 * cb))
    d = to_gpu(lin)
    y = native.gemv(x.to(dev()), d["trellis"], d["suh"], d["svh"], K, cb)
    check(y, x, lin, cb, oracle)


def test_gemv1_grouped_mixed_K(native, oracle):
    """Four shards, three with K=3 (one launch: workgroups cross shard boundaries) and one
    with K=5 (its own launch), written side by side."""
    spec = [(384, 3), (1024, 3), (128, 5), (2560, 3)]
    lins = [syn.linear(1024, oc, K, seed=300 + i) for i, (oc, K) in enumerate(spec)]
    x = syn.activations(1, 1024, torch.Generator().manual_seed(31))
    y = native.gemv_grouped(x.to(dev()), [dict(to_gpu(l), codebook=0) for l in lins])
    col = 0
    for l in lins:
        check(y[:, col:col + l["oc"]], x, l, 0, oracle)
        col += l["oc"]


@pytest.mark.parametrize("rows", [1, 3, 4])
def test_gemv1_table_tasks_cross_several_shards(native, oracle, rows):
    """Eight 128-output shards over 128 inputs (one input block per column group): a launch
    of 64 units on two workgroups, whose waves' activation-table tasks step over several
    segments at once and so cross two shard boundaries in one wave's walk (four rows: a
    wave's tasks are occurrences 0, 2, 4 = shards 0, 2, 4)."""
    lins = [syn.linear(128, 128, 3, seed=400 + i) for i in range(8)]
    x = syn.activations(rows, 128, torch.Generator().manual_seed(41 + rows))
    y = native.gemv_grouped(x.to(dev()), [dict(to_gpu(l), codebook=0) for l in lins])
    for i, l in enumerate(lins):
        check(y[:, 128 * i:128 * (i + 1)], x, l, 0, oracle)
    ragged = [syn.linear(256, oc, 4, seed=420 + i) for i, oc in enumerate([384, 128, 640, 128, 256, 128, 1152, 128])]
    x2 = syn.activations(rows, 256, torch.Generator().manual_seed(43))
    y = native.gemv_grouped(x2.to(dev()), [dict(to_gpu(l), codebook=0) for l in ragged])
    col = 0
    for l in ragged:
        check(y[:, col:col + l["oc"]], x2, l, 0, oracle)
        col += l["oc"]


def test_gemv1_workspace_head_untouched_and_deterministic(native):
    """Repeated calls give identical outputs, and no kernel writes the workspace's reserved
    16 KiB head (filled with a marker here, which it must keep)."""
    lin = to_gpu(syn.linear(4096, 2048, 4, seed=77))
    x = syn.activations(1, 4096, torch.Generator().manual_seed(7)).to(dev())
    y0 = native.gemv(x, lin["trellis"], lin["suh"], lin["svh"], 4, 0)
    key = (0, torch.cuda.current_stream(dev()).cuda_stream)
    ws = native._gemv_ws[key]
    ws[:16384].fill_(0xA5)
    ys = [native.gemv(x, lin["trellis"], lin["suh"], lin["svh"], 4, 0) for _ in range(5)]
    torch.cuda.synchronize()
    assert native._gemv_ws[key].data_ptr() == ws.data_ptr()
    for y in ys:
        assert torch.equal(y, y0)
    assert bool((ws[:16384] == 0xA5).all())


ACC0, ACC1 = 16384, 16384 + (6 << 20)   # the workspace's accumulator area


@pytest.mark.parametrize("rows", [1, 3])
def test_gemv1_accumulators_left_zero_between_calls(native, oracle, rows):
    """Split column groups are summed in the workspace's accumulator words; the add that
    completes a word's count finishes the output and clears the word.  Calls of different
    shapes, row counts and shard groupings, interleaved on one workspace, each reproduce
    their first result bit for bit and leave the whole area zero -- so no call sees another's
    leftovers."""
    down = syn.linear(17408, 5120, 4, seed=81)
    qkv = [syn.linear(5120, oc, K, seed=82 + i) for i, (oc, K) in enumerate([(6144, 4), (1024, 5), (1024, 5)])]
    xd = syn.activations(rows, 17408, torch.Generator().manual_seed(83))
    xq = syn.activations(rows, 5120, torch.Generator().manual_seed(84))
    dg = to_gpu(down)
    qg = [dict(to_gpu(l), codebook=0) for l in qkv]
    key = (0, torch.cuda.current_stream(dev()).cuda_stream)
    first = {}
    for it in range(3):
        for name in ("down", "qkv", "down1"):
            if name == "qkv":
                y = native.gemv_grouped(xq.to(dev()), qg)
            else:
                x = xd.to(dev()) if name == "down" else xd[:1].to(dev())
                y = native.gemv(x, dg["trellis"], dg["suh"], dg["svh"], 4, 0)
            torch.cuda.synchronize()
            ws = native._gemv_ws[key]
            nz = int((ws[ACC0:ACC1] != 0).sum())
            assert nz == 0, f"{name} rows={rows} call {it}: {nz} accumulator bytes left non-zero"
            if it == 0:
                first[name] = y.clone()
            else:
                assert torch.equal(y, first[name]), (name, it)
    check(first["down"], xd, down, 0, oracle)
    check(first["down1"], xd[:1], down, 0, oracle)
    col = 0
    for l in qkv:
        check(first["qkv"][:, col:col + l["oc"]], xq, l, 0, oracle)
        col += l["oc"]


def test_gemv1_one_column_group_over_many_workgroups(native, oracle):
    """A 262144 -> 128 shard (K = 2): its single column group's 16384 tile rows are split over
    every workgroup of the launch (some 500), all adding into the same 128 words."""
    lin = syn.linear(262144, 128, 2, seed=85)
    x = syn.activations(1, 262144, torch.Generator().manual_seed(86))
    g = to_gpu(lin)
    ys = [native.gemv(x.to(dev()), g["trellis"], g["suh"], g["svh"], 2, 0) for _ in range(3)]
    torch.cuda.synchronize()
    check(ys[0], x, lin, 0, oracle)
    assert torch.equal(ys[1], ys[0]) and torch.equal(ys[2], ys[0])


def test_gemv1_lm_head_sampled_column_groups(native, oracle):
    """Config-4 lm_head, 5120 -> 151936 at K=6 (1187 column groups, three per workgroup
    range): compare four column groups with the oracle on the matching trellis slice."""
    ic, oc, K = 5120, 151936, 6
    g = torch.Generator().manual_seed(4)
    t = syn.trellis(ic, oc, K, g)
    suh = syn.signs(ic, g)
    svh = syn.svh(ic, oc, g)
    x = syn.activations(1, ic, torch.Generator().manual_seed(41))
    y = native.gemv(x.to(dev()), t.to(dev()), suh.to(dev()), svh.to(dev()), K, 0).cpu()
    for cg in (0, 1, 593, 1186):
        sl = slice(cg * 128, (cg + 1) * 128)
        lin = dict(trellis=t[:, cg * 8:(cg + 1) * 8].contiguous(), suh=suh, svh=svh[sl].contiguous(), K=K)
        check(y[:, sl], x, lin, 0, oracle)


@pytest.mark.parametrize("rows", [2, 3, 4])
def test_gemv1_2_to_4_rows_on_the_lm_head(native, oracle, rows):
    """2..4 rows of the lm_head shape (5120 -> 151936, K=6): with four activation rows a
    workgroup range's tables leave fewer than three workgroups per CU resident, so the launch
    takes G1_GMAX workgroups that run in turn, and each wave keeps two units in flight (the
    deep four-row kernel); four column groups are checked against the oracle on the matching
    trellis slice."""
    ic, oc, K = 5120, 151936, 6
    g = torch.Generator().manual_seed(5)
    t = syn.trellis(ic, oc, K, g)
    suh = syn.signs(ic, g)
    svh = syn.svh(ic, oc, g)
    x = syn.activations(rows, ic, torch.Generator().manual_seed(42 + rows))
    y = native.gemv(x.to(dev()), t.to(dev()), suh.to(dev()), svh.to(dev()), K, 0).cpu()
    for cg in (0, 7, 600, 1186):
        sl = slice(cg * 128, (cg + 1) * 128)
        lin = dict(trellis=t[:, cg * 8:(cg + 1) * 8].contiguous(), suh=suh, svh=svh[sl].contiguous(), K=K)
        check(y[:, sl], x, lin, 0, oracle)


def test_gemv_2_to_4_rows_beyond_gemv1s_lds_take_gemv16(native, oracle):
    """A 16384 -> 163840 shard (K=1, 2.7e9 weights): at 2..4 rows gemv1's plan refuses it
    (a workgroup range's activation tables would exceed a CU's LDS even at G1_GMAX
    workgroups) and the call takes gemv16.  Sampled column groups against the oracle, and
    every column against the same rows run one at a time through gemv1."""
    ic, oc, K = 16384, 163840, 1
    g = torch.Generator(device=dev()).manual_seed(9)
    t = torch.randint(-32768, 32768, (ic // 16, oc // 16, 16 * K), generator=g, device=dev(),
                      dtype=torch.int32).to(torch.int16)
    gc = torch.Generator().manual_seed(10)
    suh = syn.signs(ic, gc)
    svh = syn.svh(ic, oc, gc)
    sd, vd = suh.to(dev()), svh.to(dev())
    for rows in (2, 3, 4):
        print(f"gemv rows={rows} 16384 x 163840 K=1", flush=True)
        x = syn.activations(rows, ic, torch.Generator().manual_seed(60 + rows))
        xd = x.to(dev())
        y = native.gemv(xd, t, sd, vd, K, 0)
        y1 = torch.cat([native.gemv(xd[r:r + 1], t, sd, vd, K, 0) for r in range(rows)])
        num = (y.float() - y1.float()).norm(dim=1)
        assert bool((num <= 1e-3 * y1.float().norm(dim=1)).all()), num
        y = y.cpu()
        for cg in (0, 311, 1279):
            sl = slice(cg * 128, (cg + 1) * 128)
            lin = dict(trellis=t[:, cg * 8:(cg + 1) * 8].cpu().contiguous(), suh=suh, svh=svh[sl].contiguous(), K=K)
            check(y[:, sl], x, lin, 0, oracle)
