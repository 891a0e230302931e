"""GPU parity of every HIP entry point against the CPU oracle, through the C ABI.

Bars: reconstruct and the int8 embedding gather are bit-exact; GEMV/GEMM outputs have a
per-row relative L2 error <= 1e-3 against the fp64 oracle evaluated on the same fp16
inputs (the fp16 output rounding alone is ~3e-4); the Hadamard kernel is within fp16
output rounding of the fp64 transform.
"""
import numpy as np
import pytest
import torch

from orcasaq2 import synthetic as syn

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3  # GEMV/GEMM per-row relative L2 error bound


def dev():
    return torch.device("cuda", 0)


def to_gpu(d):
    return {k: (v.to(dev()) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


def u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().numpy()


def test_single_hip_runtime_mapped(native):
    torch.zeros(1, device=dev())
    maps = open("/proc/self/maps").read()
    libs = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(libs) == 1, libs


# ---------------------------------------------------------------- reconstruct

@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1])
def test_reconstruct_bit_exact_small(native, oracle, K, cb):
    lin = syn.linear(256, 384, K, seed=10 * K + cb)
    W = native.reconstruct(lin["trellis"].to(dev()), K, cb)
    torch.cuda.synchronize()
    assert np.array_equal(u16(W), oracle.reconstruct(lin["trellis"], K, cb))


@pytest.mark.parametrize("ic,oc", [(16, 16), (16, 208), (48, 144), (32, 1040)])
def test_reconstruct_ragged_tile_counts(native, oracle, ic, oc):
    """tile-column counts that are not multiples of the 8-tile strip"""
    lin = syn.linear(ic, oc, 3, seed=ic + oc)
    W = native.reconstruct(lin["trellis"].to(dev()), 3, 0)
    assert np.array_equal(u16(W), oracle.reconstruct(lin["trellis"], 3, 0))


def test_reconstruct_bit_exact_config3_full(native, oracle):
    lin = syn.linear(17408, 5120, 4, seed=3)
    W = native.reconstruct(lin["trellis"].to(dev()), 4, 0)
    assert np.array_equal(u16(W), oracle.reconstruct(lin["trellis"], 4, 0))


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1])
def test_reconstruct_t_bit_exact_small(native, oracle, K, cb):
    """exl3_reconstruct_t writes W_q^T: the oracle's W_q transposed, bit for bit"""
    lin = syn.linear(384, 256, K, seed=10 * K + cb + 5)
    Wt = native.reconstruct_t(lin["trellis"].to(dev()), K, cb)
    assert tuple(Wt.shape) == (256, 384)
    assert np.array_equal(u16(Wt), oracle.reconstruct(lin["trellis"], K, cb).T)


@pytest.mark.parametrize("ic,oc", [(16, 16), (208, 16), (144, 48), (1040, 32), (48, 1040)])
def test_reconstruct_t_ragged_tile_counts(native, oracle, ic, oc):
    """tile-row counts that are not multiples of the transposed kernel's 8-tile band"""
    lin = syn.linear(ic, oc, 5, seed=ic + 3 * oc)
    Wt = native.reconstruct_t(lin["trellis"].to(dev()), 5, 1)
    assert np.array_equal(u16(Wt), oracle.reconstruct(lin["trellis"], 5, 1).T)


def test_reconstruct_t_config3_full(native, oracle):
    lin = syn.linear(17408, 5120, 4, seed=3)
    Wt = native.reconstruct_t(lin["trellis"].to(dev()), 4, 0)
    assert np.array_equal(u16(Wt), oracle.reconstruct(lin["trellis"], 4, 0).T)


# ---------------------------------------------------------------- hadamard

@pytest.mark.parametrize("pre,post,scale", [(False, False, 1.0), (True, False, 1.0), (False, True, 0.5),
                                            (True, True, 2.0)])
def test_had_r_128(native, oracle, pre, post, scale):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(7, 640, generator=g).half()
    p = syn.signs(640, g) if pre else None
    q = syn.svh(640, 640, g) if post else None
    y = native.had_r_128(x.to(dev()), pre=p.to(dev()) if pre else None, post=q.to(dev()) if post else None,
                         scale=scale)
    ref = oracle.had_r_128(x.numpy(), None if p is None else p.numpy(), None if q is None else q.numpy(), scale)
    err = np.abs(f16(y).astype(np.float64) - ref)
    assert (err <= np.abs(ref) * 2.0 ** -10 + 2.0 ** -24).all()


def test_had_r_128_4byte_aligned_pointers(native, oracle):
    """pointers that are 4- but not 16-byte aligned take the narrow kernel"""
    g = torch.Generator().manual_seed(7)
    buf = torch.randn(5 * 384 + 2, generator=g).half().to(dev())
    xv = buf[2:].view(5, 384)
    assert xv.data_ptr() % 16 == 4
    p = syn.signs(384, g)
    y = native.had_r_128(xv, pre=p.to(dev()))
    ref = oracle.had_r_128(xv.cpu().numpy(), p.numpy())
    err = np.abs(f16(y).astype(np.float64) - ref)
    assert (err <= np.abs(ref) * 2.0 ** -10 + 2.0 ** -24).all()


def test_had_r_128_in_place(native, oracle):
    g = torch.Generator().manual_seed(6)
    x = torch.randn(3, 256, generator=g).half()
    xd = x.to(dev())
    out = native.had_r_128(xd, out=xd)
    assert out.data_ptr() == xd.data_ptr()
    ref = oracle.had_r_128(x.numpy())
    assert np.abs(f16(xd).astype(np.float64) - ref).max() <= np.abs(ref).max() * 2.0 ** -10


# ---------------------------------------------------------------- GEMV

def check_linear_out(y, x, lin, cb, oracle, W=None):
    ref = oracle.shard_gemm_ref(x.numpy(), lin["trellis"], lin["suh"].numpy(), lin["svh"].numpy(),
                                lin["K"], cb, W=W)
    err = oracle.rel_err_rows(f16(y), ref)
    assert err.max() <= REL_TOL, err.max()
    return err.max()


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("rows", [1, 4, 5, 16])
def test_gemv_small_all_K(native, oracle, K, rows):
    """1..4 rows: the persistent kernel (4 rows in the MFMA's A operand); 5..16: gemv16 (the
    batch-1 decode on 4 x 2-tile units, one MFMA serving all 16 rows)"""
    lin = syn.linear(512, 384, K, seed=100 + K)
    x = syn.activations(rows, 512, torch.Generator().manual_seed(rows))
    d = to_gpu(lin)
    y = native.gemv(x.to(dev()), d["trellis"], d["suh"], d["svh"], K, 0)
    check_linear_out(y, x, lin, 0, oracle)


@pytest.mark.parametrize("rows", [1, 3, 16])
def test_gemv_mcg(native, oracle, rows):
    lin = syn.linear(256, 256, 4, seed=7)
    x = syn.activations(rows, 256, torch.Generator().manual_seed(3))
    d = to_gpu(lin)
    y = native.gemv(x.to(dev()), d["trellis"], d["suh"], d["svh"], 4, 1)
    check_linear_out(y, x, lin, 1, oracle)


@pytest.mark.parametrize("K", [2, 3, 4, 5])
def test_gemv_config1_down_proj(native, oracle, K):
    lin = syn.linear(17408, 5120, K, seed=1)
    x = syn.activations(1, 17408, torch.Generator().manual_seed(11))
    d = to_gpu(lin)
    y = native.gemv(x.to(dev()), d["trellis"], d["suh"], d["svh"], K, 0)
    check_linear_out(y, x, lin, 0, oracle)


def test_gemv_deterministic_and_workspace_rearmed(native):
    lin = to_gpu(syn.linear(1024, 1024, 3, seed=9))
    x = syn.activations(2, 1024, torch.Generator().manual_seed(2)).to(dev())
    ys = [native.gemv(x, lin["trellis"], lin["suh"], lin["svh"], 3, 0) for _ in range(4)]
    for y in ys[1:]:
        assert torch.equal(y, ys[0])


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 9, 16])
def test_gemv_grouped_config2(native, oracle, rows):
    """qkv: q K4 5120->6144, k/v K5 5120->1024; gate_up: 2 x K3 5120->17408.  Rows 2..4 take
    the 1..4-row kernel for both (gate_up at four rows with three workgroups per CU); 9 and
    16 rows the 5..16-row kernel (gemv16), qkv's mixed K in one launch."""
    x = syn.activations(rows, 5120, torch.Generator().manual_seed(20 + rows))
    for spec in ([(6144, 4), (1024, 5), (1024, 5)], [(17408, 3), (17408, 3)]):
        lins = [syn.linear(5120, oc, K, seed=200 + i) for i, (oc, K) in enumerate(spec)]
        shards = [dict(to_gpu(l), codebook=0) for l in lins]
        y = native.gemv_grouped(x.to(dev()), shards)
        col = 0
        for l in lins:
            check_linear_out(y[:, col:col + l["oc"]], x, l, 0, oracle)
            col += l["oc"]


@pytest.mark.parametrize("ic,ocs,K", [(128, [131200], 2), (256, [384, 128, 640], 3), (384, [1152], 5),
                                      (2048, [128], 4), (256, [2048, 2048], 4), (640, [128, 256, 128], 6)])
@pytest.mark.parametrize("rows", [1, 3])
def test_gemv1_workgroup_ranges(native, oracle, ic, ocs, K, rows):
    """1 and 3 rows with workgroup ranges that span several column groups and shards, start
    inside a 128-input block, or cover a whole launch."""
    x = syn.activations(rows, ic, torch.Generator().manual_seed(ic + K))
    lins = [syn.linear(ic, oc, K, seed=300 + i) for i, oc in enumerate(ocs)]
    shards = [dict(to_gpu(l), codebook=0) for l in lins]
    y = native.gemv_grouped(x.to(dev()), shards)
    col = 0
    for l in lins:
        check_linear_out(y[:, col:col + l["oc"]], x, l, 0, oracle)
        col += l["oc"]


@pytest.mark.parametrize("ic,ocs,K", [(128, [131200], 2), (256, [384, 128, 640], 3), (384, [1152], 5),
                                      (2048, [128], 4), (256, [2048, 2048], 4), (640, [128, 256, 128], 6),
                                      (1024, [2944], 3), (1024, [1408, 1536], 7)])
@pytest.mark.parametrize("rows", [7, 13])
def test_gemv16_workgroup_ranges(native, oracle, ic, ocs, K, rows):
    """5..16 rows (gemv16.hip) on the range-boundary shapes of the 1..4-row test: ranges that
    span several strips and shards, start inside a strip, or cover a whole launch; strips with
    one and with many contributing workgroups.  The last two are one odd-K group of 1472
    units on 46 workgroups, which the blocks take XCD by XCD (5 per XCD and 6 more: both
    parts of the block order)."""
    x = syn.activations(rows, ic, torch.Generator().manual_seed(ic + K + rows))
    lins = [syn.linear(ic, oc, K, seed=350 + i) for i, oc in enumerate(ocs)]
    shards = [dict(to_gpu(l), codebook=0) for l in lins]
    y = native.gemv_grouped(x.to(dev()), shards)
    col = 0
    for l in lins:
        check_linear_out(y[:, col:col + l["oc"]], x, l, 0, oracle)
        col += l["oc"]
    assert torch.equal(native.gemv_grouped(x.to(dev()), shards), y)


@pytest.mark.parametrize("rows", [1, 3, 9])
def test_gemv_grouped_mixed_K_and_codebooks(native, oracle, rows):
    """Shards of several K (interleaved, so a group is not a contiguous run of shards) and
    both codebooks in one grouped call; at batch 1 each codebook's groups share a launch."""
    spec = [(384, 3, 0), (256, 5, 0), (128, 3, 1), (640, 2, 0), (256, 3, 0), (128, 6, 1), (384, 5, 0)]
    x = syn.activations(rows, 768, torch.Generator().manual_seed(40 + rows))
    lins = [syn.linear(768, oc, K, seed=400 + i) for i, (oc, K, _) in enumerate(spec)]
    shards = [dict(to_gpu(l), codebook=cb) for l, (_, _, cb) in zip(lins, spec)]
    y = native.gemv_grouped(x.to(dev()), shards)
    ys = [native.gemv_grouped(x.to(dev()), shards) for _ in range(2)]
    col = 0
    for l, (_, _, cb) in zip(lins, spec):
        check_linear_out(y[:, col:col + l["oc"]], x, l, cb, oracle)
        col += l["oc"]
    for yy in ys:
        assert torch.equal(yy, y)


# ---------------------------------------------------------------- GEMM

@pytest.mark.parametrize("rows", [1, 5, 17, 40, 64, 80, 100, 144, 300])
def test_gemm_rows(native, oracle, rows):
    lin = syn.linear(512, 640, 4, seed=rows)
    x = syn.activations(rows, 512, torch.Generator().manual_seed(rows))
    d = to_gpu(lin)
    y = native.gemm(x.to(dev()), d["trellis"], d["suh"], d["svh"], 4, 0)
    check_linear_out(y, x, lin, 0, oracle)


@pytest.mark.parametrize("rows", [24, 60, 90])
def test_gemm_single_K_partial_pieces(native, oracle, rows):
    """Single-shard exl3_gemm on 32-, 64- and 96-row tiles with ic=2048, oc=1024: 4 output
    tiles of 32 K-steps over 16 workgroups of 8 K-steps, so every tile is split over four
    workgroups (partial sums through slots, counted arrivals, the last arriver adding the
    slots in workgroup order).  Repeat calls must be identical."""
    lin = syn.linear(2048, 1024, 4, seed=rows + 7)
    x = syn.activations(rows, 2048, torch.Generator().manual_seed(rows + 7))
    d = to_gpu(lin)
    y = native.gemm(x.to(dev()), d["trellis"], d["suh"], d["svh"], 4, 0)
    check_linear_out(y, x, lin, 0, oracle)
    for _ in range(2):
        assert torch.equal(native.gemm(x.to(dev()), d["trellis"], d["suh"], d["svh"], 4, 0), y)


@pytest.mark.parametrize("K,cb", [(2, 0), (3, 1), (5, 0), (6, 0)])
def test_gemm_K(native, oracle, K, cb):
    lin = syn.linear(384, 256, K, seed=K)
    x = syn.activations(40, 384, torch.Generator().manual_seed(K))
    d = to_gpu(lin)
    y = native.gemm(x.to(dev()), d["trellis"], d["suh"], d["svh"], K, cb)
    check_linear_out(y, x, lin, cb, oracle)


@pytest.mark.parametrize("rows,ic,oc,K,cb", [(257, 128, 128, 3, 0), (300, 640, 640, 4, 1), (520, 1024, 384, 2, 0),
                                          (700, 256, 1152, 5, 0), (450, 384, 256, 8, 0)])
def test_gemm_streamk_shapes(native, oracle, rows, ic, oc, K, cb):
    """128-row tiles (up to 384 rows) and 256-row tiles (above) split over workgroups by
    K-steps: ragged rows, output counts that leave half a tile, tiny ic, both codebooks"""
    lin = syn.linear(ic, oc, K, seed=rows + oc)
    x = syn.activations(rows, ic, torch.Generator().manual_seed(rows))
    d = to_gpu(lin)
    y = native.gemm(x.to(dev()), d["trellis"], d["suh"], d["svh"], K, cb)
    check_linear_out(y, x, lin, cb, oracle)


@pytest.mark.parametrize("rows", [1, 5, 17, 40, 64, 80, 100, 200, 450])
def test_gemm_grouped_mixed_K_and_codebooks(native, oracle, rows):
    """exl3_gemm_grouped: shards of several K (interleaved) and both codebooks that read one
    A; tiles of up to 128 rows (32, 48, 64, 96 or 128 by row count) take each codebook's
    shards in one launch (per-piece K), 256-row tiles one launch per K.  Deterministic
    across calls."""
    spec = [(384, 3, 0), (256, 5, 0), (128, 3, 1), (640, 2, 0), (256, 3, 0), (128, 6, 1), (384, 5, 0)]
    x = syn.activations(rows, 768, torch.Generator().manual_seed(50 + rows))
    lins = [syn.linear(768, oc, K, seed=500 + i) for i, (oc, K, _) in enumerate(spec)]
    shards = [dict(to_gpu(l), codebook=cb) for l, (_, _, cb) in zip(lins, spec)]
    y = native.gemm_grouped(x.to(dev()), shards)
    col = 0
    for l, (_, _, cb) in zip(lins, spec):
        check_linear_out(y[:, col:col + l["oc"]], x, l, cb, oracle)
        col += l["oc"]
    assert torch.equal(native.gemm_grouped(x.to(dev()), shards), y)


def test_gemm_grouped_more_shards_than_one_launch(native, oracle):
    """10 shards of one codebook: two launches (8 shards per launch), each with its own
    set-up kernel and workspace share"""
    x = syn.activations(33, 256, torch.Generator().manual_seed(70))
    lins = [syn.linear(256, 128 * (1 + i % 3), 2 + i % 4, seed=700 + i) for i in range(10)]
    shards = [dict(to_gpu(l), codebook=0) for l in lins]
    y = native.gemm_grouped(x.to(dev()), shards)
    col = 0
    for l in lins:
        check_linear_out(y[:, col:col + l["oc"]], x, l, 0, oracle)
        col += l["oc"]


@pytest.mark.parametrize("rows", [40, 144])
def test_gemm_grouped_config2(native, oracle, rows):
    """qkv (q K4 5120->6144, k/v K5 5120->1024) and gate_up (2 x K3 5120->17408) prefill
    through one grouped launch each; oracle on every row"""
    x = syn.activations(rows, 5120, torch.Generator().manual_seed(60 + rows))
    for spec in ([(6144, 4), (1024, 5), (1024, 5)], [(17408, 3), (17408, 3)]):
        lins = [syn.linear(5120, oc, K, seed=600 + i) for i, (oc, K) in enumerate(spec)]
        shards = [dict(to_gpu(l), codebook=0) for l in lins]
        y = native.gemm_grouped(x.to(dev()), shards)
        col = 0
        for l in lins:
            check_linear_out(y[:, col:col + l["oc"]], x, l, 0, oracle)
            col += l["oc"]


def test_gemm_streamk_deterministic(native):
    lin = to_gpu(syn.linear(2048, 512, 4, seed=5))
    x = syn.activations(600, 2048, torch.Generator().manual_seed(4)).to(dev())
    ys = [native.gemm(x, lin["trellis"], lin["suh"], lin["svh"], 4, 0) for _ in range(3)]
    for y in ys[1:]:
        assert torch.equal(y, ys[0])


def test_gemm_config3_sampled_rows(native, oracle):
    """M=2048 through down_proj (17408->5120, K=4); oracle on a sample of rows."""
    lin = syn.linear(17408, 5120, 4, seed=3)
    x = syn.activations(2048, 17408, torch.Generator().manual_seed(33))
    d = to_gpu(lin)
    y = native.gemm(x.to(dev()), d["trellis"], d["suh"], d["svh"], 4, 0)
    W = oracle.reconstruct_f16(lin["trellis"], 4, 0)
    idx = torch.tensor([0, 1, 63, 64, 511, 1000, 1777, 2047])
    check_linear_out(y[idx.to(dev())], x[idx], lin, 0, oracle, W=W)


# ---------------------------------------------------------------- embedding

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_embed_int8_gather_bit_exact(native, dtype):
    g = torch.Generator().manual_seed(8)
    q = torch.randint(-128, 128, (1000, 512), generator=g, dtype=torch.int8)
    s = (torch.rand(1000, 1, generator=g) * 0.02).to(dtype)
    ids = torch.tensor([[0, 999, 5], [5, 17, 0]])
    out = native.embed_int8(q.to(dev()), s.to(dev()), ids.to(dev()))
    want = q[ids].to(dtype) * s[ids]
    assert out.shape == want.shape and out.dtype == dtype
    assert torch.equal(out.cpu(), want)


def test_embed_int8_long_rows_many_ids_and_bad_ids(native):
    # dim 8196: 2049 words, so each lane of the 256-lane workgroup takes two load batches
    g = torch.Generator().manual_seed(10)
    q = torch.randint(-128, 128, (300, 8196), generator=g, dtype=torch.int8)
    s = (torch.rand(300, 1, generator=g) * 0.02).half()
    ids = torch.randint(0, 300, (3000,), generator=g)
    ids[[0, 1234, 2999]] = torch.tensor([-1, 300, 1 << 40])
    out = native.embed_int8(q.to(dev()), s.to(dev()), ids.to(dev())).cpu()
    ok = (ids >= 0) & (ids < 300)
    assert torch.equal(out[ok], q[ids[ok]].half() * s[ids[ok]])
    assert torch.equal(out[~ok], torch.zeros(int((~ok).sum()), 8196, dtype=torch.half))


def test_embed_int8_config4_shape(native):
    g = torch.Generator().manual_seed(9)
    q = torch.randint(-128, 128, (syn.VOCAB, 5120), generator=g, dtype=torch.int8)
    s = (torch.rand(syn.VOCAB, 1, generator=g) * 0.02).half()
    ids = torch.tensor([0, 151935, 77777])
    out = native.embed_int8(q.to(dev()), s.to(dev()), ids.to(dev()))
    assert torch.equal(out.cpu(), q[ids].half() * s[ids])
