"""Pins for the CPU oracle (oracle/exl3_oracle.c + oracle/oracle.py).

Each check is chosen so that a plausible slip -- a wrong constant, a dropped mask, a
reversed bit order, an off-by-one window, a transposed placement, a missing Hadamard
normalisation -- fails at least one of them:

* codebook statistics of the published 3INST constants (QTIP, arXiv 2406.11235), computed
  independently when the reference was surveyed: mean 0.00021, std 1.24371, range
  [-3.9570, 3.9727], 10,598 distinct values, smallest |v| = 2^-13 (MCG: std 1.24411,
  range +-3.9492, 10,746 distinct);
* a hand-worked known answer for state 0;
* the tail-biting shift-register property of the states, and a trellis *encoder* (symbols
  -> packed words) written from the stream definition, whose walk the decoder must follow;
* the placement against the MMA-fragment table worked by hand;
* the Hadamard against the dense Sylvester matrix, H.H = I, +-2^-3.5 entries;
* the two reference statements of the dequant algebra (orcasaq2/__init__.py:49-61 vs
  orcasaq2/ops.py:53-59) agreeing in fp64.
"""
import numpy as np
import pytest
import torch


def test_codebook_3inst_statistics(oracle):
    t = oracle.codebook_table(oracle.CB_3INST).view(np.float16).astype(np.float64)
    assert round(t.mean(), 5) == 0.00021
    assert round(t.std(), 5) == 1.24371
    assert round(t.min(), 4) == -3.9570 and round(t.max(), 4) == 3.9727
    assert len(np.unique(t)) == 10598
    assert np.abs(t[t != 0]).min() == 2.0 ** -13
    assert np.isfinite(t).all()


def test_codebook_mcg_statistics(oracle):
    t = oracle.codebook_table(oracle.CB_MCG).view(np.float16).astype(np.float64)
    assert round(t.std(), 5) == 1.24411
    assert round(t.min(), 4) == -3.9492 and round(t.max(), 4) == 3.9492
    assert len(np.unique(t)) == 10746


def test_codebook_known_answer_state0(oracle):
    # 3INST, s = 0: x = 64248484 = 0x03D45AA4; & 0x8FFF8FFF -> 0x03D40AA4;
    # ^ 0x3B603B60 -> hi 0x38B4 (0.587890625), lo 0x31C4 (0.18017578125).
    assert np.uint16(0x38B4).view(np.float16) == np.float16(0.587890625)
    assert np.uint16(0x31C4).view(np.float16) == np.float16(0.18017578125)
    v = np.uint16(oracle.codebook_value(0, oracle.CB_3INST)).view(np.float16)
    assert v == np.float16(0.587890625 + 0.18017578125)
    # MCG, s = 0: x = 0 -> 0x3B603B60 -> 2 * fp16(0x3B60) = 2 * 0.921875
    v = np.uint16(oracle.codebook_value(0, oracle.CB_MCG)).view(np.float16)
    assert np.uint16(0x3B60).view(np.float16) == np.float16(0.921875)
    assert v == np.float16(2 * 0.921875)


def test_codebook_half_sum_is_one_rounding(oracle):
    """fp16(lo) + fp16(hi) rounded once (IEEE fp16 add) for every state."""
    a, b, c = np.uint32(89226354), np.uint32(64248484), np.uint32(0xCBAC1FED)
    s = np.arange(65536, dtype=np.uint32)
    for cb, x in ((oracle.CB_3INST, s * a + b), (oracle.CB_MCG, s * c)):
        x = (x & np.uint32(0x8FFF8FFF)) ^ np.uint32(0x3B603B60)
        lo = (x & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
        hi = (x >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
        assert (np.abs(lo) >= 0.125).all() and (np.abs(hi) < 2).all()
        want = (lo + hi).astype(np.float16)   # exact sum (|v| < 4, multiple of 2^-13), one RNE
        got = oracle.codebook_table(cb).view(np.float16)
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_double_to_half_matches_numpy(oracle):
    rng = np.random.default_rng(0)
    d = rng.standard_normal(4000) * 10.0 ** rng.integers(-9, 5, 4000)
    d = np.concatenate([d, [0.0, -0.0, 65504.0, 65519.99, 65520.0, 2.0 ** -24, 2.0 ** -25,
                            3 * 2.0 ** -26, 2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]])
    with np.errstate(over="ignore"):
        want = d.astype(np.float16).view(np.uint16)
    got = np.array([oracle.double_to_half(v) for v in d], np.uint16)
    assert np.array_equal(got, want)


def _encode(symbols: np.ndarray, K: int) -> np.ndarray:
    """Trellis encoder written from the stream definition: symbol t occupies stream bits
    [tK, (t+1)K) MSB-first; the stream fills u32 words MSB-first; each u32 is stored as
    two little-endian int16 words."""
    bits = []
    for sym in symbols:
        bits.extend((int(sym) >> (K - 1 - b)) & 1 for b in range(K))
    words = []
    for j in range(0, len(bits), 32):
        u = 0
        for b in bits[j:j + 32]:
            u = (u << 1) | b
        words += [u & 0xFFFF, u >> 16]
    return np.array(words, np.uint16)


@pytest.mark.parametrize("K", range(1, 9))
def test_states_follow_the_trellis_walk(oracle, K):
    rng = np.random.default_rng(K)
    sym = rng.integers(0, 1 << K, 256)
    tile = _encode(sym, K)
    st = oracle.states(tile, K)
    L = -(-16 // K)  # symbols spanned by a 16-bit state
    for t in range(256):
        want = 0
        for d in range(L - 1, -1, -1):  # oldest first, tail-biting wrap
            want = (want << K) | int(sym[(t - d) % 256])
        assert st[t] == want & 0xFFFF, (K, t)


@pytest.mark.parametrize("K", range(1, 9))
def test_states_shift_register_property(oracle, K):
    rng = np.random.default_rng(100 + K)
    tile = rng.integers(0, 65536, 16 * K).astype(np.uint16)
    st = oracle.states(tile, K)
    mask = (1 << (16 - K)) - 1
    for t in range(256):
        assert (st[(t + 1) % 256] >> K) == (st[t] & mask)


def test_state_bit_order_known_answer(oracle):
    # K = 2, only stream bit 0 set (MSB of u32 word 0 = bit 15 of int16 word 1).
    tile = np.zeros(32, np.uint16)
    tile[1] = 0x8000
    st = oracle.states(tile, 2)
    # stream bit 0 is the first symbol's high bit: state t covers bits [2t-14, 2t+2)
    assert st[0] == 0b10
    assert [int(st[t]) for t in range(1, 8)] == [0b10 << (2 * t) for t in range(1, 8)]
    assert st[8] == 0 and (st[9:] == 0).all()


def test_placement_table(oracle):
    p = oracle.perm()
    assert sorted(p.tolist()) == list(range(256))
    rc = {t: divmod(int(p[t]), 16) for t in range(256)}
    # lane j = t // 8 of the 16x16 fragment: rows 2(j%4) + {0,1,8,9}, cols j//4 (+8)
    assert rc[0] == (0, 0) and rc[1] == (1, 0) and rc[2] == (8, 0) and rc[3] == (9, 0)
    assert rc[4] == (0, 8) and rc[5] == (1, 8) and rc[6] == (8, 8) and rc[7] == (9, 8)
    assert rc[8] == (2, 0) and rc[24] == (6, 0) and rc[32] == (0, 1)
    assert rc[255] == (15, 15) and rc[250] == (14, 7) and rc[253] == (7, 15)


@pytest.mark.parametrize("K,cb", [(2, 0), (4, 0), (5, 1), (8, 0)])
def test_reconstruct_places_tiles(oracle, K, cb):
    rng = np.random.default_rng(K)
    tr = rng.integers(0, 65536, (3, 5, 16 * K)).astype(np.uint16)
    W = oracle.reconstruct(tr, K, cb)
    assert W.shape == (48, 80)
    p = oracle.perm()
    tbl = oracle.codebook_table(cb)
    for ti in range(3):
        for tn in range(5):
            st = oracle.states(tr[ti, tn], K)
            blk = np.empty(256, np.uint16)
            blk[p] = tbl[st]
            assert np.array_equal(W[16 * ti:16 * ti + 16, 16 * tn:16 * tn + 16], blk.reshape(16, 16))


def test_hadamard_closed_forms(oracle):
    H = oracle.had_matrix(128)
    n = np.arange(128)
    sylv = (-1.0) ** np.array([[bin(i & j).count("1") for j in n] for i in n]) / np.sqrt(128)
    assert np.array_equal(H, sylv)
    assert np.allclose(H @ H, np.eye(128), atol=1e-15)
    assert np.allclose(np.abs(H), 2 ** -3.5)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 384))
    want = (x.reshape(5, 3, 128) @ H).reshape(5, 384)
    assert np.allclose(oracle.had128(x), want, rtol=0, atol=1e-13)
    assert np.allclose(oracle.had128(oracle.had128(x)), x, atol=1e-13)


def test_package_t128_matches_oracle(oracle):
    from orcasaq2 import _t128
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 256))
    got = _t128(torch.from_numpy(x)).numpy()
    assert np.allclose(got, oracle.had128(x), atol=1e-12)


@pytest.mark.parametrize("ic,oc", [(128, 128), (256, 128), (128, 256)])
def test_dequant_algebra_two_statements_agree(oracle, ic, oc):
    """F.linear(x, reconstruct_weight) == H(H(x*suh) W_q) * svh (fp64, no fp16 A_had)."""
    rng = np.random.default_rng(ic + oc)
    tr = rng.integers(0, 65536, (ic // 16, oc // 16, 64)).astype(np.uint16)
    Wq = oracle.reconstruct_f16(tr, 4)
    suh = rng.choice([-1.0, 1.0], ic)
    svh = rng.choice([-1.0, 1.0], oc) * np.abs(rng.standard_normal(oc)) / np.sqrt(ic)
    x = rng.standard_normal((3, ic))
    deploy = oracle.deploy_weight(Wq, suh, svh)                 # (oc, ic)
    y1 = x @ deploy.T
    y2 = oracle.had_r_128(oracle.had_r_128(x, pre=suh) @ Wq.astype(np.float64), post=svh)
    assert np.allclose(y1, y2, rtol=1e-12, atol=1e-12)
    # and the fused reference model, whose A_had is rounded to fp16, is within fp16 noise
    y3 = oracle.shard_gemm_ref(x.astype(np.float16), tr, suh.astype(np.float16), svh.astype(np.float16), 4)
    y1h = x.astype(np.float16).astype(np.float64) @ oracle.deploy_weight(
        Wq, suh, svh.astype(np.float16).astype(np.float64)).T
    assert oracle.rel_err_rows(y3, y1h).max() < 1e-3


def test_embed_int8_reference_semantics(oracle):
    rng = np.random.default_rng(3)
    q = rng.integers(-128, 128, (50, 8)).astype(np.int8)
    s = (rng.random((50, 1)) * 0.02).astype(np.float16)
    ids = np.array([0, 7, 49, 7])
    want = (torch.from_numpy(q)[torch.from_numpy(ids)].to(torch.float16)
            * torch.from_numpy(s)[torch.from_numpy(ids)]).numpy()
    assert np.array_equal(oracle.embed_int8_ref(q, s, ids).view(np.uint16), want.view(np.uint16))


# ---------------------------------------------------------------- top-k / argmax of the head's logits

def _brute_topk(row, k):
    # total order written out case by case: NaN first (ties by column), then by value
    # (-0 == +0), ties by column
    def rank(i):
        v = float(row[i])
        return (0, 0.0, i) if np.isnan(v) else (1, -v, i)
    order = sorted(range(len(row)), key=rank)[:k]
    return np.array(order, np.int64)


def test_fp16_order_key_is_monotone_over_every_fp16(oracle):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    v = h.view(np.float16)
    key = oracle.fp16_order_key(v)
    finite = ~np.isnan(v)
    f = v[finite].astype(np.float64)
    kf = key[finite]
    o = np.argsort(f, kind="stable")
    assert np.all(np.diff(kf[o]) >= 0)                      # value order kept
    assert np.all((np.diff(f[o]) == 0) == (np.diff(kf[o]) == 0))   # equal keys iff equal values
    assert np.all(key[~finite] == 0xFFFF) and kf.max() == 0xFC00 and kf.min() == 0x03FF
    assert key[np.float16(0.0).view(np.uint16)] == key[np.float16(-0.0).view(np.uint16)] == 0x8000


def test_topk_oracle_matches_torch_argmax_and_topk(oracle):
    rng = np.random.default_rng(5)
    # heavy ties: values drawn from a small set, plus +-0, +-inf and NaN in some rows
    x = rng.choice(np.array([-3, -1, -0.0, 0.0, 0.5, 2, 7], np.float16), size=(40, 300))
    x[3, 17] = np.inf
    x[5, [9, 200]] = np.nan
    x[6, :] = -np.inf
    x[7, 150] = -np.inf
    xt = torch.from_numpy(x)
    v1, i1 = oracle.topk_rows(x, 1)
    assert np.array_equal(i1[:, 0], torch.argmax(xt, dim=1).numpy())
    assert np.array_equal(i1[:, 0], torch.argmax(xt.float(), dim=1).numpy())
    # distinct values: torch.topk's order is the oracle's
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    finite = bits[~np.isnan(bits.view(np.float16)) & (bits != 0x8000)]          # distinct values
    y = rng.choice(finite, size=4000, replace=False).view(np.float16).reshape(4, 1000)
    for k in (1, 5, 64):
        vk, ik = oracle.topk_rows(y, k)
        tv, ti = torch.topk(torch.from_numpy(y).float(), k, dim=1, sorted=True)
        assert np.array_equal(vk.astype(np.float32), tv.numpy()) and np.array_equal(ik, ti.numpy())


def test_topk_oracle_matches_brute_force_on_ties_and_special_values(oracle):
    rng = np.random.default_rng(9)
    pool = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -1.0, 65504, -65504, 6e-8, -6e-8], np.float16)
    for case in range(200):
        n = int(rng.integers(1, 40))
        row = rng.choice(pool, size=n)
        k = int(rng.integers(1, n + 1))
        v, i = oracle.topk_rows(row[None, :], k)
        want = _brute_topk(row, k)
        assert np.array_equal(i[0], want), (case, row, k)
        assert np.array_equal(v[0].view(np.uint16), row[want].view(np.uint16))   # the entries' own bits
