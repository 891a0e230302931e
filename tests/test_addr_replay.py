"""CPU address replay of the GEMV and stream-K GEMM kernels (libexl3replay.so, built from
orcasaq2-kernel_amd/csrc/replay with the same __host__ __device__ plan and index functions
the kernels call).

Each case plans a call with the product's planning code over fake device buffers and walks
every workgroup, wave and lane of each launch in the kernels' loop order, checking every
global and LDS index against the buffer it addresses and the coverage invariants: each unit /
K-step decoded once, each output element written once, each slot read holding the partial the
reader expects, each activation-table read of the block its unit needs.  No GPU is used.

Shapes: every BASELINE configuration (config 0: 5120->5120 K=4; config 1: down_proj
17408->5120 at K=2..5; config 2: grouped qkv and gate_up at 1..16 rows; config 3: M=2048 on
down_proj; config 4: o_proj 6144->5120, qkv with three distinct K, the K=6 lm_head
151936x5120), both codebooks, K=1..8, several CU counts, and a seeded sweep of random shapes,
for the 1..4-row kernel (gemv1), the 5..16-row kernel (gemv16) and the stream-K GEMM.
"""
import ctypes
import os
import random

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "orcasaq2-kernel_amd", "orcasaq2", "libexl3replay.so")

CUS = (256, 304, 80, 8, 1)   # MI355X, MI300X, smaller parts, a one-CU device


@pytest.fixture(scope="module")
def rl():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is missing: run __graft_entry__.build() first")
    lib = ctypes.CDLL(LIB)
    lib.exl3r_message.restype = ctypes.c_char_p
    return lib


def _arr(v):
    return (ctypes.c_int * len(v))(*v)


def gemv1(rl, rows, ic, ocs, Ks, cbs=None, cus=256):
    cbs = cbs or [0] * len(ocs)
    st = (ctypes.c_longlong * 4)()
    rc = rl.exl3r_gemv1(rows, ic, len(ocs), _arr(ocs), _arr(Ks), _arr(cbs), cus, st)
    return rc, rl.exl3r_message().decode(), list(st)


def gemm_sk(rl, mode, rows, ic, ocs, Ks, cbs=None, cus=256):
    cbs = cbs or [0] * len(ocs)
    st = (ctypes.c_longlong * 4)()
    rc = rl.exl3r_gemm_sk(mode, rows, ic, len(ocs), _arr(ocs), _arr(Ks), _arr(cbs), cus, st)
    return rc, rl.exl3r_message().decode(), list(st)


def ok(res, what):
    rc, msg, st = res
    assert rc == 0, f"{what}: {msg}"
    assert st[0] >= 1 and st[1] > 0, f"{what}: nothing replayed {st}"
    return st


QKV = ([6144, 1024, 1024], [4, 5, 5])
GATE_UP = ([17408, 17408], [3, 3])


# ---------------------------------------------------------------- 1..4-row GEMV (gemv1)

@pytest.mark.parametrize("cus", CUS)
@pytest.mark.parametrize("K", [2, 3, 4, 5])
def test_gemv1_config1_down_proj(rl, K, cus):
    st = ok(gemv1(rl, 1, 17408, [5120], [K], cus=cus), f"down_proj K={K} cus={cus}")
    assert st[2] == 5120 // 128 * 17408 // 16   # every unit decoded once


@pytest.mark.parametrize("cb", [0, 1])
def test_gemv1_config0(rl, cb):
    ok(gemv1(rl, 1, 5120, [5120], [4], [cb]), f"config 0 cb={cb}")


@pytest.mark.parametrize("rows", [1, 2, 3, 4])
@pytest.mark.parametrize("cus", [256, 304, 8])
def test_gemv1_config2_grouped(rl, rows, cus):
    ok(gemv1(rl, rows, 5120, *QKV, cus=cus), f"qkv rows={rows}")
    ok(gemv1(rl, rows, 5120, *GATE_UP, cus=cus), f"gate_up rows={rows}")


@pytest.mark.parametrize("rows", [1, 4])
def test_gemv1_config4_layers(rl, rows):
    ok(gemv1(rl, rows, 6144, [5120], [4]), "o_proj")
    ok(gemv1(rl, rows, 5120, [6144, 1024, 1024], [2, 3, 5]), "qkv, three K in one launch")
    ok(gemv1(rl, rows, 5120, [17408, 17408], [2, 5]), "gate_up, two K")
    ok(gemv1(rl, rows, 17408, [5120], [3]), "down_proj")


@pytest.mark.parametrize("rows", [1, 2, 4])
def test_gemv1_lm_head(rl, rows):
    """At 2..4 rows the launch's LDS leaves two workgroups per CU, so the kernel keeps two
    units in flight per wave (g1_depth): the replay walks that ring too."""
    st = ok(gemv1(rl, rows, 5120, [151936], [6]), f"K=6 lm_head rows={rows}")
    assert st[2] == 151936 // 128 * 5120 // 16


def test_gemv1_large_shard_uses_more_workgroups_than_resident(rl):
    # a 262144-entry vocabulary at hidden 5120: with only resident workgroups each range
    # would need more LDS than a CU has; the plan takes more (non-resident) workgroups
    ok(gemv1(rl, 1, 5120, [262144], [6]), "262144 x 5120 lm_head")
    ok(gemv1(rl, 1, 17408, [5120], [4], cus=8), "down_proj on 8 CUs")


def test_gemv1_refuses_a_shard_beyond_the_lds_limit(rl):
    rc, msg, _ = gemv1(rl, 1, 16384, [128 * 16000], [4])
    assert rc == 2 and "bytes of LDS per workgroup" in msg


@pytest.mark.parametrize("K", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1])
def test_gemv1_every_K(rl, K, cb):
    ok(gemv1(rl, 1, 768, [384, 128], [K, K], [cb, cb]), f"K={K} cb={cb}")
    ok(gemv1(rl, 3, 2048, [1024], [K], [cb]), f"K={K} cb={cb} 3 rows")


def test_gemv1_many_shards(rl):
    # more shards than one launch holds: several launches, each with its share of the slots
    ocs = [128 * (i % 5 + 1) for i in range(19)]
    Ks = [1 + i % 8 for i in range(19)]
    cbs = [i % 2 for i in range(19)]
    st = ok(gemv1(rl, 2, 1024, ocs, Ks, cbs), "19 shards")
    assert st[0] >= 3


@pytest.mark.parametrize("rows", [1, 3, 4])
def test_gemv1_table_tasks_cross_several_shards(rl, rows):
    # 128 inputs (one block per column group) and nine column groups per shard on one CU: each
    # workgroup's range spans ~18 segments, and a wave's activation-table tasks step over
    # 8 / rows of them at a time, crossing two shard boundaries in one wave's walk
    ok(gemv1(rl, rows, 128, [1152] * 8, [2, 3, 4, 5, 6, 7, 8, 1], [0, 1] * 4, cus=1), f"rows={rows}")
    ok(gemv1(rl, rows, 256, [384, 128, 640, 128, 256, 128, 1152, 128], [4] * 8, cus=1), f"rows={rows} ragged")


def test_gemv1_random_shapes(rl):
    rnd = random.Random(20260)
    for case in range(300):
        ic = 128 * rnd.randint(1, 48)
        n = rnd.randint(1, 9)
        ocs = [128 * rnd.randint(1, 40) for _ in range(n)]
        Ks = [rnd.randint(1, 8) for _ in range(n)]
        cbs = [rnd.randint(0, 1) for _ in range(n)]
        rows = rnd.randint(1, 4)
        cus = rnd.choice(CUS + (2, 3, 33, 120))
        ok(gemv1(rl, rows, ic, ocs, Ks, cbs, cus), f"case {case}: rows={rows} ic={ic} oc={ocs} K={Ks} cus={cus}")


# ---------------------------------------------------------------- 5..16-row GEMV (gemv16)

def gemv16(rl, rows, ic, ocs, Ks, cbs=None, cus=256):
    cbs = cbs or [0] * len(ocs)
    st = (ctypes.c_longlong * 4)()
    rc = rl.exl3r_gemv16(rows, ic, len(ocs), _arr(ocs), _arr(Ks), _arr(cbs), cus, st)
    return rc, rl.exl3r_message().decode(), list(st)


@pytest.mark.parametrize("rows", [5, 9, 16])
@pytest.mark.parametrize("cus", [256, 304, 8, 1])
def test_gemv16_layers(rl, rows, cus):
    ok(gemv16(rl, rows, 5120, *QKV, cus=cus), f"qkv rows={rows}")
    ok(gemv16(rl, rows, 5120, *GATE_UP, cus=cus), f"gate_up rows={rows}")
    ok(gemv16(rl, rows, 17408, [5120], [4], cus=cus), f"down_proj rows={rows}")
    ok(gemv16(rl, rows, 6144, [5120], [4], cus=cus), f"o_proj rows={rows}")
    ok(gemv16(rl, rows, 5120, [6144, 1024, 1024], [2, 3, 5], cus=cus), f"qkv three K rows={rows}")


def test_gemv16_lm_head(rl):
    ok(gemv16(rl, 16, 5120, [151936], [6]), "lm_head 16 rows")


@pytest.mark.parametrize("rows", [2, 3, 4])
def test_gemv_2_to_4_rows_take_gemv16_beyond_gemv1s_lds(rl, rows):
    # exl3_gemv's routing at 2..4 rows: gemv1 wherever its plan fits, the lm_head included
    # (more workgroups than stay resident); gemv16 for the shards gemv1's plan refuses
    ok(gemv1(rl, rows, 5120, [151936], [6]), f"lm_head rows={rows} (gemv1)")
    rc, msg, _ = gemv1(rl, rows, 16384, [163840], [1])
    assert rc == 2 and "bytes of LDS per workgroup" in msg
    ok(gemv16(rl, rows, 16384, [163840], [1]), f"16384 x 163840 rows={rows} (gemv16)")


@pytest.mark.parametrize("cus", [256, 8, 1])
def test_gemv16_odd_K_block_order(rl, cus):
    # one odd-K group of 1472 units: 46 workgroups, which the blocks take XCD by XCD (the
    # replay walks the blocks in that order and checks it is a bijection)
    ok(gemv16(rl, 7, 1024, [2944], [3], cus=cus), f"1024 x 2944 K=3 on {cus} CUs")
    ok(gemv16(rl, 13, 1024, [1408, 1536], [7, 7], cus=cus), f"two K=7 shards on {cus} CUs")


@pytest.mark.parametrize("K", range(1, 9))
def test_gemv16_every_K(rl, K):
    ok(gemv16(rl, 7, 768, [384, 128], [K, K], [0, 1]), f"K={K}")


def test_gemv16_random_shapes(rl):
    rnd = random.Random(1616)
    for case in range(200):
        ic = 128 * rnd.randint(1, 48)
        n = rnd.randint(1, 9)
        ocs = [128 * rnd.randint(1, 40) for _ in range(n)]
        Ks = [rnd.randint(1, 8) for _ in range(n)]
        cbs = [rnd.randint(0, 1) for _ in range(n)]
        rows = rnd.randint(1, 16)
        cus = rnd.choice(CUS + (2, 3, 33, 120))
        ok(gemv16(rl, rows, ic, ocs, Ks, cbs, cus), f"case {case}: rows={rows} ic={ic} oc={ocs} K={Ks} cus={cus}")


# ---------------------------------------------------------------- stream-K GEMM

@pytest.mark.parametrize("rows", [17, 32, 40, 48, 64, 80, 96, 144, 300, 385, 2048])
def test_gemm_down_proj(rl, rows):
    st = ok(gemm_sk(rl, 0, rows, 17408, [5120], [4]), f"exl3_gemm down_proj rows={rows}")
    assert st[2] > 0


@pytest.mark.parametrize("cus", CUS)
def test_gemm_config3(rl, cus):
    ok(gemm_sk(rl, 0, 2048, 17408, [5120], [4], cus=cus), f"config 3 cus={cus}")


@pytest.mark.parametrize("rows", [17, 64, 144, 400])
def test_gemm_grouped_layers(rl, rows):
    ok(gemm_sk(rl, 1, rows, 5120, *QKV), f"grouped qkv rows={rows}")
    ok(gemm_sk(rl, 1, rows, 5120, *GATE_UP), f"grouped gate_up rows={rows}")
    ok(gemm_sk(rl, 1, rows, 5120, [6144, 1024, 1024], [2, 3, 5]), f"grouped qkv, three K, rows={rows}")


def test_gemm_sk_random_shapes(rl):
    rnd = random.Random(4099)
    for case in range(120):
        ic = 128 * rnd.randint(1, 40)
        mode = rnd.choice([0, 1])
        n = 1 if mode == 0 else rnd.randint(1, 9)
        ocs = [128 * rnd.randint(1, 30) for _ in range(n)]
        Ks = [rnd.randint(1, 8) for _ in range(n)]
        cbs = [rnd.randint(0, 1) for _ in range(n)]
        rows = rnd.randint(1, 600)
        cus = rnd.choice(CUS + (2, 3, 33, 120))
        ok(gemm_sk(rl, mode, rows, ic, ocs, Ks, cbs, cus),
           f"case {case}: mode={mode} rows={rows} ic={ic} oc={ocs} K={Ks} cus={cus}")


def test_replay_reports_a_refused_plan(rl):
    # rows outside 1..4 are refused by the GEMV plan itself, before any launch
    rc, msg, _ = gemv1(rl, 5, 1024, [128], [4])
    assert rc == 2 and "rows=5" in msg
