"""C ABI of libexl3hip.so on the CPU: the library loads, exports every function the public
header declares, and its host-side argument checks reject bad calls before anything is
enqueued (no GPU call is made by any of these)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "exl3hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(exl3_\w+)\s*\(", text, flags=re.M)))


def test_header_lists_the_entry_points():
    fns = header_functions()
    for f in ("exl3_reconstruct", "exl3_reconstruct_t", "exl3_had_r_128", "exl3_gemv", "exl3_gemv_grouped",
              "exl3_gemm", "exl3_gemm_grouped", "exl3_embed_int8_gather", "exl3_last_error"):
        assert f in fns


def test_library_exports_every_declared_symbol(native):
    L = native.lib()
    for f in header_functions():
        assert hasattr(L, f), f
    assert set(native.EXPORTED) == set(header_functions())


def test_abi_version(native):
    assert native.lib().exl3_abi_version() == native.ABI_VERSION


def _err(native):
    return native.lib().exl3_last_error().decode()


P = ctypes.c_void_p


def test_gemv_rejects_bad_arguments_on_host(native):
    L = native.lib()
    fake = P(0x10000)  # never dereferenced: every call below fails its host checks
    ws = P(0x100000)
    # rows out of range
    rc = L.exl3_gemv(fake, fake, fake, fake, fake, ws, 1 << 20, 17, 256, 256, 4, 0, None)
    assert rc == 1 and "rows=17" in _err(native)
    rc = L.exl3_gemv(fake, fake, fake, fake, fake, ws, 1 << 20, 0, 256, 256, 4, 0, None)
    assert rc == 1
    # K out of range
    rc = L.exl3_gemv(fake, fake, fake, fake, fake, ws, 1 << 20, 1, 256, 256, 9, 0, None)
    assert rc == 1 and "K=9" in _err(native)
    # ic not a multiple of 128
    rc = L.exl3_gemv(fake, fake, fake, fake, fake, ws, 1 << 20, 1, 200, 256, 4, 0, None)
    assert rc == 1 and "multiples of 128" in _err(native)
    # mul1 codebook
    rc = L.exl3_gemv(fake, fake, fake, fake, fake, ws, 1 << 20, 1, 256, 256, 4, 2, None)
    assert rc == 2 and "mul1" in _err(native)
    # workspace too small
    rc = L.exl3_gemv(fake, fake, fake, fake, fake, ws, 16, 1, 256, 256, 4, 0, None)
    assert rc == 3 and "workspace" in _err(native)
    # misaligned pointer
    rc = L.exl3_gemv(P(0x10001), fake, fake, fake, fake, ws, 1 << 20, 1, 256, 256, 4, 0, None)
    assert rc == 1 and "aligned" in _err(native)


def test_other_entry_points_reject_bad_arguments(native):
    L = native.lib()
    fake = P(0x10000)
    assert L.exl3_reconstruct(fake, fake, 100, 256, 4, 0, None) == 1
    assert L.exl3_reconstruct(fake, fake, 256, 256, 0, 0, None) == 1
    assert L.exl3_reconstruct(P(0x10008), fake, 256, 256, 4, 0, None) == 1  # W not 16-aligned
    assert L.exl3_reconstruct_t(fake, fake, 256, 100, 4, 0, None) == 1
    assert "exl3_reconstruct_t" in _err(native) and "multiples of 16" in _err(native)
    assert L.exl3_reconstruct_t(fake, fake, 256, 256, 9, 0, None) == 1
    assert "K=9" in _err(native)
    assert L.exl3_reconstruct_t(P(0x10008), fake, 256, 256, 4, 0, None) == 1
    assert L.exl3_reconstruct_t(fake, fake, 256, 256, 4, 7, None) != 0      # unknown codebook
    assert L.exl3_had_r_128(fake, fake, None, None, 1.0, 4, 100, None) == 1
    assert L.exl3_gemm(fake, fake, fake, fake, fake, P(0x100000), 1 << 30, 0, 256, 256, 4, 0, None) == 1
    assert L.exl3_gemm(fake, fake, fake, fake, fake, P(0x100000), 8, 32, 256, 256, 4, 0, None) == 3
    assert L.exl3_embed_int8_gather(fake, fake, 0, fake, fake, 4, 100, 10, None) == 1  # dim % 4
    assert L.exl3_embed_int8_gather(fake, fake, 5, fake, fake, 4, 100, 16, None) == 1  # dtype
    assert L.exl3_embed_int8_gather(None, None, 0, None, None, 0, 0, 16, None) == 0    # empty: no-op
    # one 256-lane workgroup per id: more than (2^32 - 1) / 256 ids would exceed a launch
    assert L.exl3_embed_int8_gather(fake, fake, 0, fake, fake, 1 << 24, 100, 16, None) == 1
    assert "at most 16777215" in _err(native)
    sh = (native.Shard * 2)()
    sh[0] = native.Shard(0x10000, 0x10000, 0x10000, 0x10000, 512, 256, 4, 0)
    sh[1] = native.Shard(0x10000, 0x10000, 0x10000, 0x10100, 512, 256, 5, 0)
    assert L.exl3_gemm_grouped(fake, sh, 0, P(0x100000), 1 << 30, 32, 256, None) == 1      # no shards
    assert L.exl3_gemm_grouped(fake, sh, 2, P(0x100000), 1 << 30, 0, 256, None) == 1       # rows
    assert L.exl3_gemm_grouped(fake, sh, 2, P(0x100000), 8, 32, 256, None) == 3            # workspace
    assert "exl3_gemm_grouped" in _err(native) and "needed" in _err(native)
    sh[1] = native.Shard(0x10000, 0x10000, 0x10000, 0x10100, 100, 256, 5, 0)
    assert L.exl3_gemm_grouped(fake, sh, 2, P(0x100000), 1 << 30, 32, 256, None) == 1     # ldc < oc
    assert "shard 1" in _err(native)
    assert L.exl3_gemm_grouped_workspace_bytes(sh, 2, 32, 256) > 0
    assert L.exl3_gemm_grouped_workspace_bytes(sh, 2, 0, 256) == 0


def test_workspace_sizes(native):
    L = native.lib()
    b1 = L.exl3_gemv_workspace_bytes(1, 17408, 5120)
    b16 = L.exl3_gemv_workspace_bytes(16, 17408, 5120)
    assert b1 > 0 and b16 > b1 and b1 % 256 == 0
    arr = (native.Shard * 2)()
    arr[0].oc, arr[1].oc = 6144, 1024
    g = L.exl3_gemv_grouped_workspace_bytes(arr, 2, 4, 5120)
    # the reserved 16 KiB head and the 6 MiB accumulator area lead every GEMV workspace once;
    # shards add their shares
    head = 16384 + (6 << 20)
    assert g == (L.exl3_gemv_workspace_bytes(4, 5120, 6144) + L.exl3_gemv_workspace_bytes(4, 5120, 1024)
                 - head)
    arr[0].oc = 100
    assert L.exl3_gemv_grouped_workspace_bytes(arr, 2, 4, 5120) == 0
    assert L.exl3_gemm_workspace_bytes(2048, 17408, 5120) >= 2048 * 17408 * 2


@pytest.mark.parametrize("ic,oc", [(5120, 6144), (5120, 1024), (17408, 5120), (5120, 151936), (16384, 163840),
                                   (128, 128)])
def test_gemv_workspace_at_2_to_4_rows_covers_the_gemv16_fallback(native, ic, oc):
    """A 2..4-row call runs gemv1 where its plan takes the shards and gemv16 where it does not
    (the choice is made per call, after the caller sized the workspace), so the 2..4-row size
    holds gemv16's: the 5..16-row size, which does not depend on the row count."""
    L = native.lib()
    b16 = L.exl3_gemv_workspace_bytes(16, ic, oc)
    assert L.exl3_gemv_workspace_bytes(5, ic, oc) == b16
    for rows in (2, 3, 4):
        b = L.exl3_gemv_workspace_bytes(rows, ic, oc)
        assert b >= b16 and b >= L.exl3_gemv_workspace_bytes(1, ic, oc) and b % 256 == 0


def test_wrappers_refuse_cpu_tensors(native):
    import torch
    x = torch.zeros(1, 128, dtype=torch.float16)
    t = torch.zeros(8, 8, 64, dtype=torch.int16)
    with pytest.raises(RuntimeError, match="GPU"):
        native.gemv(x, t, torch.ones(128, dtype=torch.float16), torch.ones(128, dtype=torch.float16), 4, 0)
    with pytest.raises(RuntimeError, match="GPU"):
        native.reconstruct(t, 4, 0)


def test_topk_rejects_bad_arguments_on_host(native):
    L = native.lib()
    fake, ws = P(0x10000), P(0x100000)
    big = 1 << 30

    def call(rows=2, n=4096, ld=4096, k=8, x=fake, wsb=big, values=fake, indices=fake):
        return L.exl3_topk(x, rows, n, ld, k, values, indices, ws, wsb, None)

    assert call(k=0) == 1 and "k=0" in _err(native)
    assert call(k=65) == 1 and "k=65" in _err(native)
    assert call(n=7, ld=8) == 1                                  # k > n
    assert call(n=(1 << 19) + 8, ld=(1 << 19) + 8) == 1           # n beyond the bound
    assert call(ld=4100) == 1 and "ld=4100" in _err(native)      # ld % 8
    assert call(ld=4088) == 1                                    # ld < n
    assert call(rows=-1) == 1 and call(rows=70000) == 1
    assert call(x=P(0x10008)) == 1 and "misaligned" in _err(native)
    assert call(indices=P(0x10004)) == 1
    assert call(wsb=8) == 3 and "workspace" in _err(native)
    assert L.exl3_topk_workspace_bytes(2, 4096, 8) == 2 * 1 * 8 * 8
    assert L.exl3_topk_workspace_bytes(1, 151936, 64) == 38 * 64 * 8     # 4096-column chunks
    assert call(rows=0) == 0                                     # nothing to do, nothing enqueued
