"""CPU-only checks of the dense hub block's C ABI: the workspace sizes follow
the stated layout, and every launcher rejects bad arguments with
PS_ERR_INVALID and a message before it makes any device call (the pointers
below are never dereferenced)."""
import ctypes

import pytest

from powersparse_amd import _native

FAKE = 0x10000  # a non-null, 16-byte aligned stand-in address


def r256(b):
    return (b + 255) & ~255


def block(rows=8, cols=64, **kw):
    hb = _native.HubBlock(matrix_rows=100, matrix_cols=200, rows=rows, cols=cols,
                          hub_rows=FAKE, hub_index=FAKE, hot_cols=FAKE, hot_rank=FAKE,
                          dense=FAKE, stored=FAKE)
    for k, v in kw.items():
        setattr(hb, k, v)
    return hb


def last_error():
    return _native.hip().ps_last_error().decode()


def test_dense_ld_rounds_to_64():
    lib = _native.hip()
    assert [lib.ps_hub_dense_ld(c) for c in (0, -3, 1, 63, 64, 65, 70, 200)] == \
        [0, 0, 64, 64, 64, 128, 128, 256]
    # rows padded to 64 as well
    assert [lib.ps_hub_dense_floats(r, c) for r, c in ((0, 5), (5, 0), (1, 1), (64, 64),
                                                       (65, 70), (130, 200))] == \
        [0, 0, 64 * 64, 64 * 64, 128 * 128, 192 * 256]


def test_workspace_and_stored_words():
    lib = _native.hip()
    hb = block(rows=5, cols=70)
    assert lib.ps_hub_stored_words(ctypes.byref(hb)) == 5 * 3
    assert lib.ps_hub_stored_words(None) == 0
    ld = 128  # 70 hot columns padded to a multiple of 64
    for N, slice_ in ((32, 32), (128, 128), (256, 128)):
        spmm = r256(slice_ * ld * 4) + r256(70 * 4) + 256
        assert lib.ps_hub_workspace_bytes(ctypes.byref(hb), _native.PS_OP_SPMM, N) == spmm
    # SDDMM: X[hub_rows] padded to 64 rows and Y[hot_cols] to 128, N floats each
    for N in (32, 128, 512):
        sddmm = r256(64 * N * 4) + r256(128 * N * 4)
        assert lib.ps_hub_workspace_bytes(ctypes.byref(hb), _native.PS_OP_SDDMM, N) == sddmm
    assert lib.ps_hub_workspace_bytes(ctypes.byref(hb), _native.PS_OP_SPMM, 0) == 0
    assert lib.ps_hub_workspace_bytes(ctypes.byref(hb), 7, 32) == 0


def test_plan_bytes_follow_the_tile_grid():
    lib = _native.hip()
    # 130 hub rows -> 3 row panels of 64; 600 hot columns -> 5 column tiles of 128
    hb = block(rows=130, cols=600)
    for tiles in (0, 1, 7):
        n = 64 * tiles
        want = r256((3 * 5 + 1) * 4) + r256(n * 8) + r256(n * 4)
        assert lib.ps_hub_sddmm_plan_bytes(ctypes.byref(hb), tiles) == want
    assert lib.ps_hub_sddmm_plan_bytes(None, 4) == 0


@pytest.mark.parametrize("change,N,ws,msg", [
    (dict(rows=0), 32, 1 << 40, "empty block"),
    (dict(hot_rank=None), 32, 1 << 40, "missing arrays"),
    (dict(dense=None), 32, 1 << 40, "missing dense block"),
    ({}, 48, 1 << 40, "multiple of 32"),
    ({}, 32, 1024, "workspace too small"),
])
def test_spmm_launch_rejects(change, N, ws, msg):
    lib = _native.hip()
    hb = block(**change)
    rc = lib.ps_hub_spmm_launch(ctypes.byref(hb), N, FAKE, FAKE, FAKE, ws, None)
    assert rc == _native.PS_ERR_INVALID and msg in last_error()


def test_spmm_launch_rejects_null_descriptor_and_misaligned_operands():
    lib = _native.hip()
    assert lib.ps_hub_spmm_launch(None, 32, FAKE, FAKE, FAKE, 1 << 40, None) == \
        _native.PS_ERR_INVALID and "null descriptor" in last_error()
    hb = block()
    assert lib.ps_hub_spmm_launch(ctypes.byref(hb), 32, FAKE + 4, FAKE, FAKE, 1 << 40, None) == \
        _native.PS_ERR_INVALID and "16-byte aligned" in last_error()
    hb = block(dense=FAKE + 4)
    assert lib.ps_hub_spmm_launch(ctypes.byref(hb), 32, FAKE, FAKE, FAKE, 1 << 40, None) == \
        _native.PS_ERR_INVALID and "16-byte aligned" in last_error()


def sddmm(hb, N=32, plan=FAKE, count=1, out=True, worksets=2, ws=1 << 40):
    lib = _native.hip()
    w = (_native.Workset * max(worksets, 1))()
    outs = (ctypes.c_void_p * max(worksets, 1))(*([FAKE] * max(worksets, 1)))
    return lib.ps_hub_sddmm_launch(ctypes.byref(hb), worksets, w, plan, count, N, FAKE,
                                   FAKE, outs if out else None, None, None, FAKE, ws, None)


@pytest.mark.parametrize("kw,msg", [
    (dict(N=544), "between 32 and 512"),
    (dict(N=40), "between 32 and 512"),
    (dict(plan=None), "missing plan"),
    (dict(out=False), "missing outputs"),
    (dict(worksets=0), "invalid worksets"),
    (dict(ws=1024), "workspace too small"),
])
def test_sddmm_launch_rejects(kw, msg):
    rc = sddmm(block(), **kw)
    assert rc == _native.PS_ERR_INVALID and msg in last_error()


def test_sddmm_plan_rejects():
    lib = _native.hip()
    hb = block()
    w = (_native.Workset * 2)()
    need = lib.ps_hub_sddmm_plan_bytes(ctypes.byref(hb), 1)
    rc = lib.ps_hub_sddmm_plan(ctypes.byref(hb), 2, w, FAKE, 1, FAKE, need - 1, None)
    assert rc == _native.PS_ERR_INVALID and "plan buffer too small" in last_error()
    rc = lib.ps_hub_sddmm_plan(ctypes.byref(hb), 2, w, None, 1, FAKE, need, None)
    assert rc == _native.PS_ERR_INVALID and "missing tile list" in last_error()
    rc = lib.ps_hub_sddmm_plan(ctypes.byref(hb), 0, w, FAKE, 1, FAKE, need, None)
    assert rc == _native.PS_ERR_INVALID and "invalid worksets" in last_error()
    rc = lib.ps_hub_sddmm_plan(None, 2, w, FAKE, 1, FAKE, need, None)
    assert rc == _native.PS_ERR_INVALID and "null descriptor" in last_error()
    # 2^25 tiles of 64 entries reach 2^31: refused by the plan and the launch
    big = 1 << 25
    rc = lib.ps_hub_sddmm_plan(ctypes.byref(hb), 2, w, FAKE, big, FAKE, 1 << 40, None)
    assert rc == _native.PS_ERR_INVALID and "too many tiles" in last_error()
    assert sddmm(hb, count=big) == _native.PS_ERR_INVALID and "too many tiles" in last_error()
    assert lib.ps_hub_sddmm_plan_bytes(ctypes.byref(hb), big - 1) > 0
    # an empty list needs no plan work on the device beyond its empty tile table
    assert sddmm(hb, plan=None, count=0) == _native.PS_OK
