"""CPU-only checks of the dense hub block's C ABI: the workspace sizes follow
the stated layout, and every launcher rejects bad arguments with
PS_ERR_INVALID and a message before it makes any device call (the pointers
below are never dereferenced)."""
import ctypes

import pytest

from powersparse_amd import _native

FAKE = 0x10000  # a non-null, 16-byte aligned stand-in address
BLAS_WS = 32 << 20


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


def test_workspace_and_stored_words():
    lib = _native.hip()
    hb = block(rows=5, cols=70)
    assert lib.ps_hub_stored_words(ctypes.byref(hb)) == 5 * 3
    assert lib.ps_hub_stored_words(None) == 0
    N = 32
    spmm = r256(70 * N * 4) + r256(5 * N * 4) + r256(70 * 4) + 256 + BLAS_WS
    sddmm = r256(5 * N * 4) + r256(70 * N * 4) + r256(5 * 70 * 4) + BLAS_WS
    assert lib.ps_hub_workspace_bytes(ctypes.byref(hb), _native.PS_OP_SPMM, N) == spmm
    assert lib.ps_hub_workspace_bytes(ctypes.byref(hb), _native.PS_OP_SDDMM, N) == sddmm
    assert lib.ps_hub_workspace_bytes(ctypes.byref(hb), _native.PS_OP_SPMM, 0) == 0


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


def sddmm(hb, N=32, ws=1 << 40, tiles=FAKE, doff=FAKE, count=1, out=True, worksets=2):
    lib = _native.hip()
    w = (_native.Workset * worksets)()
    outs = (ctypes.c_void_p * max(worksets, 1))(*([FAKE] * max(worksets, 1)))
    return lib.ps_hub_sddmm_launch(ctypes.byref(hb), worksets, w, tiles, doff, count, N, FAKE,
                                   FAKE, outs if out else None, None, None, FAKE, ws, None)


@pytest.mark.parametrize("kw,msg", [
    (dict(N=544), "between 32 and 512"),
    (dict(N=40), "between 32 and 512"),
    (dict(doff=None), "missing tile offsets"),
    (dict(tiles=None), "missing tile list"),
    (dict(out=False), "missing outputs"),
    (dict(ws=1024), "workspace too small"),
    (dict(worksets=0), "invalid worksets"),
])
def test_sddmm_launch_rejects(kw, msg):
    rc = sddmm(block(), **kw)
    assert rc == _native.PS_ERR_INVALID and msg in last_error()


def test_offsets_need_32_bit_dense_elements():
    lib = _native.hip()
    hb = block(rows=1 << 16, cols=1 << 16)  # 2^32 dense elements
    w = (_native.Workset * 2)()
    rc = lib.ps_hub_tile_offsets(ctypes.byref(hb), 2, w, FAKE, 1, FAKE, None)
    assert rc == _native.PS_ERR_INVALID and "32-bit offsets" in last_error()
    assert sddmm(hb) == _native.PS_ERR_INVALID and "32-bit offsets" in last_error()
    hb = block()
    assert lib.ps_hub_tile_offsets(ctypes.byref(hb), 2, w, FAKE, 1, None, None) == \
        _native.PS_ERR_INVALID and "null output" in last_error()
    # an empty list is a no-op
    assert lib.ps_hub_tile_offsets(ctypes.byref(hb), 2, w, None, 0, None, None) == _native.PS_OK
