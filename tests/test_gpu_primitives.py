"""Device scan and stable radix sort against numpy."""
import ctypes

import numpy as np
import pytest

import powersparse_amd as ps
from powersparse_amd import _native
from gpu_util import say, setup

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 100, 4096, 4097, 100000, 3000001])
def test_exclusive_scan(n):
    setup()
    say(f"scan n={n}")
    rng = np.random.default_rng(n)
    x = rng.integers(0, 1000, n).astype(np.uint32)
    d = ps.DeviceBuffer(host=x)
    ws = ps.DeviceBuffer(_native.hip().ps_scan_workspace_bytes(n))
    ps._hip_call(_native.hip().ps_exclusive_scan_u32(d.ptr, d.ptr, n, ws.ptr, None))
    got = d.download(np.uint32, n)
    expect = np.concatenate([[0], np.cumsum(x, dtype=np.uint64)[:-1]]).astype(np.uint32)
    np.testing.assert_array_equal(got, expect)


@pytest.mark.parametrize("bits", [64, 32])
@pytest.mark.parametrize("n,lo,hi,keymax", [
    (1, 0, 32, 10), (2, 0, 8, 3), (1000, 0, 24, 1 << 20), (4096, 0, 32, 1 << 32),
    (70001, 4, 20, 1 << 20), (1000003, 0, 40, 1 << 40), (300000, 8, 16, 7)])
def test_radix_sort_pairs_stable(bits, n, lo, hi, keymax):
    setup()
    if bits == 32:
        hi = min(hi, 32)
        keymax = min(keymax, 1 << 32)
    say(f"radix u{bits} n={n} bits=[{lo},{hi})")
    rng = np.random.default_rng(n + bits)
    kt = np.uint64 if bits == 64 else np.uint32
    keys = rng.integers(0, keymax, n, dtype=np.uint64).astype(kt)
    vals = np.arange(n, dtype=np.uint32)
    k1, k2 = ps.DeviceBuffer(host=keys), ps.DeviceBuffer(keys.nbytes)
    v1, v2 = ps.DeviceBuffer(host=vals), ps.DeviceBuffer(vals.nbytes)
    ws = ps.DeviceBuffer(_native.hip().ps_radix_workspace_bytes(n))
    alt = ctypes.c_int(0)
    fn = _native.hip().ps_radix_sort_pairs_u64 if bits == 64 else _native.hip().ps_radix_sort_pairs_u32
    ps._hip_call(fn(k1.ptr, k2.ptr, v1.ptr, v2.ptr, n, lo, hi, ws.ptr, ctypes.byref(alt), None))
    kd, vd = (k2, v2) if alt.value else (k1, v1)
    got_k, got_v = kd.download(kt, n), vd.download(np.uint32, n)
    # only the digits covering [lo, hi) are sorted: 8-bit digits from lo upward
    nd = (hi - lo + 7) // 8
    width = min(nd * 8, bits - lo)
    sel = (keys.astype(np.uint64) >> np.uint64(lo)) & np.uint64((1 << width) - 1)
    order = np.argsort(sel, kind="stable")
    np.testing.assert_array_equal(got_v, vals[order])
    np.testing.assert_array_equal(got_k, keys[order])
