"""ps_exclusive_scan_u32_noalloc (the scan that allocates nothing: its tile
sums live in a static per-GPU scratch array) against ps_exclusive_scan_u32
with a caller workspace, through the C ABI: bitwise-equal results on two calls
in a row (the second smaller, so stale tile sums of the first would show), in
place and out of place; a size beyond the scratch is rejected before any work."""
import numpy as np
import pytest

import powersparse_amd as ps
from powersparse_amd import _native
from gpu_util import say, setup

pytestmark = pytest.mark.gpu


def scan_with_workspace(x):
    d = ps.DeviceBuffer(host=x)
    ws = ps.DeviceBuffer(max(_native.hip().ps_scan_workspace_bytes(x.size), 16))
    ps._hip_call(_native.hip().ps_exclusive_scan_u32(d.ptr, d.ptr, x.size, ws.ptr, None))
    return d.download(np.uint32, x.size)


def test_noalloc_scan_matches_workspace_scan():
    setup()
    rng = np.random.default_rng(5)
    st = ps.Stream()
    for n, in_place in ((3000001, False), (100000, True), (4097, False)):
        say(f"no-alloc scan n={n} in_place={in_place}")
        x = rng.integers(0, 5000, n).astype(np.uint32)
        d_in = ps.DeviceBuffer(host=x)
        d_out = d_in if in_place else ps.DeviceBuffer(n * 4)
        ps._hip_call(_native.hip().ps_exclusive_scan_u32_noalloc(d_in.ptr, d_out.ptr, n, st.ptr))
        st.synchronize()
        got = d_out.download(np.uint32, n)
        np.testing.assert_array_equal(got, scan_with_workspace(x))
        # the closed form as well: exclusive prefix sums modulo 2^32
        expect = np.zeros(n, np.uint64)
        expect[1:] = np.cumsum(x[:-1], dtype=np.uint64)
        np.testing.assert_array_equal(got, (expect & 0xFFFFFFFF).astype(np.uint32))


def test_noalloc_scan_rejects_sizes_beyond_its_scratch():
    setup()
    d = ps.DeviceBuffer(16)
    rc = _native.hip().ps_exclusive_scan_u32_noalloc(d.ptr, d.ptr, 1 << 31, None)
    assert rc == _native.PS_ERR_INVALID
    assert b"static scratch" in _native.hip().ps_last_error()
    # n = 0 is a no-op
    assert _native.hip().ps_exclusive_scan_u32_noalloc(d.ptr, d.ptr, 0, None) == _native.PS_OK
