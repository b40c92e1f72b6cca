"""SpMM / SDDMM kernels on worksets built by the CPU oracle and uploaded, so
the kernels are checked independently of the GPU preprocessing. Outputs are
compared with the oracle's double-precision CheckSpmm / CheckSddmm
(tests/tolerance.py states the bound)."""
import numpy as np
import pytest

import oracle
import powersparse_amd as ps
import tolerance
from gpu_util import Uploaded, random_graph, say, setup

pytestmark = pytest.mark.gpu

GRAPHS = {
    # name: (builder, cu_count) -- cu_count picks how many worksets appear
    "c0_fine": (lambda: ps.synth("C0", seed=1), 256),
    "c1_small": (lambda: ps.synth("C1", seed=2, scale=200), 1),
    "c3_small": (lambda: ps.synth("C3", seed=3, scale=400), 1),
    "c4_small": (lambda: ps.synth("C4", seed=4, scale=128), 2),
    "hubs": (lambda: random_graph(np.random.default_rng(5), 300, 5000, 40, hubs=6,
                                  hub_deg=4500), 1),
    "dups": (lambda: random_graph(np.random.default_rng(6), 200, 50, 90, dup=True), 1),
}
_cache = {}


def graph(name):
    if name not in _cache:
        build, cu = GRAPHS[name]
        csr = build()
        w = oracle.preprocess(csr.rows, csr.cols, csr.row_ptr, csr.col_ind, csr.values, cu)
        _cache[name] = (csr, w)
    return _cache[name]


def row_factor(csr, w):
    """1 for rows written by a single non-atomic residue group, 2 otherwise:
    the factor two back-to-back calls without clearing C leave on each row."""
    f = np.full(csr.rows, 2.0)
    for g, r in enumerate(w.des[0]):
        if not w.residue_atomic[g]:
            f[r] = 1.0
    return f


@pytest.mark.parametrize("name", sorted(GRAPHS))
@pytest.mark.parametrize("N", [32, 64, 128, 96, 256, 288])
def test_spmm_kernel(name, N):
    setup()
    csr, w = graph(name)
    say(f"spmm kernel {name} S={w.S} groups={w.group_num} N={N}")
    up = Uploaded(w)
    rng = np.random.default_rng(N)
    B = rng.uniform(-1, 1, (csr.cols, N)).astype(np.float32)
    dB = ps.DeviceBuffer(host=B)
    dC = ps.DeviceBuffer.zeros(csr.rows * N * 4)
    ps.spmm_launch(up.worksets, up.offset, up.atomic, csr.rows, csr.cols, N, dB, dC)
    ps.synchronize()
    C = dC.download(np.float32).reshape(csr.rows, N)
    E, M = oracle.spmm(csr.row_ptr, csr.col_ind, csr.values, N, B, with_mag=True)
    stats = tolerance.check(C, E, M, f"spmm {name} N={N}")
    say("  ", stats)
    # second call without clearing: atomic rows accumulate, stored rows are rewritten
    ps.spmm_launch(up.worksets, up.offset, up.atomic, csr.rows, csr.cols, N, dB, dC)
    ps.synchronize()
    C2 = dC.download(np.float32).reshape(csr.rows, N)
    f = row_factor(csr, w)[:, None]
    tolerance.check(C2, E * f, M * f, f"spmm {name} N={N} second call")


@pytest.mark.parametrize("name", sorted(GRAPHS))
@pytest.mark.parametrize("N", [32, 64, 128, 96])
def test_sddmm_kernel(name, N):
    setup()
    csr, w = graph(name)
    say(f"sddmm kernel {name} S={w.S} groups={w.group_num} N={N}")
    up = Uploaded(w)
    rng = np.random.default_rng(1000 + N)
    X = rng.normal(size=(csr.rows, N)).astype(np.float32)
    Y = rng.normal(size=(csr.cols, N)).astype(np.float32)
    dX, dY = ps.DeviceBuffer(host=X), ps.DeviceBuffer(host=Y)
    outs = [ps.DeviceBuffer.zeros(max(w.col[s].size, 1) * 4) for s in range(w.S)]
    ps.sddmm_launch(up.worksets, up.offset, csr.rows, csr.cols, N, dX, dY, outs)
    ps.synchronize()
    got = []
    for s in range(w.S):
        E, M = oracle.sddmm(w.des[s], w.offsets(s), w.col[s], w.val[s], N, X, Y, with_mag=True)
        G = outs[s].download(np.float32, w.col[s].size)
        got.append(G)
        tolerance.check(G, E, M, f"sddmm {name} N={N} workset {s}")
    # second call: block outputs are stored again, residue outputs accumulate
    ps.sddmm_launch(up.worksets, up.offset, csr.rows, csr.cols, N, dX, dY, outs)
    ps.synchronize()
    for s in range(w.S):
        G2 = outs[s].download(np.float32, w.col[s].size)
        if s == 0:
            np.testing.assert_allclose(G2, 2 * got[0], rtol=1e-6, atol=1e-6)
        else:
            np.testing.assert_array_equal(G2, got[s])


def test_launch_argument_checks():
    setup()
    csr, w = graph("c1_small")
    up = Uploaded(w)
    dB = ps.DeviceBuffer(csr.cols * 48 * 4)
    dC = ps.DeviceBuffer(csr.rows * 48 * 4)
    with pytest.raises(ValueError, match="multiple of 32"):
        ps.spmm_launch(up.worksets, up.offset, up.atomic, csr.rows, csr.cols, 48, dB, dC)
    with pytest.raises(ValueError, match="between 32 and 512"):
        ps.sddmm_launch(up.worksets, up.offset, csr.rows, csr.cols, 544, dB, dB,
                        [dC] * w.S)
    with pytest.raises(ValueError, match="Missing SDDMM output"):
        ps.sddmm_launch(up.worksets, up.offset, csr.rows, csr.cols, 32, dB, dB,
                        [None] * w.S)
