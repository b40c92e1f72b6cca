"""Helpers shared by the GPU tests: device setup, uploading oracle worksets,
and running the product path next to the oracle."""
import sys

import numpy as np

import oracle
import powersparse_amd as ps

_ready = False


def setup():
    global _ready
    if not _ready:
        ps.set_device(0)
        _ready = True


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


class Uploaded:
    """Oracle worksets copied to the device, in ps_workset tuple form."""

    def __init__(self, w):
        self.bufs = []
        self.worksets = []
        for s in range(w.S):
            col = ps.DeviceBuffer(host=w.col[s]) if w.col[s].size else None
            val = ps.DeviceBuffer(host=w.val[s]) if w.val[s].size else None
            des = ps.DeviceBuffer(host=w.des[s]) if w.des[s].size else None
            self.bufs += [col, val, des]
            gs = 0 if s == 0 else 32 << (s - 1)
            self.worksets.append((col, val, des, w.group_num[s], gs))
        self.offset = ps.DeviceBuffer(host=w.residue_offset)
        self.atomic = ps.DeviceBuffer(host=w.residue_atomic) if w.residue_atomic.size else \
            ps.DeviceBuffer(16)


def csr_arrays(csr):
    return csr.rows, csr.cols, csr.row_ptr, csr.col_ind, csr.values


def random_graph(rng, rows, cols, max_deg, hubs=0, hub_deg=0, dup=False):
    rp = [0]
    ci = []
    for r in range(rows):
        d = int(rng.integers(0, max_deg + 1))
        if r < hubs:
            d = hub_deg
        d = min(d, cols) if not dup else d
        if dup:
            row = rng.integers(0, cols, size=d)
        else:
            row = np.sort(rng.choice(cols, size=d, replace=False))
        ci.append(row.astype(np.int32))
        rp.append(rp[-1] + d)
    ci = np.concatenate(ci) if ci else np.zeros(0, np.int32)
    va = rng.uniform(-1, 1, ci.size).astype(np.float32)
    return ps.HostCsr(rows, cols, np.array(rp, np.int32), ci, va)


def star_graph(rng, rows, cols, max_deg, long_rows=0, long_deg=0):
    """Every row holds the two hub columns 0 and 1 plus up to max_deg random
    other columns (long_rows rows: long_deg): two columns as popular as there
    are rows, ties everywhere else."""
    rp, ci = [0], []
    for r in range(rows):
        d = long_deg if r < long_rows else int(rng.integers(0, max_deg + 1))
        other = np.unique(rng.integers(2, cols, d))
        ci.append(np.concatenate([[0, 1], other]).astype(np.int32))
        rp.append(rp[-1] + len(ci[-1]))
    ci = np.concatenate(ci)
    return ps.HostCsr(rows, cols, np.array(rp, np.int32), ci,
                      rng.uniform(-1, 1, ci.size).astype(np.float32))
