"""Host logic of the measurement tooling, on the CPU: the rocprofv3 summary
(`python -m powersparse_amd.perf summarize`) on small SQLite databases shaped
like rocprofv3's, the counters bench.py reads back from it, and bench.py's
refusal of more than one GPU."""
import json
import os
import sqlite3
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from powersparse_amd import perf  # noqa: E402

KIB = 1024.0
SPMM32 = "void ps::spmm_kernel<8, true>(ps::(anonymous namespace)::SpmmArgs)"
SPMM128 = "void ps::spmm_kernel<8, true>(ps::(anonymous namespace)::SpmmArgs)"
SDDMM128 = "void ps::(anonymous namespace)::sddmm_kernel<4, true, 0>(ps::SddmmArgs)"
SDDMM32 = "void ps::(anonymous namespace)::sddmm_kernel<1, true, 0>(ps::SddmmArgs)"
COPY = "void ps::copy_f32_kernel(float*, float const*, unsigned long)"
PRE = "void ps::rank_small_kernel(int const*, int, int const*)"
FILL = "void ps::(anonymous namespace)::fill_random_kernel(float*, unsigned long)"
HUB = "void ps::(anonymous namespace)::hub_sddmm_kernel<16, true>(ps::HubSddmmArgs)"
GATHER = "ps::(anonymous namespace)::gather_rows_kernel(float const*, int const*, int)"


def counter_db(path, counter, dispatches):
    """dispatches: [(kernel, grid, value)] in dispatch order."""
    con = sqlite3.connect(path)
    con.execute("create table counters_collection (dispatch_id integer, kernel_name text, "
                "grid_size integer, counter_name text, value real)")
    con.executemany("insert into counters_collection values (?, ?, ?, ?, ?)",
                    [(i, k, g, counter, v) for i, (k, g, v) in enumerate(dispatches)])
    con.commit()
    con.close()
    return str(path)


def workload(values):
    """The perf workload's dispatch order: a warm-up and a timed copy, a
    preprocessing kernel, then each C1 operator 1 + 3 times (values[i] for
    operator i; the copy gets values['copy']), its operands filled by a kernel
    first; SDDMM N=128 calls are followed by two hub block kernels (a gather
    and the product, values['hub'] each, when given)."""
    out = [(COPY, 1 << 20, values["copy"])] * 2 + [(PRE, 4096, 7.0)]
    # SpMM N=32 and N=128 share a kernel and differ in grid (32-column slices)
    launches = [(SPMM32, 1000), (SPMM128, 4000), (SDDMM128, 3000), (SDDMM32, 3000)]
    for (kernel, grid), v in zip(launches, values["ops"]):
        out.append((FILL, 512, 1e6))  # not part of any call
        call = [(kernel, grid, v)]
        if kernel == SDDMM128 and "hub" in values:
            call += [(GATHER, 64, values["hub"]), (HUB, 128, values["hub"])]
        out += call * 4
    return out


@pytest.fixture
def dbs(tmp_path):
    trace = tmp_path / "kt.db"
    con = sqlite3.connect(trace)
    con.execute("create table kernels (name text, grid_x integer, grid_y integer, "
                "grid_z integer, duration real)")
    con.executemany("insert into kernels values (?, ?, 1, 1, ?)",
                    [(SPMM32, 1000, 640e3), (SPMM32, 1000, 650e3), (SDDMM128, 3000, 2.77e6),
                     (PRE, 4096, 10e3)])
    con.commit()
    con.close()
    # FETCH reads the 1 GiB copy as 2 GiB (factor 0.5), WRITE as 1 GiB (factor 1)
    fetch = counter_db(tmp_path / "f.db", "FETCH_SIZE",
                       workload({"copy": 2 * (1 << 30) / KIB, "ops": [1000, 2000, 3000, 4000],
                                 "hub": 100}))
    write = counter_db(tmp_path / "w.db", "WRITE_SIZE",
                       workload({"copy": (1 << 30) / KIB, "ops": [10, 20, 30, 40]}))
    # hit rates 45, 30, 25 (with the hub kernels: (250 + 2 * 375) / 2000 = 50),
    # 40 % from TCC_HIT_sum / (TCC_HIT_sum + TCC_MISS_sum), over each call
    l2 = counter_db(tmp_path / "l2.db", "TCC_HIT_sum",
                    workload({"copy": 1.0, "ops": [450.0, 300.0, 250.0, 40.0], "hub": 375.0}))
    con = sqlite3.connect(l2)
    con.executemany("insert into counters_collection values (?, ?, ?, ?, ?)",
                    [(100 + i, k, g, "TCC_MISS_sum", v) for i, (k, g, v) in enumerate(
                        workload({"copy": 1.0, "ops": [550.0, 700.0, 750.0, 60.0],
                                  "hub": 125.0}))])
    con.commit()
    con.close()
    valu = tmp_path / "v.db"
    counter_db(valu, "VALUBusy", workload({"copy": 5.0, "ops": [11.0, 12.0, 13.0, 14.0]}))
    con = sqlite3.connect(valu)
    con.executemany("insert into counters_collection values (?, ?, ?, ?, ?)",
                    [(100 + i, k, g, "VALUUtilization", v) for i, (k, g, v) in enumerate(
                        workload({"copy": 99.0, "ops": [90.0, 91.0, 92.0, 93.0]}))])
    con.commit()
    con.close()
    return dict(trace=str(trace), fetch=fetch, write=write, l2=l2, valu=str(valu))


def test_summary_traffic_and_counters(dbs, tmp_path, capsys):
    out = tmp_path / "traffic.json"
    perf.main(["summarize", "--config", "C1", "--trace", dbs["trace"], "--fetch", dbs["fetch"],
               "--write", dbs["write"], "--l2", dbs["l2"], "--valu", dbs["valu"],
               "--json", str(out)])
    summary = json.loads(out.read_text())
    assert summary["calibration"] == {"fetch": 0.5, "write": 1.0}
    t = summary["traffic"]
    assert list(t) == ["spmm_N32", "spmm_N128", "sddmm_N128", "sddmm_N32"]
    # bytes = KiB * 1024 * calibration factor; a call's bytes include the hub
    # kernels after the sparse launch, the operand fills belong to no call
    assert t["spmm_N32"]["fetch_bytes"] == 1000 * KIB * 0.5
    assert t["sddmm_N32"]["write_bytes"] == 40 * KIB
    assert t["sddmm_N128"]["traffic_bytes"] == (3000 + 2 * 100) * KIB * 0.5 + 30 * KIB
    assert t["sddmm_N128"]["kernel_traffic_bytes"] == 3000 * KIB * 0.5 + 30 * KIB
    assert t["sddmm_N128"]["kernels_per_call"] == 3 and t["spmm_N128"]["kernels_per_call"] == 1
    assert t["spmm_N128"]["traffic_bytes"] == t["spmm_N128"]["kernel_traffic_bytes"]
    c = summary["counters"]
    assert c["spmm_N128"] == {"l2_hit_pct": 30.0, "valu_busy_pct": 12.0,
                              "valu_utilization_pct": 91.0}
    assert c["sddmm_N128"]["l2_hit_pct"] == 50.0
    assert c["sddmm_N32"]["l2_hit_pct"] == 40.0
    # kernel table: busiest first (dispatches x mean duration)
    table = summary["kernels"]
    assert table[0]["kernel"].startswith("ps::") and "sddmm_kernel<4" in table[0]["kernel"]
    assert table[1]["dispatches"] == 2 and table[1]["mean_us"] == pytest.approx(645.0)
    assert "| sddmm N=32 | 40.0 | 14.0 | 93.0 |" in capsys.readouterr().out


def test_bench_reads_counters(dbs, tmp_path, monkeypatch):
    import bench
    profiles = tmp_path / "profiles"
    profiles.mkdir()
    perf.main(["summarize", "--config", "C1", "--trace", dbs["trace"], "--fetch", dbs["fetch"],
               "--write", dbs["write"], "--l2", dbs["l2"], "--valu", dbs["valu"],
               "--json", str(profiles / "traffic_C1.json")])
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    traffic, counters, src, note = bench.measured_counters("C1", "sddmm", 128)
    assert traffic == (3000 + 2 * 100) * KIB * 0.5 + 30 * KIB  # the whole call
    assert counters["valu_busy_pct"] == 13.0 and src == os.path.join("profiles", "traffic_C1.json")
    assert "same kernel sources" in note
    assert bench.measured_counters("C4", "spmm", 64) == (None, {}, None, "no profile summary")
    # a summary made from other kernel sources is not used
    path = profiles / "traffic_C1.json"
    summary = json.loads(path.read_text())
    summary["sources_digest"] = "0" * 16
    path.write_text(json.dumps(summary))
    traffic, counters, src, note = bench.measured_counters("C1", "sddmm", 128)
    assert traffic is None and counters == {} and "other kernel sources" in note


def test_bench_one_gpu_only():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU only" in r.stderr


def test_operator_calls_take_the_hub_kernels_that_follow():
    """A call is the operator kernel's dispatch plus the dispatches after it up
    to the next operator kernel; calls take the workload's operators in turn;
    dispatches before the first operator kernel belong to no call."""
    HUB_SPMM = "void ps::(anonymous namespace)::hub_spmm_kernel<4, 4>(ps::HubSpmmArgs)"
    HUB_SDDMM = "void ps::(anonymous namespace)::hub_sddmm_kernel<16, true>(ps::HubSddmmArgs)"
    GATHER = "ps::(anonymous namespace)::gather_rows_kernel(float const*, int const*, int)"
    assert perf.kernel_op(HUB_SPMM) is None and perf.kernel_op(HUB_SDDMM) is None
    assert perf.kernel_op(SDDMM128) == ("sddmm", 4) and perf.kernel_op(SPMM32) == ("spmm", 8)
    seq = [(PRE, 4096, 50.0)]
    for _ in range(3):  # three steps of C3: SpMM 32, SpMM 128, SDDMM 128
        seq += [(SPMM32, 1000, 1300.0), (HUB_SPMM, 64, 140.0), (HUB_SPMM, 64, 60.0),
                (SPMM128, 4000, 5100.0), (HUB_SPMM, 64, 340.0),
                (SDDMM128, 3000, 5500.0), (GATHER, 64, 430.0), (HUB_SDDMM, 512, 340.0)]
    got = perf.operator_calls(seq, [("spmm", 32), ("spmm", 128), ("sddmm", 128)])
    assert got == {"spmm_N32": (3, 3, 1500.0), "spmm_N128": (3, 2, 5440.0),
                   "sddmm_N128": (3, 3, 6270.0)}


def test_class_split_summary(tmp_path, capsys):
    """`classes-summarize`: operator dispatches matched to the manifest in
    order (2 launches per class), durations averaged, FETCH / WRITE scaled by
    the calibration copy, bytes per nonzero and the share of the all-class
    launch; a dispatch count that disagrees with the manifest is refused."""
    manifest = tmp_path / "m.txt"
    entries = [{"op": "sddmm", "N": 128, "class": "all", "nnz": 1000, "tasks": 10, "launches": 2},
               {"op": "sddmm", "N": 128, "class": "residue", "nnz": 250, "tasks": 4,
                "launches": 2}]
    manifest.write_text("noise\n" + "\n".join(json.dumps(e) for e in entries) + "\ndone\n")
    trace = tmp_path / "kt.db"
    con = sqlite3.connect(trace)
    con.execute("create table kernels (name text, grid_x integer, grid_y integer, "
                "grid_z integer, duration real, start integer)")
    rows = [(COPY, 1 << 20, 1e6), (SDDMM128, 3000, 100e3), (SDDMM128, 3000, 300e3),
            (PRE, 64, 5e3), (SDDMM128, 1000, 40e3), (SDDMM128, 1000, 60e3)]
    con.executemany("insert into kernels values (?, ?, 1, 1, ?, ?)",
                    [(k, g, d, i) for i, (k, g, d) in enumerate(rows)])
    con.commit()
    con.close()
    # FETCH reads the 1 GiB copy as 2 GiB (factor 0.5), WRITE as 1 GiB
    fetch = counter_db(tmp_path / "f.db", "FETCH_SIZE",
                       [(COPY, 1 << 20, 2 * (1 << 30) / KIB), (SDDMM128, 3000, 2e6 / KIB),
                        (SDDMM128, 3000, 2e6 / KIB), (SDDMM128, 1000, 1e6 / KIB),
                        (SDDMM128, 1000, 1e6 / KIB)])
    write = counter_db(tmp_path / "w.db", "WRITE_SIZE",
                       [(COPY, 1 << 20, (1 << 30) / KIB), (SDDMM128, 3000, 1e6 / KIB),
                        (SDDMM128, 3000, 1e6 / KIB), (SDDMM128, 1000, 0.0),
                        (SDDMM128, 1000, 0.0)])
    args = ["classes-summarize", "--manifest", str(manifest), "--trace", str(trace),
            "--fetch", fetch, "--write", write]
    assert perf.main(args) == 0
    out = capsys.readouterr().out.splitlines()
    # all: 200 us, 1 + 1 = 2 MB, 2000 B per nonzero; residue: 50 us, 0.5 MB, 25 %
    assert out[2] == "| sddmm N=128 | all | 0.0 | 10 | 200.0 | 2.0 | 2000.0 |  |"
    assert out[3] == "| sddmm N=128 | residue | 0.0 | 4 | 50.0 | 0.5 | 2000.0 | 25.0% |"
    entries[1]["launches"] = 3
    manifest.write_text("\n".join(json.dumps(e) for e in entries) + "\n")
    with pytest.raises(SystemExit, match="dispatch counts differ"):
        perf.main(args)


def test_sources_digest_follows_code_not_comments(tmp_path):
    """The digest tying a profile summary to its kernel sources changes with
    the code and not with comments, blank lines or indentation."""
    def tree(text):
        root = tmp_path / str(abs(hash(text)))
        (root / "powersparse_amd" / "csrc").mkdir(parents=True)
        (root / "include").mkdir()
        (root / "powersparse_amd" / "csrc" / "k.hip").write_text(text)
        (root / "include" / "powersparse_hip.h").write_text("int f(int);\n")
        return perf.sources_digest(str(root))

    base = tree("__global__ void k(float* p) {\n  p[0] = 1.f;  // one\n}\n")
    assert tree("/* a kernel */\n__global__ void k(float* p) {\n\n    p[0] = 1.f;\n}\n") == base
    assert tree("__global__ void k(float* p) {\n  p[0] = 2.f;  // one\n}\n") != base
    assert perf.code_text("a; // b\n/* c\n d */ e  f;\n") == "a;\ne f;"
