"""Batch runner: every selected matrix x every width through one benchmark
binary, into one CSV.

    python -m powersparse_amd.cli.run_benchmarks BUILD_DIR DATASET_ROOT {spmm|sddmm} DEVICE
        OUTPUT.csv [N_LIST] [REPEATS] [CHECK]

Contract of the reference's scripts/run_benchmarks.sh:1-64, kept:
  * arguments, defaults (N_LIST 32,128; REPEATS 100; CHECK 0) and checks;
    usage and argument errors exit 2, missing inputs or an existing output exit 1;
  * the binary is BUILD_DIR/bin/powersparse_{spmm,sddmm} (BUILD_DIR is
    `powersparse_amd` for the in-tree build);
  * inputs: every *.mtx directly in DATASET_ROOT (sorted by name), or the
    entries of the manifest named by $DATASET_LIST, relative to DATASET_ROOT,
    blank lines and '#' comments skipped, CR line ends tolerated; every input
    is checked before anything runs;
  * the CSV is written to OUTPUT.partial (created exclusively: an existing
    OUTPUT or OUTPUT.partial is refused) and renamed to OUTPUT only when every
    run succeeded; a failed run leaves the .partial file and returns the
    binary's exit status. Rows are matrix-major, widths inner.
Differences, following this build's binaries: N = 64 is accepted besides 32
and 128; the default selection also takes *.pscsr binary CSRs; a manifest
entry `synth:NAME[:SEED[:SCALE]]` names a generated graph and is passed through.
With PS_BENCH_LAUNCHER=python every run goes through the same harness from a
Python process instead (`python -m powersparse_amd.cli OP ...`, the package
being BUILD_DIR, which must hold lib/libpowersparse_bench.so), with the same
arguments, output and exit codes.
"""
import os
import re
import subprocess
import sys

USAGE = """\
Usage: python -m powersparse_amd.cli.run_benchmarks BUILD_DIR DATASET_ROOT {spmm|sddmm} DEVICE OUTPUT.csv [N_LIST] [REPEATS] [CHECK]
N_LIST is comma-separated (default: 32,128). REPEATS defaults to 100; CHECK to 0.
By default, all .mtx (and .pscsr) files directly in DATASET_ROOT are selected.
Set DATASET_LIST to a manifest to select specific inputs.
Paths in the manifest are relative to DATASET_ROOT. Blank lines and # comments are ignored.
Manifest entries of the form synth:NAME[:SEED[:SCALE]] select generated graphs.
"""
WIDTHS = (32, 64, 128)


class Stop(Exception):
    """Ends the run with a message on stderr and an exit status."""

    def __init__(self, status, message=None):
        super().__init__(message)
        self.status = status
        self.message = message


def parse(argv):
    if not 5 <= len(argv) <= 8:
        raise Stop(2, USAGE.rstrip("\n"))
    build_dir, root, op, device, output = argv[:5]
    n_list = argv[5] if len(argv) > 5 else "32,128"
    repeats = argv[6] if len(argv) > 6 else "100"
    check = argv[7] if len(argv) > 7 else "0"
    if op not in ("spmm", "sddmm"):
        raise Stop(2, "Operator must be spmm or sddmm.")
    if not (re.fullmatch(r"[0-9]+", device) and re.fullmatch(r"[1-9][0-9]*", repeats)
            and re.fullmatch(r"[01]", check)):
        raise Stop(2, "Invalid DEVICE, REPEATS or CHECK.")
    if not re.fullmatch(r"[1-9][0-9]*(,[1-9][0-9]*)*", n_list):
        raise Stop(2, "Invalid N_LIST.")
    widths = [int(n) for n in n_list.split(",")]
    for n in widths:
        if n not in WIDTHS:
            raise Stop(2, f"{op} benchmark: N={n} was not selected in main; "
                          "please use N=32, 64 or 128.")
    return dict(build_dir=build_dir, root=root, op=op, device=device, output=output,
                widths=widths, repeats=repeats, check=check)


def select_inputs(root, manifest):
    """Matrix arguments for the binary, in run order."""
    if manifest:
        if not (os.path.isfile(manifest) and os.access(manifest, os.R_OK)):
            raise Stop(1, f"Cannot read manifest: {manifest}")
        inputs = []
        with open(manifest, newline="") as fh:
            for line in fh.read().split("\n"):
                entry = line[:-1] if line.endswith("\r") else line
                stripped = entry.strip()
                if not stripped or stripped.startswith("#"):
                    continue
                inputs.append(entry if entry.startswith("synth:") else os.path.join(root, entry))
    else:
        try:
            names = sorted(os.listdir(root))
        except OSError:
            names = []
        inputs = [os.path.join(root, n) for n in names
                  if n.endswith((".mtx", ".pscsr")) and os.path.isfile(os.path.join(root, n))]
    if not inputs:
        raise Stop(1, "No matrices selected.")
    for path in inputs:
        if path.startswith("synth:"):
            continue
        if not (os.path.isfile(path) and os.access(path, os.R_OK)):
            raise Stop(1, f"Missing matrix: {path}")
    return inputs


def launcher(cfg, kind):
    """(command prefix, environment) that runs one benchmark call."""
    op = cfg["op"]
    if kind == "python":
        package = os.path.abspath(cfg["build_dir"])
        lib = os.path.join(package, "lib", "libpowersparse_bench.so")
        if not os.path.isfile(lib):
            raise Stop(1, f"Missing library: {lib}")
        env = dict(os.environ)
        parent = os.path.dirname(package)
        env["PYTHONPATH"] = os.pathsep.join(
            p for p in (parent, env.get("PYTHONPATH", "")) if p)
        return [sys.executable, "-m", f"{os.path.basename(package)}.cli", op], env
    if kind not in ("", "binary"):
        raise Stop(2, f"Unknown PS_BENCH_LAUNCHER: {kind} (use binary or python)")
    binary = os.path.join(cfg["build_dir"], "bin", f"powersparse_{op}")
    if not (os.path.isfile(binary) and os.access(binary, os.X_OK)):
        raise Stop(1, f"Missing executable: {binary}")
    return [binary], None


def run(cfg, manifest, kind=""):
    command, env = launcher(cfg, kind)
    inputs = select_inputs(cfg["root"], manifest)
    output = cfg["output"]
    partial = output + ".partial"
    parent = os.path.dirname(output)
    if parent:
        os.makedirs(parent, exist_ok=True)
    # Refuse to overwrite a previous run; a failed run stays explicitly partial.
    if os.path.exists(output) or os.path.exists(partial):
        raise Stop(1, f"Output already exists: {output} (or .partial)")
    try:
        fd = os.open(partial, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o644)
    except FileExistsError:
        raise Stop(1, f"Output already exists: {output} (or .partial)") from None
    with os.fdopen(fd, "w") as fh:
        fh.flush()
        status = subprocess.call(command + ["--header"], stdout=fh, env=env)
        if status != 0:
            raise Stop(status)
        for path in inputs:
            for n in cfg["widths"]:
                fh.flush()
                status = subprocess.call(command + [path, str(n), cfg["device"], cfg["check"],
                                                    cfg["repeats"]], stdout=fh, env=env)
                if status != 0:
                    raise Stop(status)
    os.replace(partial, output)
    print(f"Results saved to {output}", file=sys.stderr)


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    try:
        run(parse(argv), os.environ.get("DATASET_LIST", ""),
            os.environ.get("PS_BENCH_LAUNCHER", ""))
    except Stop as stop:
        if stop.message:
            print(stop.message, file=sys.stderr)
        return stop.status
    return 0


if __name__ == "__main__":
    sys.exit(main())
