"""Command-line tools around the benchmark binaries (powersparse_amd/bin)."""
