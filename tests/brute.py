"""Independent, deliberately naive restatement of the reference preprocessing
(ParCIS/PowerSparse utils/matrix_utils.cu:31-663) for tiny graphs, used to
cross-check the C++ oracle. It shares no code with it and uses different
means: Python's stable sorted() with explicit keys, signatures as one big
integer per group (bit i of the L-bit signature has weight 2^(L-1-i), so the
reference's lexicographic word-by-word descending order is plain integer
order), and a direct comparison sort of the groups.

The column signature bits come from the caller: they depend on libstdc++'s
unstable std::sort tie order, which only C++ can reproduce (checked separately).
"""


def group_size(s):
    return 32 << (s - 1)


def worksets_count(degrees, cu_count):
    threshold = 8 * cu_count * 4
    s = 1
    while sum(d // group_size(s) for d in degrees) >= threshold:
        s += 1
    return s


def preprocess(rows, cols, row_ptr, col_ind, values, cu_count, sigbit, sig_len, fine=16,
               max_group_types=0):
    """max_group_types caps S (0: no cap); the split of each row below is the
    same greedy cut from the largest allowed group size down."""
    degrees = [row_ptr[r + 1] - row_ptr[r] for r in range(rows)]
    S = worksets_count(degrees, cu_count)
    if max_group_types:
        S = min(S, max_group_types)
    col_nnz = [0] * cols
    for c in col_ind:
        col_nnz[c] += 1
    # groups[s] = list of (row, [positions in ranked order])
    groups = [[] for _ in range(S)]
    atomic0 = []
    for r in range(rows):
        ranked = sorted(range(row_ptr[r], row_ptr[r + 1]), key=lambda p: -col_nnz[col_ind[p]])
        d = len(ranked)
        if S == 1:
            chunks = [ranked[i:i + fine] for i in range(0, d, fine)]
            for ch in chunks:
                groups[0].append((r, ch))
                atomic0.append(len(chunks) > 1)
            continue
        at = 0
        for s in range(S - 1, 0, -1):
            size = group_size(s)
            while d - at >= size:
                groups[s].append((r, ranked[at:at + size]))
                at += size
        if at < d:
            groups[0].append((r, ranked[at:]))
            atomic0.append(d > 32)

    def signature(members):
        value = 0
        for p in members:
            value |= 1 << (sig_len - 1 - sigbit[col_ind[p]])
        return value

    out = []
    for s in range(S):
        sigs = [signature(m) for _, m in groups[s]]
        order = sorted(range(len(groups[s])), key=lambda g: (-sigs[g], g))
        cols_out, vals_out, des, offs, atom = [], [], [], [0], []
        for g in order:
            r, members = groups[s][g]
            members = sorted(members, key=lambda p: (col_ind[p], members.index(p)))
            cols_out += [col_ind[p] for p in members]
            vals_out += [values[p] for p in members]
            des.append(r)
            offs.append(offs[-1] + len(members))
            if s == 0:
                atom.append(atomic0[g])
        out.append({"col": cols_out, "val": vals_out, "des": des, "offsets": offs,
                    "atomic": atom, "perm": order})
    return S, out
