"""Fill-reducing ordering and no-pivot LU of a synthetic building's system matrix.

csim does not factorize anything: it replays baked CSC factors in SuperLU's
convention (complete_port/csim/sb_lu.c:38-63, baked by
complete_port/pysim/bake_scenario.py:131-135 with MMD on A+A^T):

    Pr A Pc = L U,   Pr[perm_r[i], i] = 1,   Pc[i, perm_c[i]] = 1
    solve:  w = b[inv(perm_r)];  L w' = w (unit);  U z = w';  x = z[perm_c]

The synthetic systems are strictly diagonally dominant by rows, so a symmetric
permutation with static diagonal pivots is stable and perm_r = inv(perm_c).
The ordering is an exact minimum-degree elimination on the pattern of A + A^T
(ties broken by the lowest index, so it is deterministic). L keeps its unit
diagonal explicitly and both factors keep their full symbolic pattern, so the
same pattern serves every numeric refactorization of A + diag(g) on the device.
"""
from __future__ import annotations

import numpy as np


def minimum_degree(pattern: list[set[int]]) -> np.ndarray:
    """Exact minimum degree on an undirected graph given as adjacency sets."""
    n = len(pattern)
    adj = [set(s) - {i} for i, s in enumerate(pattern)]
    alive = np.ones(n, dtype=bool)
    order = []
    deg = np.array([len(a) for a in adj])
    for _ in range(n):
        cand = np.where(alive)[0]
        v = int(cand[np.argmin(deg[cand])])
        order.append(v)
        nb = [u for u in adj[v] if alive[u]]
        alive[v] = False
        for u in nb:
            adj[u].discard(v)
            adj[u].update(w for w in nb if w != u)
            deg[u] = len(adj[u])
        adj[v] = set()
    return np.asarray(order, dtype=np.int64)


def symbolic_pattern(Bpat: list[set[int]]) -> list[set[int]]:
    """Filled pattern of a symmetric-pattern matrix eliminated in natural order.

    Returns for each column j the set of rows i > j with a structural entry in L
    (by symmetry, the columns of row j of U).
    """
    n = len(Bpat)
    lower = [set(i for i in Bpat[j] if i > j) for j in range(n)]
    for j in range(n):
        s = sorted(lower[j])
        for a_i, i in enumerate(s):
            lower[i].update(s[a_i + 1:])
    return lower


def factorize(A_csc) -> dict:
    """Orders and factorizes A. Returns the SuperLU-convention arrays csim reads."""
    A = A_csc.tocsc()
    n = A.shape[0]
    S = (abs(A) + abs(A.T)).tocsr()
    pattern = [set(S.indices[S.indptr[i]:S.indptr[i + 1]].tolist()) for i in range(n)]
    q = minimum_degree(pattern)               # permuted position k holds node q[k]
    pos = np.empty(n, dtype=np.int64)
    pos[q] = np.arange(n)
    Bpat = [set(int(pos[j]) for j in pattern[int(q[k])]) for k in range(n)]
    lower = symbolic_pattern(Bpat)

    B = A.toarray()[np.ix_(q, q)]
    # Doolittle without pivoting (diagonal dominance makes this stable)
    LU = B.copy()
    for k in range(n):
        piv = LU[k, k]
        if piv == 0.0:
            raise ValueError("zero pivot")
        rows = np.fromiter(sorted(lower[k]), dtype=np.int64)
        if rows.size == 0:
            continue
        LU[rows, k] /= piv
        LU[np.ix_(rows, rows)] -= np.outer(LU[rows, k], LU[k, rows])

    Lp, Li, Lx = [0], [], []
    Up, Ui, Ux = [0], [], []
    urows = [[] for _ in range(n)]            # rows r < j with a structural U[r, j]
    for r in range(n):
        for j in sorted(lower[r]):
            urows[j].append(r)
    for j in range(n):
        Li.append(j); Lx.append(1.0)
        for i in sorted(lower[j]):
            Li.append(i); Lx.append(LU[i, j])
        Lp.append(len(Li))
        for r in urows[j]:
            Ui.append(r); Ux.append(LU[r, j])
        Ui.append(j); Ux.append(LU[j, j])
        Up.append(len(Ui))
    # B = A[q][:, q] = Pr A Pc. Pr[perm_r[i], i] = 1 moves row i of A to row
    # pos[i]; Pc[i, perm_c[i]] = 1 moves column i to column pos[i].
    perm_r = pos.astype(np.int32)
    perm_c = pos.astype(np.int32)
    return {
        "perm_r": perm_r, "perm_c": perm_c,
        "L_indptr": np.asarray(Lp, np.int32), "L_indices": np.asarray(Li, np.int32),
        "L_data": np.asarray(Lx, np.float64),
        "U_indptr": np.asarray(Up, np.int32), "U_indices": np.asarray(Ui, np.int32),
        "U_data": np.asarray(Ux, np.float64),
        "order": q, "lower": lower,
    }
