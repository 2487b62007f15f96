"""The field scenarios' convection plan (csrc/field_env_kernel.hip,
fe_conv_plan_kernel) restated step for step in Python and checked against
the reference core's sequential algorithm (complete_port/csim/sb_convect.c:
39-73 with sb_rng.c's masked-rejection interval draw), on the CPU:

  - window rounds: lane i of a 64-lane window holds the stream words at
    offsets 2i, 2i + 1, 2i + 2; the two parities' swap bits (P0, P1) shifted
    by half the drift give every cell's decision, and each swap's candidate
    draw reads its words from the same window's first 128 words (or, past
    them, from the stream):
    the pairs and the stream position after the room equal the sequential
    draws, over random rooms (sizes 1..700, p from 0.05 to 1, cells without
    or with one candidate);
  - the shuffle composed into the room's inverse permutation q from the top
    (q <- q o (a b) as each pair becomes final) and applied as moves
    T_new[q[i]] = T_old[i] equals the reference's Fisher-Yates shuffle then
    swaps in order.
"""
from __future__ import annotations

import numpy as np

W = 64


def smear(x: int) -> int:
    for s in (1, 2, 4, 8, 16):
        x |= x >> s
    return x


def interval(words: list, pos: int, mx: int) -> tuple[int, int]:
    """sb_rng_interval (sb_rng.c:45-54) on the stream from pos: (value, next pos)."""
    if mx == 0:
        return 0, pos
    mask = smear(mx)
    while True:
        v = words[pos] & mask
        pos += 1
        if v <= mx:
            return v, pos


def sequential_pairs(words: list, pos: int, ncand, thr: int):
    """sb_conv_apply's cell loop: u <= p (as the 53-bit draw <= thr) and candidates."""
    pairs = []
    for j in range(len(ncand)):
        a, b = words[pos], words[pos + 1]
        pos += 2
        if (((a >> 5) << 26) | (b >> 6)) > thr or ncand[j] == 0:
            continue
        pick, pos = interval(words, pos, int(ncand[j]) - 1)
        pairs.append((j, pick))
    return pairs, pos


def window_pairs(words: list, pos: int, ncand, thr: int):
    """The plan kernel's window rounds."""
    n = len(ncand)
    pairs, j = [], 0
    full = (1 << 64) - 1
    while j < n:
        w0 = [words[pos + 2 * i] for i in range(W)]
        w1 = [words[pos + 2 * i + 1] for i in range(W)]
        w2 = [words[pos + 2 * i + 2] for i in range(W)]
        nc = [int(ncand[j + i]) if j + i < n else 0 for i in range(W)]
        P0 = sum(1 << i for i in range(W) if (((w0[i] >> 5) << 26) | (w1[i] >> 6)) <= thr)
        P1 = sum(1 << i for i in range(W) if (((w1[i] >> 5) << 26) | (w2[i] >> 6)) <= thr)
        HC = sum(1 << i for i in range(W) if nc[i] > 0)

        def wreg(q):
            return w1[q >> 1] if q & 1 else w0[q >> 1]

        c, drift, slow, smax = 0, 0, False, 0
        while True:
            tt, par = drift >> 1, drift & 1
            if c + tt >= W:
                break
            cand = ((P1 if par else P0) >> tt) & HC & ((full << c) & full)
            if cand == 0:
                c = W - tt
                break
            cc = (cand & -cand).bit_length() - 1
            mx = nc[cc] - 1
            q = 2 * (cc + tt) + par + 2
            pick = 0
            if mx:
                mask = smear(mx)
                while True:
                    if q >= 2 * W:
                        slow = True
                        break
                    v = wreg(q) & mask
                    q += 1
                    if v <= mx:
                        pick = v
                        break
            if slow:
                pos += q
                j += cc
                smax = mx
                break
            pairs.append((j + cc, pick))
            drift = q - 2 * (cc + 1)
            c = cc + 1
        if slow:
            pick, pos = interval(words, pos, smax)
            pairs.append((j, pick))
            j += 1
            continue
        ce = min(c, n - j)
        pos += 2 * ce + drift
        j += ce
    return pairs, pos


def test_window_rounds_equal_sequential_draws():
    rng = np.random.default_rng(20261202)
    for trial in range(200):
        n = int(rng.integers(1, 700))
        p = float(rng.choice([0.05, 0.1, 0.3, 0.6, 0.95, 1.0]))
        thr = (1 << 53) if p >= 1 else int(np.floor(p * 2.0 ** 53))
        ncand = rng.integers(0, 25, size=n)
        ncand[rng.random(n) < 0.1] = 0
        ncand[rng.random(n) < 0.1] = 1
        words = [int(x) for x in rng.integers(0, 2 ** 32, size=6 * n + 1000, dtype=np.uint64)]
        start = int(rng.integers(0, 50))
        assert window_pairs(words, start, ncand, thr) == sequential_pairs(words, start, ncand, thr), (trial, n, p)


def test_composed_moves_equal_shuffled_swaps():
    rng = np.random.default_rng(7)
    for trial in range(200):
        n = int(rng.integers(2, 300))
        m = int(rng.integers(0, n + 1))
        left = rng.integers(0, n, size=m).tolist()
        right = rng.integers(0, n, size=m).tolist()
        words = [int(x) for x in rng.integers(0, 2 ** 32, size=8 * m + 64, dtype=np.uint64)]
        T = rng.normal(size=n)
        # the reference: Fisher-Yates over the pairs from the top, then swaps in order
        L, R, pos = list(left), list(right), 0
        for t in range(m - 1, 0, -1):
            j2, pos = interval(words, pos, t)
            L[t], L[j2] = L[j2], L[t]
            R[t], R[j2] = R[j2], R[t]
        ref = T.copy()
        for a, b in zip(L, R):
            ref[a], ref[b] = ref[b], ref[a]
        # the plan kernel: pair t final once the shuffle passes it, composed into q
        pr = [a | (b << 16) for a, b in zip(left, right)]
        q = list(range(n))
        pos = 0

        def compose(y):
            a, b = y & 0xFFFF, y >> 16
            q[a], q[b] = q[b], q[a]

        for t in range(m - 1, 0, -1):
            j2, pos = interval(words, pos, t)
            x, y = pr[t], pr[j2]
            pr[j2] = x
            compose(y)
        if m > 0:
            compose(pr[0])
        got = T.copy()
        moves = [(q[i], i) for i in range(n) if q[i] != i]
        vals = [T[src] for _, src in moves]
        for (dst, _), v in zip(moves, vals):
            got[dst] = v
        assert np.array_equal(got, ref), trial
