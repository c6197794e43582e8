"""The Jacobi eigensolver's sweep order (csrc/oa_eig.hip), replayed on the CPU: 64 quads hold
column pairs (a, b); within level l (h = 64 >> l quads per block) quad i takes the b column of
quad (i + 1) mod h of its block after every step but the last, and between levels the first
h / 2 quads of a block trade their b column for the a column of quad i + h / 2.  Every sweep
must pair every two of the 128 columns exactly once (the Jacobi method's cyclic condition), in
127 steps of 64 disjoint pairs, and the column set must be preserved.  A plausible slip in the
index arithmetic (the wrong neighbour, a missing trade, a trade with the wrong quad) breaks
one of these, as the planted variants below show."""

N, Q = 128, 64


def sweeps(n_sweeps=3, neighbour=1, trade=True, partner_shift=None):
    a = list(range(Q))
    b = list(range(Q, N))
    out = []
    for _ in range(n_sweeps):
        steps = []
        for lev in range(7):
            h = Q >> lev
            for t in range(h):
                steps.append(list(zip(a, b)))
                if t + 1 < h:
                    b = [b[(g - (g % h)) + ((g % h + neighbour) % h)] for g in range(Q)]
            if lev < 6 and trade:
                hb = h // 2
                shift = hb if partner_shift is None else partner_shift
                slot = [b[g] if g % h < hb else a[g] for g in range(Q)]
                na, nb = list(a), list(b)
                for g in range(Q):
                    if g % h < hb:
                        nb[g] = slot[(g + shift) % Q]
                    else:
                        na[g] = slot[(g - shift) % Q]
                a, b = na, nb
        out.append(steps)
    return out


def covers_every_pair_once(steps):
    seen = set()
    for st in steps:
        cols = [c for p in st for c in p]
        if len(set(cols)) != N:
            return False
        for x, y in st:
            key = (min(x, y), max(x, y))
            if key in seen:
                return False
            seen.add(key)
    return len(seen) == N * (N - 1) // 2


def test_every_sweep_meets_every_pair_once():
    for steps in sweeps(4):
        assert len(steps) == 127
        assert all(len(st) == Q for st in steps)
        assert covers_every_pair_once(steps)


def test_planted_slips_break_the_order():
    assert not covers_every_pair_once(sweeps(1, neighbour=2)[0])      # the wrong neighbour
    assert not covers_every_pair_once(sweeps(1, trade=False)[0])      # no trade between levels
    assert not covers_every_pair_once(sweeps(1, partner_shift=1)[0])  # trade with the wrong quad


def test_pairs_of_a_sweep_differ_from_the_last():
    """Consecutive sweeps are not the same sequence of pairs (the partition moves), but each is
    complete; the kernel's convergence test is per sweep."""
    s = sweeps(2)
    assert [sorted(map(tuple, map(sorted, st))) for st in s[0]] != [sorted(map(tuple, map(sorted, st))) for st in s[1]]
