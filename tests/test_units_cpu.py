"""The work-unit partition's index arithmetic (kvq_decode_amd/csrc/decode_common.h:
unit_lo, unit_of, for_unit_segments; decode.hip: merge_units_kernel), restated in Python
and checked for the invariants the kernels rely on, over many small batches including
empty sequences:
  * the units tile the concatenated chunks [0, N) exactly, none empty;
  * unit_of(x) is the unit whose range holds chunk x;
  * segment (u, b) writes row u + b < units + B, and no two segments share a row;
  * the merge's rows for sequence b, first..last from unit_of(P_b) and
    unit_of(P_b + n_b - 1), are exactly the rows its segments wrote.
"""
import numpy as np


def unit_lo(u, N, NU):
    return (u * N) // NU


def unit_of(x, N, NU):
    return ((x + 1) * NU + N - 1) // N - 1


def segments(lens, units):
    """(u, b, c_lo, c_hi) as for_unit_segments enumerates them, and (N, NU)."""
    n = [-(-length // 16) for length in lens]
    pref = np.concatenate([[0], np.cumsum(n)]).astype(int)
    N = int(pref[-1])
    NU = min(units, N)
    out = []
    for u in range(NU):
        lo, hi = unit_lo(u, N, NU), unit_lo(u + 1, N, NU)
        # the largest b with P_b <= lo (binary search in the kernel)
        b, top = 0, len(lens)
        while top - b > 1:
            mid = (b + top) // 2
            if pref[mid] <= lo:
                b = mid
            else:
                top = mid
        while b < len(lens) and pref[b] < hi:
            c_lo, c_hi = max(lo, pref[b]) - pref[b], min(hi, pref[b + 1]) - pref[b]
            if c_lo < c_hi:
                out.append((u, b, int(c_lo), int(c_hi)))
            b += 1
    return out, N, NU, pref


def test_unit_partition_invariants():
    rng = np.random.default_rng(0)
    cases = 0
    for _ in range(3000):
        B = int(rng.integers(1, 12))
        lens = rng.integers(0, 200, B)
        lens[rng.random(B) < 0.2] = 0  # empty sequences
        units = int(rng.integers(1, 40))
        segs, N, NU, pref = segments(lens, units)
        if N == 0:
            assert not segs
            continue
        cases += 1
        # the units tile [0, N), none empty
        bounds = [unit_lo(u, N, NU) for u in range(NU + 1)]
        assert bounds[0] == 0 and bounds[-1] == N
        assert all(bounds[u] < bounds[u + 1] for u in range(NU))
        # unit_of inverts unit_lo
        for x in range(N):
            u = unit_of(x, N, NU)
            assert bounds[u] <= x < bounds[u + 1]
        # every chunk of every sequence covered exactly once
        seen = np.zeros(N, int)
        for u, b, c_lo, c_hi in segs:
            seen[pref[b] + c_lo:pref[b] + c_hi] += 1
        assert np.all(seen == 1)
        # rows: u + b, below units + B, no collisions
        rows = [u + b for u, b, _, _ in segs]
        assert len(set(rows)) == len(rows)
        assert max(rows) < units + B
        # the merge finds exactly each sequence's rows
        for b in range(B):
            n_b = int(pref[b + 1] - pref[b])
            mine = sorted(u + bb for u, bb, _, _ in segs if bb == b)
            if n_b == 0:
                assert not mine
                continue
            first, last = unit_of(pref[b], N, NU), unit_of(pref[b] + n_b - 1, N, NU)
            assert mine == list(range(first + b, last + b + 1))
    assert cases > 2000


def test_unit_of_large_values_do_not_overflow_int64():
    # the host keeps a kv head's chunk count N below 2^31 (kvq_decode_units rejects larger
    # batch * chunks-per-sequence bounds), and NU <= N: (x + 1) * NU < 2^62
    N, NU = 2**31 - 1, 2**31 - 1
    NU = min(NU, N)
    assert N * NU < 2**62 and (N - 1) * N < 2**62  # unit_of's and unit_lo's products
    assert unit_of(N - 1, N, NU) == NU - 1
    assert unit_of(0, N, NU) == 0
