"""Host replay of the automatic streaming partition (pvlc_hip_paged_decode_streaming_partition).

The streaming decode kernel may lengthen the planned partition P0 on the device so its items spread evenly over
the compute units.  A wave keeps the block ids of its tiles one per lane (32 chunks of 2 tiles), so a 4-wave
workgroup covers at most 4096 tokens of one partition: a longer choice would read keys and values through wrapped
lane indices.  These tests pin the rule on the CPU, where the device kernel makes the same choice from the same
lengths: the bound, optimality over the candidates by brute force, and known answers.
"""

import numpy as np
import pytest

from __graft_entry__ import load_package

pvlc = load_package()


def candidates(p0):
    step = max(16, (p0 // 4) & ~15)
    return [p0 + c * step for c in range(5)]


def cost(lens, p, units):
    items = 2 * sum(-(-(int(t) + 1) // p) for t in lens)
    return -(-items // units) * p


@pytest.mark.parametrize("rows,num_seqs", [(200000, 8), (140000, 16), (131073, 4), (262144, 3)])
def test_planned_4096_is_never_lengthened(rows, num_seqs):
    """Contexts beyond 131072 rows plan 4096-token partitions; every candidate above it is skipped (on 256 units
    8 seqs at T=200000 would otherwise pick 7168 and 16 seqs at T=140000 6144)."""
    assert pvlc.decode_partition(num_seqs, rows) == 4096
    lens = np.full(num_seqs, rows - 1, np.int32)
    for units in (1, 80, 256, 304):
        assert pvlc.decode_streaming_partition(lens, rows, units) == 4096


def test_lengthening_stops_at_the_workgroup_span():
    """P0 = 2048 (contexts in (65536, 131072]): candidates 2560, 3072, 3584, 4096 stay admissible."""
    rng = np.random.default_rng(7)
    seen = set()
    for trial in range(200):
        n = int(rng.integers(1, 40))
        lens = rng.integers(60000, 131072, n).astype(np.int32)
        max_context = int(lens.max()) + 1
        p0 = pvlc.decode_partition(n, max_context)
        units = int(rng.choice([64, 128, 256]))
        got = pvlc.decode_streaming_partition(lens, max_context, units)
        cands = [p for p in candidates(p0) if p <= 4096]
        assert got in cands and got <= 4096
        best = min(cost(lens, p, units) for p in cands)
        assert cost(lens, got, units) == best
        assert got == next(p for p in cands if cost(lens, p, units) == best)  # first on ties
        seen.add((p0, got))
    assert any(p0 == 2048 and got > 2048 for p0, got in seen)


def test_known_answers():
    # 15 x 8192 + 8300 rows at P0 = 512: 514 items (3 per unit on 256 units), 416 at 640 (2 per unit)
    lens = np.array([8191] * 15 + [8299], np.int32)
    assert pvlc.decode_streaming_partition(lens, 8300, 256) == 640
    # 4 sequences near 68000 rows plan 2048 (272 items, 2 rounds on 256 units); 2560 needs one round
    lens = np.array([67999, 66999, 67499, 65999], np.int32)
    assert pvlc.decode_partition(4, 68000) == 2048
    assert pvlc.decode_streaming_partition(lens, 68000, 256) == 2560
    # few items: one round at every candidate, so the planned partition stays
    p0 = pvlc.decode_partition(2, 3001)
    assert pvlc.decode_streaming_partition(np.array([3000, 100], np.int32), 3001, 256) == p0


def test_lengths_outside_the_context_are_not_counted():
    lens = np.array([8191] * 15 + [8299, -5, 9000], np.int32)
    assert pvlc.decode_streaming_partition(lens, 8300, 256) == 640
    assert pvlc.decode_streaming_partition(np.array([], np.int32), 8300, 256) == 0
