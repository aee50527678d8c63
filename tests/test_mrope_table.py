"""pvlc_hip_mrope_table_f32: the section selection of decoder_mrope_f32 / decoder_prefill_mrope_f32 (pvlc-wgsl
lib.rs:1185-1234, 1334-1380) on raw [3][capacity][128] tables, checked against the same selection written out
with numpy indexing, and its rejections (zero or mis-summed sections, non-finite values, rows whose halves differ,
which the one-cos-per-pair device tables cannot represent)."""

import numpy as np
import pytest

from pvlc_testlib import pvlc


def raw_tables(capacity, seed):
    rng = np.random.default_rng(seed)
    half_c = rng.standard_normal((3, capacity, 64)).astype(np.float32)
    half_s = rng.standard_normal((3, capacity, 64)).astype(np.float32)
    return np.concatenate([half_c, half_c], axis=2), np.concatenate([half_s, half_s], axis=2)


@pytest.mark.parametrize("sections", [(16, 24, 24), (8, 28, 28), (1, 1, 62), (62, 1, 1)])
def test_section_selection_matches_numpy_indexing(sections):
    capacity = 37
    rc, rs = raw_tables(capacity, sum(sections))
    cos, sin = pvlc.mrope_table(rc, rs, capacity, sections)
    axis = np.repeat([0, 1, 2], sections)
    f = np.arange(64)
    for slot in range(capacity):
        np.testing.assert_array_equal(cos[slot], rc[axis, slot, f])
        np.testing.assert_array_equal(sin[slot], rs[axis, slot, f])


def test_equal_axes_reduce_to_the_neox_table():
    capacity = 50
    cos, sin = pvlc.rope_table(500000.0, capacity)
    full_c = np.concatenate([cos, cos], axis=1)
    full_s = np.concatenate([sin, sin], axis=1)
    mc, ms = pvlc.mrope_table(np.stack([full_c] * 3), np.stack([full_s] * 3), capacity)
    np.testing.assert_array_equal(mc, cos)
    np.testing.assert_array_equal(ms, sin)


def test_rejections():
    capacity = 4
    rc, rs = raw_tables(capacity, 3)
    cases = [((rc, rs, capacity, (0, 32, 32)), "ZeroDimension"),
             ((rc, rs, capacity, (16, 24, 25)), "InvalidRotaryDimension"),
             ((rc, rs, 0, (16, 24, 24)), "LengthMismatch")]
    bad_half = rc.copy()
    bad_half[1, 2, 70] += 1.0
    cases.append(((bad_half, rs, capacity, (16, 24, 24)), "InvalidRotaryDimension"))
    nan = rs.copy()
    nan[2, 3, 5] = np.nan
    cases.append(((rc, nan, capacity, (16, 24, 24)), "NonFiniteInput"))
    for args, want in cases:
        with pytest.raises(pvlc.PvlcHipError) as e:
            pvlc.mrope_table(*args)
        assert e.value.invocation_code == want, (want, str(e.value))
