"""Plan contract of the decoder GEMV (GemvTiledDescriptor::plan, runtime-core lib.rs:753-785), restated
from crates/pvlc-runtime-core/tests/gemv_tiled_plan_contract.rs, and the device entry point's admission
(validated before any GPU effect)."""

import pytest

from pvlc_testlib import pvlc

ADMITTED = (1024, 2048, 3072)


def code(e):
    return e.code, e.invocation_code


def test_plan_pins_the_exact_vec4_tiled_lattice():
    plan = pvlc.plan_gemv_tiled(2048, 1024)
    assert (plan["tile_rows"], plan["threads_per_row"], plan["vector_width"]) == (8, 32, 4)
    assert (plan["shared_capacity"], plan["workgroup_storage_bytes"]) == (3072, 13312)
    assert plan["dispatch"] == [256, 1, 1] and plan["workgroup_size"] == [256, 1, 1]
    assert plan["uniform_words"] == [2048, 1024, 0, 0]
    assert plan["output_elements"] == 2048 and plan["output_bytes"] == 2048 * 4


@pytest.mark.parametrize("columns,rows,workgroups", [(1024, 256, 32), (1024, 2048, 256), (1024, 3072, 384),
                                                     (1024, 103_424, 12_928), (2048, 1024, 128), (3072, 1024, 128)])
def test_every_real_decoder_width_has_the_same_tiling_authority(columns, rows, workgroups):
    plan = pvlc.plan_gemv_tiled(rows, columns)
    assert plan["dispatch"] == [workgroups, 1, 1]
    assert plan["uniform_words"] == [rows, columns, 0, 0]
    assert plan["output_elements"] == rows and plan["output_bytes"] == rows * 4


def test_dispatch_is_the_ceil_of_rows_over_eight():
    for rows, wgs in [(1, 1), (7, 1), (8, 1), (9, 2), (256, 32), (1024, 128), (2048, 256), (3072, 384),
                      (103_424, 12_928)]:
        for columns in ADMITTED:
            plan = pvlc.plan_gemv_tiled(rows, columns)
            assert plan["dispatch"] == [wgs, 1, 1]
            assert plan["uniform_words"] == [rows, columns, 0, 0]


def test_descriptor_rejects_zero_rows_and_non_decoder_widths():
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.plan_gemv_tiled(0, 1024)
    assert code(e.value) == ("InvalidInvocation", "InvalidDecoderGeometry")
    for columns in (0, 4, 512, 1020, 1028, 4096):
        with pytest.raises(pvlc.PvlcHipError) as e:
            pvlc.plan_gemv_tiled(2048, columns)
        assert code(e.value) == ("InvalidInvocation", "InvalidDecoderGeometry")


def test_descriptor_enforces_the_dispatch_limit():
    maximum = 8 * 65_535
    assert pvlc.plan_gemv_tiled(maximum, 1024)["dispatch"] == [65_535, 1, 1]
    for rows in (maximum + 1, 2**32 - 1):
        with pytest.raises(pvlc.PvlcHipError) as e:
            pvlc.plan_gemv_tiled(rows, 1024)
        assert code(e.value) == ("InvalidInvocation", "InvalidDecoderGeometry")


def test_device_gemv_validates_before_touching_the_gpu():
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.gemv_f16(1, 1, 1, 2048, 4096)
    assert code(e.value) == ("InvalidInvocation", "InvalidDecoderGeometry")
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.gemv_f16(None, 1, 1, 2048, 1024)
    assert code(e.value) == ("InvalidInvocation", "LengthMismatch")


def test_dot_bound_of_the_gemv_parity_test_catches_planted_mistakes():
    """The bound the GPU parity test holds the kernel to (depth columns/64 + 6) accepts an f32 sum in the
    kernel's order and rejects an oracle with a dropped column, a shifted row or a transposed stride."""
    import numpy as np

    import oracle as O
    from pvlc_testlib import dot_error_ratio, widen
    rows, columns = 32, 1024
    wf = widen(O.normal_f16(77, rows * columns, 0.05)).reshape(rows, columns)
    x = O.normal_f32(78, columns)
    # the kernel's order in f32: lane l accumulates its 16 columns, then a 6-level xor tree
    lanes = np.zeros((rows, 64), np.float32)
    for c in range(columns // 512):
        for j in range(8):
            col = (c * 64 + np.arange(64)) * 8 + j
            lanes = (lanes + (wf[:, col] * x[col]).astype(np.float32)).astype(np.float32)
    for o in (32, 16, 8, 4, 2, 1):
        lanes = (lanes + lanes[:, np.arange(64) ^ o]).astype(np.float32)
    assert dot_error_ratio(lanes[:, 0], wf, x, columns // 64 + 6 + columns // 64) <= 1.0
    zero = np.zeros(rows, np.float32)
    good = O.linear_f32(x, 1, columns, wf, zero, rows)
    assert dot_error_ratio(good, wf, x, columns) <= 1.0
    dropped = wf.copy()
    dropped[:, 513] = 0
    assert dot_error_ratio(O.linear_f32(x, 1, columns, dropped, zero, rows), wf, x, columns // 64 + 6) > 10
    shifted = np.roll(wf, 1, axis=0)
    assert dot_error_ratio(O.linear_f32(x, 1, columns, shifted, zero, rows), wf, x, columns // 64 + 6) > 10
    square = wf[:, :rows].T.copy()
    assert dot_error_ratio(O.linear_f32(x[:rows], 1, rows, square, zero, rows), wf[:, :rows], x[:rows], 6) > 10


def test_top1_workspace_is_a_fixed_small_block():
    assert pvlc.top1_workspace_bytes() == 64 * 256


def test_device_top1_entry_points_validate_before_touching_the_gpu():
    nbytes = pvlc.top1_workspace_bytes()
    aligned = 1 << 20  # a fake 256-byte aligned device address: never dereferenced on these paths
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.logits_top1_f32(aligned, 0, aligned, aligned, nbytes)
    assert code(e.value) == ("InvalidInvocation", "LengthMismatch")
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.logits_top1_f32(aligned, 2**31 + 1, aligned, aligned, nbytes)
    assert code(e.value) == ("InvalidInvocation", "LengthMismatch")
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.logits_top1_f32(aligned, 100, aligned, aligned, nbytes - 8)
    assert code(e.value) == ("InvalidInvocation", "LengthMismatch")
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.logits_top1_f32(aligned, 100, aligned, aligned + 8, nbytes)
    assert code(e.value) == ("InvalidInvocation", "LengthMismatch")
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.logits_top1_f32(aligned, 100, None, aligned, nbytes)
    assert code(e.value) == ("InvalidInvocation", "LengthMismatch")
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.lm_head_top1_f16(aligned, aligned, None, 103_424, 4096, aligned, aligned, nbytes)
    assert code(e.value) == ("InvalidInvocation", "InvalidDecoderGeometry")
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.lm_head_top1_f16(aligned, aligned, None, 0, 1024, aligned, aligned, nbytes)
    assert code(e.value) == ("InvalidInvocation", "InvalidDecoderGeometry")
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.lm_head_top1_f16(aligned, aligned, None, 103_424, 1024, aligned, None, nbytes)
    assert code(e.value) == ("InvalidInvocation", "LengthMismatch")


def test_grouped_gemv_rejects_bad_groups_before_any_launch():
    """pvlc_hip_gemv_group_f16 admission (no device work): 1..4 members, no NULL pointer, no empty member, total
    rows and width admitted as one pvlc_hip_gemv_f16."""
    with pytest.raises(pvlc.PvlcHipError):
        pvlc.gemv_group_f16([], 1, 1024)
    with pytest.raises(pvlc.PvlcHipError):
        pvlc.gemv_group_f16([(1, 1, 8)] * 5, 1, 1024)
    with pytest.raises(pvlc.PvlcHipError):
        pvlc.gemv_group_f16([(1, 1, 8), (None, 1, 8)], 1, 1024)
    with pytest.raises(pvlc.PvlcHipError):
        pvlc.gemv_group_f16([(1, 1, 8), (1, 1, 0)], 1, 1024)
    with pytest.raises(pvlc.PvlcHipError):
        pvlc.gemv_group_f16([(1, 1, 8)], 1, 4096)
    with pytest.raises(pvlc.PvlcHipError):
        pvlc.gemv_group_f16([(1, 1, 8)], None, 1024)
