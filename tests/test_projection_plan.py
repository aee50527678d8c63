"""Plan contract of the prefill projection with fp16 weights (VisionPatchProjectionBytesDescriptor,
runtime-core lib.rs:1733-1913), restated from crates/pvlc-runtime-core/tests/
vision_patch_projection_bytes_contract.rs, and the device entry point's admission (checked before any GPU
effect)."""

import struct

import pytest

from pvlc_testlib import pvlc


def f32_bytes(values):
    return b"".join(struct.pack("<f", v) for v in values)


def f16_bytes(bits):
    return b"".join(struct.pack("<H", b) for b in bits)


def code(fn, *args):
    with pytest.raises(pvlc.ProjectionPlanError) as e:
        fn(*args)
    return e.value.code


def test_realistic_plan_selects_the_storage_specific_kernel_and_exact_buffers():
    f32 = pvlc.plan_projection(1276, 588, 1152, "f32")
    assert f32.kernel == "vision_patch_projection_f32"
    assert (f32.input_bytes, f32.weight_bytes, f32.bias_bytes, f32.output_bytes) == (
        1276 * 588 * 4, 1152 * 588 * 4, 1152 * 4, 1276 * 1152 * 4)
    assert f32.dispatch == [36, 40, 1] and not f32.requires_shader_f16()
    f16 = pvlc.plan_projection(1276, 588, 1152, "f16")
    assert f16.kernel == "linear_projection_f16_weights"
    assert f16.input_bytes == f32.input_bytes and f16.weight_bytes == f32.weight_bytes // 2
    assert f16.bias_bytes == f32.bias_bytes and f16.output_bytes == f32.output_bytes
    assert f16.dispatch == [36, 40, 1] and f16.requires_shader_f16()


def test_production_token_count_rounds_to_fifty_eight_row_tiles():
    for storage in ("f32", "f16"):
        assert pvlc.plan_projection(1836, 1152, 4304, storage).dispatch == [135, 58, 1]


def test_exact_finite_operands_and_capabilities_are_admitted():
    f32 = pvlc.plan_projection(2, 3, 4, "f32")
    f32.validate_capabilities(False, 65535)
    f32.validate_operands(f32_bytes([1.0, -2.0, 3.0, 4.0, 5.0, -6.0]),
                          f32_bytes([0.1, 0.2, 0.3, -0.4, 0.5, 0.6, 0.7, -0.8, 0.9, 1.0, 1.1, -1.2]),
                          f32_bytes([0.25, -0.5, 0.75, 1.0]))
    f16 = pvlc.plan_projection(2, 4, 4, "f16")
    f16.validate_capabilities(True, 65535)
    f16.validate_operands(f32_bytes([1.0, -2.0, 3.0, 4.0, 5.0, -6.0, 7.0, -8.0]),
                          f16_bytes([0x2e66, 0x3266, 0x34cd, 0xb666, 0x3800, 0x38cd, 0x399a, 0xba66, 0x3b33, 0x3c00,
                                     0x3c66, 0xbccd, 0x3d00, 0x3d33, 0x3d66, 0x3d9a]),
                          f32_bytes([0.25, -0.5, 0.75, 1.0]))


def test_every_operand_requires_exact_byte_length_in_both_storage_modes():
    bias = f32_bytes([0.0] * 4)
    for plan, inp, w in ((pvlc.plan_projection(2, 3, 4, "f32"), f32_bytes([1.0, -2.0, 3.0, 4.0, 5.0, -6.0]),
                          f32_bytes([0.5] * 12)),
                         (pvlc.plan_projection(2, 4, 4, "f16"), f32_bytes([1.0, -2.0, 3.0, 4.0, 5.0, -6.0, 7.0, -8.0]),
                          f16_bytes([0x3800] * 16))):
        exact = [inp, w, bias]
        for operand in range(3):
            for delta in (-1, 1):
                changed = list(exact)
                changed[operand] = changed[operand][:-1] if delta < 0 else changed[operand] + b"\0"
                assert code(plan.validate_operands, *changed) == "LengthMismatch"


def test_every_non_finite_operand_is_rejected_before_gpu_execution():
    plan = pvlc.plan_projection(2, 3, 4, "f32")
    inp, w, bias = f32_bytes([1.0, -2.0, 3.0, 4.0, 5.0, -6.0]), f32_bytes([0.5] * 12), f32_bytes([0.0] * 4)
    for bad in (float("nan"), float("inf"), float("-inf")):
        for operand in range(3):
            changed = [bytearray(inp), bytearray(w), bytearray(bias)]
            changed[operand][:4] = struct.pack("<f", bad)
            assert code(plan.validate_operands, *changed) == "NonFinite"
    f16 = pvlc.plan_projection(2, 4, 4, "f16")
    packed = f32_bytes([1.0, -2.0, 3.0, 4.0, 5.0, -6.0, 7.0, -8.0])
    for bits in (0x7c00, 0xfc00, 0x7e00):
        weights = bytearray(f16_bytes([0x3c00] * 16))
        weights[:2] = struct.pack("<H", bits)
        assert code(f16.validate_operands, packed, weights, bias) == "NonFinite"


def test_fp16_projection_rejects_widths_that_cannot_use_packed_vec4_io():
    for iw, ow in ((3, 4), (4, 5), (7, 9)):
        assert code(pvlc.plan_projection, 2, iw, ow, "f16") == "InvalidGeometry"
    pvlc.plan_projection(2, 3, 5, "f32")  # the f32 path keeps arbitrary widths


def test_zero_and_overflowing_geometry_have_stable_error_classes():
    for pc, iw, ow in ((0, 588, 1152), (1276, 0, 1152), (1276, 588, 0)):
        assert code(pvlc.plan_projection, pc, iw, ow, "f32") == "InvalidGeometry"
    m = 2**32 - 1
    assert code(pvlc.plan_projection, m, m, m, "f32") == "Overflow"


def test_dispatch_rounding_and_capabilities_fail_closed():
    assert pvlc.plan_projection(9, 3, 17, "f32").dispatch == [1, 1, 1]
    rounded_f16 = pvlc.plan_projection(9, 4, 36, "f16")
    assert rounded_f16.dispatch == [2, 1, 1]
    exact = pvlc.plan_projection(1, 1, 65535 * 32, "f32")
    exact.validate_capabilities(False, 65535)
    over = pvlc.plan_projection(1, 1, 65535 * 32 + 1, "f32")
    assert over.dispatch[0] == 65536
    assert code(over.validate_capabilities, False, 65535) == "DispatchLimitExceeded"
    exact16 = pvlc.plan_projection(1, 4, 65535 * 32, "f16")
    assert exact16.dispatch == [65535, 1, 1]
    exact16.validate_capabilities(True, 65535)
    over16 = pvlc.plan_projection(1, 4, 65535 * 32 + 4, "f16")
    assert over16.dispatch == [65536, 1, 1]
    assert code(over16.validate_capabilities, True, 65535) == "DispatchLimitExceeded"
    assert code(rounded_f16.validate_capabilities, False, 65535) == "MissingShaderF16"


def test_device_projection_validates_before_touching_the_gpu():
    fake = 1 << 20  # never dereferenced: validation fails first
    ws = pvlc.linear_projection_workspace_bytes(64, 1024)
    assert ws >= 64 * 1024 * 4 + 64 * 4
    cases = [
        ((fake, fake, fake, fake, 64, 1000, 256, fake, ws), "InvalidDecoderGeometry"),  # width not a multiple of 32
        ((fake, fake, fake, fake, 64, 1024, 6, fake, ws), "InvalidDecoderGeometry"),    # not a multiple of 4
        ((fake, fake, fake, fake, 0, 1024, 256, fake, ws), "InvalidDecoderGeometry"),
        ((fake, fake, fake, fake, 64 * 128, 1024, 2**32 - 4, fake, ws), "InvalidDecoderGeometry"),  # tiles > 2^24
        ((fake, fake, fake, fake, 64, 1024, 256, fake, ws - 4), "LengthMismatch"),
        ((fake, fake, fake, fake, 64, 1024, 256, fake + 16, ws), "LengthMismatch"),    # workspace alignment
        ((fake + 8, fake, fake, fake, 64, 1024, 256, fake, ws), "LengthMismatch"),     # input alignment
        ((None, fake, fake, fake, 64, 1024, 256, fake, ws), "LengthMismatch"),
    ]
    for args, want in cases:
        with pytest.raises(pvlc.PvlcHipError) as e:
            pvlc.linear_projection_f16(*args)
        assert e.value.invocation_code == want, args
