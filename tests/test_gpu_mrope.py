"""Multimodal RoPE on the device paths (decoder_mrope_f32 and decoder_prefill_mrope_f32, pvlc-wgsl
lib.rs:1185-1234, 1334-1380): raw cos/sin tables [3][capacity][128] built from distinct temporal, height and
width positions (an image grid inside a text prompt) go through pvlc_hip_mrope_table_f32, and the prefill and
decode entry points rotate with the selected rows.  The keys written to the cache equal the oracle's
apply_multimodal_rope_f32 (cpu-ref lib.rs:562-672) rounded to fp16 bit for bit; attention matches the oracle
over the rotated inputs within the north-star tolerance."""

import numpy as np
import pytest

import oracle as O
from pvlc_testlib import (W, check_close, f16_bits, from_dev, gather_rows, log, pvlc, scatter_rows, to_dev,
                          to_dev_f32, to_dev_i32, widen)

pytestmark = pytest.mark.gpu
SECTIONS = (16, 24, 24)


def thw_positions(tokens, text_before=10, grid=(6, 8)):
    """(t, h, w) of every token: text tokens share one index on all axes; the image grid keeps t and walks h, w;
    text after the image resumes past the largest index used."""
    pos = np.zeros((3, tokens), np.int64)
    gh, gw = grid
    for i in range(min(tokens, text_before)):
        pos[:, i] = i
    img = range(text_before, min(tokens, text_before + gh * gw))
    for j, i in enumerate(img):
        pos[:, i] = (text_before, text_before + j // gw, text_before + j % gw)
    nxt = text_before + max(gh, gw)
    for i in range(text_before + gh * gw, tokens):
        pos[:, i] = nxt
        nxt += 1
    return pos


def raw_tables(pos, base=500000.0):
    inv = (base ** (-(2.0 * np.arange(64) / 128.0))).astype(np.float32)
    ang = pos[:, :, None].astype(np.float32) * inv[None, None, :]
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    return np.concatenate([c, c], axis=2), np.concatenate([s, s], axis=2)


def test_prefill_with_image_grid_positions():
    import torch
    n = 90
    log(f"case: M-RoPE prefill N={n} (text, 6x8 image grid, text)")
    pos = thw_positions(n)
    assert len({tuple(p) for p in pos.T}) == n and np.any(pos[1] != pos[2])
    raw_c, raw_s = raw_tables(pos)
    cos, sin = pvlc.mrope_table(raw_c, raw_s, n, SECTIONS)
    q, k, v = f16_bits(70, n * 2048, 0.5), f16_bits(71, n * W, 0.5), f16_bits(72, n * W, 0.5)
    nb = (n + 15) // 16
    d_k = torch.zeros(nb * 16 * W, dtype=torch.int16, device="cuda")
    d_v = torch.zeros_like(d_k)
    out = torch.zeros(n * 2048, dtype=torch.int16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    keep = [to_dev(q), to_dev(k), to_dev(v), to_dev_f32(cos), to_dev_f32(sin)]
    pvlc.paged_prefill_f16(tokens=n, num_blocks=nb, key_cache=d_k, value_cache=d_v, query=keep[0], key=keep[1],
                           value=keep[2], out=out, rope_cos=keep[3], rope_sin=keep[4], rope_rows=n, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    rq, rk = O.mrope_f32(widen(q), widen(k), n, 16, 2, 128, raw_c, raw_s, SECTIONS)
    kr = O.f32_to_f16(rk)
    gk, gv = gather_rows(from_dev(d_k), from_dev(d_v), n, np.arange(nb))
    np.testing.assert_array_equal(gk, kr)
    np.testing.assert_array_equal(gv, v)
    got = widen(from_dev(out)).reshape(n, 2048)
    for i in (0, 9, 10, 11, 33, 57, 58, 89):
        want = O.decode_gqa_f32(rq[i * 2048:(i + 1) * 2048], widen(kr)[:(i + 1) * W], widen(v)[:(i + 1) * W], i + 1,
                                16, 2, 128)
        check_close(got[i], want, f"mrope prefill row {i}")


@pytest.mark.parametrize("thw", [(12, 3, 5), (40, 40, 40)])
def test_decode_appends_a_token_with_its_own_axes(thw):
    """One decode step whose appended token has (t, h, w) positions (an image token, or a text token with equal
    axes): the table row of its slot carries the selected axes; query and key rotate with it."""
    import torch
    prefix, capacity = 40, 64
    log(f"case: M-RoPE decode, appended token at slot {prefix} with (t, h, w) = {thw}")
    pos = np.zeros((3, capacity), np.int64)
    pos[:, :] = np.arange(capacity)
    pos[:, prefix] = thw
    raw_c, raw_s = raw_tables(pos)
    cos, sin = pvlc.mrope_table(raw_c, raw_s, capacity, SECTIONS)
    nb_per = capacity // 16
    rows_k, rows_v = f16_bits(80, prefix * W, 0.5), f16_bits(81, prefix * W, 0.5)
    kp = np.zeros(nb_per * 16 * W, np.uint16)
    vp = np.zeros_like(kp)
    scatter_rows(kp, vp, rows_k, rows_v, prefix, np.arange(nb_per))
    q, nk, nv = f16_bits(82, 2048, 0.5), f16_bits(83, W, 0.5), f16_bits(84, W, 0.5)
    d_k, d_v = to_dev(kp), to_dev(vp)
    d_out = torch.zeros(2048, dtype=torch.int16, device="cuda")
    wsb = pvlc.decode_workspace_bytes(1, capacity, 0)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    pvlc.workspace_init(ws, wsb)
    keep = [to_dev(q), to_dev(nk), to_dev(nv), to_dev_f32(cos), to_dev_f32(sin), to_dev_i32(np.array([prefix]))]
    args = pvlc.paged_decode_args(num_seqs=1, num_blocks=nb_per, max_blocks_per_seq=nb_per, key_cache=d_k,
                                  value_cache=d_v, query=keep[0], new_key=keep[1], new_value=keep[2], out=d_out,
                                  workspace=ws, workspace_bytes=wsb, max_context=capacity, uniform_cache_len=prefix,
                                  rope_cos=keep[3], rope_sin=keep[4], rope_rows=capacity, positions=keep[5],
                                  rotate_query=True)
    pvlc.paged_decode_f16(args)
    torch.cuda.synchronize()
    assert pvlc.workspace_error(ws, wsb) == 0
    # oracle: M-RoPE of the appended token's query and key with the raw tables of its slot
    slot_c = np.ascontiguousarray(raw_c[:, prefix:prefix + 1, :])
    slot_s = np.ascontiguousarray(raw_s[:, prefix:prefix + 1, :])
    rq, rk = O.mrope_f32(widen(q), widen(nk), 1, 16, 2, 128, slot_c, slot_s, SECTIONS)
    gk, gv = gather_rows(from_dev(d_k), from_dev(d_v), prefix + 1, np.arange(nb_per))
    np.testing.assert_array_equal(gk, np.concatenate([rows_k, O.f32_to_f16(rk)]))
    np.testing.assert_array_equal(gv, np.concatenate([rows_v, nv]))
    want = O.decode_gqa_f32(rq, widen(gk), widen(gv), prefix + 1, 16, 2, 128)
    check_close(widen(from_dev(d_out)), want, f"mrope decode {thw}")


def test_f32_operand_prefill_with_image_grid_positions():
    """pvlc_hip_paged_prefill_f32io with M-RoPE tables and f32 inputs fp16 cannot hold: the keys in the cache are
    apply_multimodal_rope_f32 of the f32 keys rounded once, bit for bit; the values are the f32 values rounded;
    the f32 output is within tolerance of the oracle over the query rotated and rounded the same way."""
    import torch
    n = 90
    log(f"case: M-RoPE prefill with f32 operands N={n}")
    pos = thw_positions(n)
    raw_c, raw_s = raw_tables(pos)
    cos, sin = pvlc.mrope_table(raw_c, raw_s, n, SECTIONS)
    rng = np.random.default_rng(73)
    q = (rng.standard_normal(n * 2048) * 0.5).astype(np.float32)
    k = (rng.standard_normal(n * W) * 0.5).astype(np.float32)
    v = (rng.standard_normal(n * W) * 0.5).astype(np.float32)
    nb = (n + 15) // 16
    d_k = torch.zeros(nb * 16 * W, dtype=torch.int16, device="cuda")
    d_v = torch.zeros_like(d_k)
    out = torch.full((n * 2048,), float("nan"), dtype=torch.float32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    keep = [to_dev_f32(q), to_dev_f32(k), to_dev_f32(v), to_dev_f32(cos), to_dev_f32(sin)]
    pvlc.paged_prefill_f32io(tokens=n, num_blocks=nb, key_cache=d_k, value_cache=d_v, query=keep[0], key=keep[1],
                             value=keep[2], out=out, rope_cos=keep[3], rope_sin=keep[4], rope_rows=n, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    rq, rk = O.mrope_f32(q, k, n, 16, 2, 128, raw_c, raw_s, SECTIONS)
    kr, vr, qr = O.f32_to_f16(rk), O.f32_to_f16(v), O.f32_to_f16(rq)
    gk, gv = gather_rows(from_dev(d_k), from_dev(d_v), n, np.arange(nb))
    np.testing.assert_array_equal(gk, kr)
    np.testing.assert_array_equal(gv, vr)
    got = out.cpu().numpy().reshape(n, 2048)
    for i in (0, 9, 10, 33, 57, 89):
        want = O.decode_gqa_f32(widen(qr)[i * 2048:(i + 1) * 2048], widen(kr)[:(i + 1) * W], widen(vr)[:(i + 1) * W],
                                i + 1, 16, 2, 128)
        check_close(got[i], want, f"mrope f32-operand prefill row {i}")


def test_f32_operand_decode_appends_a_token_with_its_own_axes():
    """pvlc_hip_paged_decode_f32io with an appended image token's (t, h, w) positions and f32 query, key and value:
    the appended key is apply_multimodal_rope_f32 of the f32 key at its slot's axes rounded once."""
    import torch
    prefix, capacity, thw = 40, 64, (12, 3, 5)
    log(f"case: M-RoPE decode with f32 operands, appended token at slot {prefix} with (t, h, w) = {thw}")
    pos = np.zeros((3, capacity), np.int64)
    pos[:, :] = np.arange(capacity)
    pos[:, prefix] = thw
    raw_c, raw_s = raw_tables(pos)
    cos, sin = pvlc.mrope_table(raw_c, raw_s, capacity, SECTIONS)
    nb_per = capacity // 16
    rows_k, rows_v = f16_bits(85, prefix * W, 0.5), f16_bits(86, prefix * W, 0.5)
    kp = np.zeros(nb_per * 16 * W, np.uint16)
    vp = np.zeros_like(kp)
    scatter_rows(kp, vp, rows_k, rows_v, prefix, np.arange(nb_per))
    rng = np.random.default_rng(87)
    q = (rng.standard_normal(2048) * 0.5).astype(np.float32)
    nk = (rng.standard_normal(W) * 0.5).astype(np.float32)
    nv = (rng.standard_normal(W) * 0.5).astype(np.float32)
    d_k, d_v = to_dev(kp), to_dev(vp)
    d_out = torch.full((2048,), float("nan"), dtype=torch.float32, device="cuda")
    wsb = pvlc.decode_workspace_bytes(1, capacity, 0)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    pvlc.workspace_init(ws, wsb)
    keep = [to_dev_f32(q), to_dev_f32(nk), to_dev_f32(nv), to_dev_f32(cos), to_dev_f32(sin),
            to_dev_i32(np.array([prefix]))]
    args = pvlc.paged_decode_args(num_seqs=1, num_blocks=nb_per, max_blocks_per_seq=nb_per, key_cache=d_k,
                                  value_cache=d_v, query=None, new_key=None, new_value=None, out=None,
                                  workspace=ws, workspace_bytes=wsb, max_context=capacity, uniform_cache_len=prefix,
                                  rope_cos=keep[3], rope_sin=keep[4], rope_rows=capacity, positions=keep[5],
                                  rotate_query=True)
    pvlc.paged_decode_f32io(args, keep[0], keep[1], keep[2], d_out)
    torch.cuda.synchronize()
    assert pvlc.workspace_error(ws, wsb) == 0
    slot_c = np.ascontiguousarray(raw_c[:, prefix:prefix + 1, :])
    slot_s = np.ascontiguousarray(raw_s[:, prefix:prefix + 1, :])
    rq, rk = O.mrope_f32(q, nk, 1, 16, 2, 128, slot_c, slot_s, SECTIONS)
    gk, gv = gather_rows(from_dev(d_k), from_dev(d_v), prefix + 1, np.arange(nb_per))
    np.testing.assert_array_equal(gk, np.concatenate([rows_k, O.f32_to_f16(rk)]))
    np.testing.assert_array_equal(gv, np.concatenate([rows_v, O.f32_to_f16(nv)]))
    want = O.decode_gqa_f32(widen(O.f32_to_f16(rq)), widen(gk), widen(gv), prefix + 1, 16, 2, 128)
    check_close(d_out.cpu().numpy(), want, "mrope f32-operand decode")
