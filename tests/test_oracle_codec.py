"""Pins the oracle's C codec (oracle/codec.c) and checks the product codecs
against it bit for bit.

Known-answer vectors come from the reference's own tests:
  tests/unit/test_q4.py:19-67     nibble order, 129-element layout, -8 and
                                  tail rejection, zero groups, bad scales
  tests/unit/test_bf16.py:44-63 f32 -> bf16 round-to-nearest-even words
What those leave open (the choice of code for every value) is pinned by
brute force: each code must be the nearest grid point, ties to even.
"""

from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from oracle import codec as oc


def test_q4_nibble_order_known_answer():
    # tests/unit/test_q4.py:19-23
    packed = oc.q4_pack(np.array([-7, -1, 0, 1, 7], dtype=np.int8))
    assert packed == bytes((0xF9, 0x10, 0x07))
    assert oc.q4_unpack(packed, 5).tolist() == [-7, -1, 0, 1, 7]


def test_q4_group128_tail_and_error_bound():
    # tests/unit/test_q4.py:26-40
    src = np.linspace(-3.0, 3.0, 129, dtype=np.float32)
    packed, scales = oc.q4_quantize(src, 128)
    assert len(packed) == 65 and len(scales) == 8
    s = np.frombuffer(scales, dtype="<f4")
    restored = oc.q4_dequantize(packed, scales, (129,), 128)
    assert np.max(np.abs(restored[:128] - src[:128])) <= s[0] / 2 + 1e-6
    assert np.max(np.abs(restored[128:] - src[128:])) <= s[1] / 2 + 1e-6


def test_q4_rejects_reserved_code_and_tail_padding():
    # tests/unit/test_q4.py:43-47
    with pytest.raises(oc.CodecError, match="reserved"):
        oc.q4_unpack(bytes((0x08,)), 1)
    with pytest.raises(oc.CodecError, match="tail"):
        oc.q4_unpack(bytes((0x10,)), 1)
    with pytest.raises(oc.CodecError):
        oc.q4_pack(np.array([-8], dtype=np.int8))


def test_q4_zero_group_round_trips_with_unit_scale():
    # tests/unit/test_q4.py:50-55
    src = np.zeros((3, 43), dtype=np.float32)
    packed, scales = oc.q4_quantize(src)
    assert np.array_equal(oc.q4_dequantize(packed, scales, (3, 43)), src)
    assert np.frombuffer(scales, dtype="<f4").tolist() == [1.0, 1.0]


@pytest.mark.parametrize("scale", [0.0, -1.0, float("nan"), float("inf")])
def test_q4_rejects_invalid_scales(scale):
    # tests/unit/test_q4.py:58-67
    with pytest.raises(oc.CodecError, match="finite and positive"):
        oc.q4_dequantize(b"\x00", struct.pack("<f", scale), (2,), 128)


def test_bf16_round_to_nearest_even_known_answers():
    # tests/unit/test_bf16.py:44-63
    words = [0x3F808000, 0x3F818000, 0x7F800000, 0xFF800000, 0x7F800001, 0xFF800001]
    f = np.array(words, dtype=np.uint32).view(np.float32)
    assert oc.f32_to_bf16_bits(f).tolist() == [0x3F80, 0x3F82, 0x7F80, 0xFF80, 0x7FC0, 0xFFC0]


def _brute_force_codes(w: np.ndarray, group: int, qmax: int):
    """Nearest grid point per element by exhaustive search (ties to even code)."""
    n = w.size
    g = -(-n // group)
    padded = np.zeros(g * group, np.float32)
    padded[:n] = w
    absmax = np.abs(padded.reshape(g, group)).max(axis=1)
    scales = (absmax / np.float32(qmax)).astype(np.float32)
    scales[scales == 0] = 1.0
    grid = np.arange(-qmax, qmax + 1, dtype=np.float32)
    codes = np.empty(n, np.int8)
    for i in range(n):
        r = np.float32(w[i] / scales[i // group])  # the same float32 quotient
        d = np.abs(grid - r)
        best = np.flatnonzero(d == d.min())
        pick = best[0] if len(best) == 1 else best[np.argmin(np.abs(grid[best]) % 2)]
        codes[i] = int(grid[pick])
    return codes, scales


@pytest.mark.parametrize("qmax", [7, 127])
def test_codes_are_nearest_grid_points(qmax):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal(3 * 128 + 17) * 0.02).astype(np.float32)
    # plant exact half-way quotients to exercise ties
    w[5] = 0.0
    codes, scales = _brute_force_codes(w, 128, qmax)
    if qmax == 7:
        packed, sc = oc.q4_quantize(w, 128)
        got = oc.q4_unpack(packed, w.size)
    else:
        data, sc = oc.q8_quantize(w, 128)
        got = np.frombuffer(data, dtype=np.int8)
    assert np.array_equal(np.frombuffer(sc, "<f4"), scales)
    assert np.array_equal(got, codes)


def test_q4_tie_rounds_half_to_even():
    # absmax 7*s puts k + 0.5 quotients on exact ties: 0.5 -> 0, 1.5 -> 2, 2.5 -> 2
    s = np.float32(0.25)
    w = np.array([7 * s, 0.5 * s, 1.5 * s, 2.5 * s, -2.5 * s, -0.5 * s] + [0.0] * 122, dtype=np.float32)
    packed, sc = oc.q4_quantize(w, 128)
    assert np.frombuffer(sc, "<f4")[0] == s
    assert oc.q4_unpack(packed, 128)[:6].tolist() == [7, 0, 2, 2, -2, 0]


def test_q8_round_trip_and_absmax_code():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((4, 256)) * 0.02).astype(np.float32)
    data, sc = oc.q8_quantize(w)
    q = np.frombuffer(data, np.int8).reshape(4, 256)
    # the absmax element of each group maps to +-127 exactly
    for gi in range(8):
        row, col = divmod(gi * 128, 256)
        grp = w[row, col:col + 128]
        assert abs(int(q[row, col + np.argmax(np.abs(grp))])) == 127
    restored = oc.q8_dequantize(data, sc, (4, 256))
    s = np.repeat(np.frombuffer(sc, "<f4"), 128).reshape(4, 256)
    assert np.all(np.abs(restored - w) <= s / 2 + 1e-9)


# ---------------------------------------------------- product vs oracle ----
def test_product_q4_codec_matches_oracle():
    from uma_qmoe_amd import formats as pq

    rng = np.random.default_rng(2)
    for n in (1, 5, 128, 129, 1000):
        w = (rng.standard_normal(n) * 0.02).astype(np.float32)
        t = pq.quantize_q4(w)
        packed, scales = oc.q4_quantize(w, 128)
        assert t.packed == packed and t.scales == scales
        assert np.array_equal(pq.dequantize_q4(t), oc.q4_dequantize(packed, scales, (n,)))
    assert pq.pack_int4(np.array([-7, -1, 0, 1, 7])) == bytes((0xF9, 0x10, 0x07))
    with pytest.raises(ValueError, match="reserved -8"):
        pq.unpack_int4(bytes((0x08,)), 1)
    with pytest.raises(ValueError, match="tail padding"):
        pq.unpack_int4(bytes((0x10,)), 1)


def test_product_bulk_torch_codecs_match_oracle():
    from uma_qmoe_amd.formats import bf16_words, encode_projection, encode_target_tensor

    g = torch.Generator().manual_seed(3)
    w = torch.randn(3, 8, 256, generator=g) * 0.02
    d4, s4 = encode_projection(w, "q4_group128")
    d8, s8 = encode_projection(w, "q8_group128")
    for e in range(3):
        ref_p, ref_s = oc.q4_quantize(w[e].numpy(), 128)
        assert d4[e].numpy().tobytes() == ref_p and s4[e].numpy().astype("<f4").tobytes() == ref_s
        ref_q, ref_s8 = oc.q8_quantize(w[e].numpy(), 128)
        assert d8[e].numpy().tobytes() == ref_q and s8[e].numpy().astype("<f4").tobytes() == ref_s8
        t8 = encode_target_tensor(w[e].numpy(), "q8_group128")
        assert t8.data == ref_q and t8.scales == ref_s8
    f = w.reshape(-1)
    assert np.array_equal(bf16_words(f).numpy().view(np.uint16), oc.f32_to_bf16_bits(f.numpy()))
    db, sb = encode_projection(w, "bf16_le")
    assert sb is None and np.array_equal(db.view(torch.int16).numpy().view(np.uint16).reshape(-1),
                                         oc.f32_to_bf16_bits(f.numpy()))
