"""Pins the oracle's bf16 rounding, RoPE, paged index math and split counts.

* bf16 rounding: torch's float32 -> bfloat16 conversion is the library routine.
* RoPE: torch CPU bf16 elementwise ops are correctly rounded, so
  `x * c + rotate_half(x) * s` in bf16 (the reference torch fallback,
  slimkv/llama3/fa2_decode.py:118-121) must equal the oracle bit for bit;
  position 0 is the identity; tables match float64 closed forms.
* Paged cache: the reference test suite's known-answer cases
  (tests/test_slimkv_paged_cache.py:45-82) and the backend page-size formula
  (slimkv/vllm_plugin/backend.py:112-116).
* Split counts: tests/test_llama_paired_decode.py:35-38.
"""
import math

import numpy as np
import pytest
import torch

from oracle import paged, rope, splits
from oracle.bf16 import from_bits, round_bf16, to_bits


def test_bf16_rounding_matches_torch_conversion():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(2000) * 1e-38).astype(np.float32),       # subnormals
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1.0, 1.00390625, 1.01171875], np.float32),
        # exact ties between bf16 neighbours: round half to even
        from_bits(np.arange(0x3f80, 0x3fa0, dtype=np.uint16)) + np.float32(2.0 ** -8),
    ]).astype(np.float32)
    expected = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (to_bits(vals) == expected).all()
    # NaN stays NaN (torch's CPU kernel and this oracle pick different NaN bit patterns)
    assert np.isnan(from_bits(to_bits(np.array([np.nan], np.float32)))).all()


def test_tables_match_closed_form_and_torch():
    from slimkv_amd.workloads import rope_tables
    inv = rope.inv_freq(128, 500000.0)
    exact = 1.0 / 500000.0 ** (np.arange(0, 128, 2) / 128.0)
    np.testing.assert_allclose(inv, exact, rtol=2.5e-7)              # one fp32 ulp of the closed form
    torch_inv = (1.0 / (500000.0 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))).numpy()
    np.testing.assert_allclose(inv, torch_inv, rtol=2.5e-7)          # torch's pow may differ by one ulp
    cos, sin = rope.tables(4097, torch_inv)
    t = np.arange(4097, dtype=np.float32)
    ang = np.outer(t, torch_inv).astype(np.float32).astype(np.float64)
    np.testing.assert_allclose(cos[:, :64], np.cos(ang), rtol=0, atol=6e-8)
    np.testing.assert_array_equal(cos[:, :64], cos[:, 64:])
    tc, ts = rope_tables(4097, 128, 500000.0)
    # Same fp32 angles: torch's fp32 cos/sin agree with the correctly rounded value to a few ulp.
    np.testing.assert_allclose(tc.numpy(), cos, rtol=0, atol=5e-7)
    np.testing.assert_allclose(ts.numpy(), sin, rtol=0, atol=5e-7)
    assert (cos[0] == 1).all() and (sin[0] == 0).all()


def _torch_rotate(x, c, s):
    xb = torch.from_numpy(x).to(torch.bfloat16)
    cb = torch.from_numpy(c).to(torch.bfloat16)
    sb = torch.from_numpy(s).to(torch.bfloat16)
    half = x.shape[-1] // 2
    rot = torch.cat([-xb[..., half:], xb[..., :half]], dim=-1)
    return (xb * cb + rot * sb).view(torch.int16).numpy().view(np.uint16)


def test_rotation_matches_torch_bf16_arithmetic_bit_for_bit():
    rng = np.random.default_rng(3)
    cos, sin = rope.tables(40000, rope.inv_freq(128, 500000.0))
    x = round_bf16(rng.standard_normal((64, 128)).astype(np.float32) * 4)
    pos = rng.integers(0, 40000, 64)
    ours = to_bits(rope.rotate_bf16(x, cos[pos], sin[pos]))
    assert (ours == _torch_rotate(x, cos[pos], sin[pos])).all()
    # position 0 is the identity
    np.testing.assert_array_equal(rope.rotate_bf16(x, cos[[0]], sin[[0]]), x)


def test_llama3_frequency_smoothing_regions():
    base = rope.inv_freq(128, 500000.0)
    scaled = rope.llama3_inv_freq(128, 500000.0, 8.0, 8192, 1.0, 4.0)
    wavelen = 2 * math.pi / base.astype(np.float64)
    high = wavelen < 8192 / 4
    low = wavelen > 8192 / 1
    np.testing.assert_array_equal(scaled[high], base[high])
    np.testing.assert_allclose(scaled[low], base[low] / 8.0, rtol=1e-7)
    mid = ~(high | low)
    assert mid.any() and (scaled[mid] < base[mid]).all() and (scaled[mid] > base[mid] / 8.0).all()


@pytest.mark.parametrize('base_theta,factor,orig,low_f,high_f', [
    (500000.0, 8.0, 8192, 1.0, 4.0),      # Llama-3.1 rope_scaling
    (10000.0, 4.0, 2048, 1.0, 8.0),       # a wider mid band at another base
])
def test_llama3_mid_band_matches_closed_form(base_theta, factor, orig, low_f, high_f):
    """Every mid-band entry against the closed form in float64: with
    s = (orig / wavelen - low) / (high - low), f' = f * ((1 - s) / factor + s).
    The interpolation weight tends to 1 at the high-frequency edge (f' -> f)
    and to 0 at the low-frequency edge (f' -> f / factor); a swapped s / 1 - s
    or a wrong factor moves every mid-band value by far more than fp32 ulps."""
    base = rope.inv_freq(128, base_theta).astype(np.float64)
    scaled = rope.llama3_inv_freq(128, base_theta, factor, orig, low_f, high_f).astype(np.float64)
    wavelen = 2 * math.pi / base
    mid = (wavelen >= orig / high_f) & (wavelen <= orig / low_f)
    assert mid.sum() >= 3
    s = (orig / wavelen[mid] - low_f) / (high_f - low_f)
    assert ((s >= 0) & (s <= 1)).all()
    expected = base[mid] * ((1 - s) / factor + s)
    np.testing.assert_allclose(scaled[mid], expected, rtol=1e-6, atol=0)
    # monotone in the weight: the ratio f'/f falls from ~1 to ~1/factor across the band
    ratio = scaled[mid] / base[mid]
    assert (np.diff(ratio) <= 1e-7).all()
    np.testing.assert_allclose(ratio, (1 - s) / factor + s, rtol=1e-6)
    # the band edges of the piecewise rule continue the two outer regions
    edge_hi = (orig / (orig / high_f) - low_f) / (high_f - low_f)
    edge_lo = (orig / (orig / low_f) - low_f) / (high_f - low_f)
    assert edge_hi == 1.0 and edge_lo == 0.0


def test_decode_key_positions_rule():
    # slots: 2 sinks, 3 tail slots with window raw indices [0, 1, 3], current token
    pos = rope.decode_key_positions(6, 2, 10, [0, 1, 3], 99)
    assert pos.tolist() == [0, 1, 12, 13, 15, 99]
    # with no sink slot the first slot is a tail slot; the last is always current
    assert rope.decode_key_positions(3, 0, 5, [4, 6], 20).tolist() == [9, 11, 20]


def test_prefill_beacon_mask_rule():
    # keys = 1 sink + 3 history beacons + 6 window slots with roles
    roles = [0, 0, 1, 0, 2, 0]
    mask = rope.prefill_beacon_mask(10, 6, roles, 1)
    assert mask.tolist() == [False, True, True, True, False, False, True, False, True, False]


def _page_store(n_pages, layout, fill=-13.0):
    return np.full((n_pages, layout.page_elements + 7), fill)


def test_beacon_pages_reference_known_answer():
    """tests/test_slimkv_paged_cache.py:45-67: layout (4, 2, 3, 5, 4), tables
    [7,2,9] / [4,1,10], arange-valued K/V appended in two parts, sink writes."""
    layout = paged.Layout(4, 2, 3, 5, 4)
    assert (layout.slots, layout.width, layout.sink_elements, layout.page_elements, layout.storage_rows) == \
        (2, 8, 8, 24, 3)
    store = _page_store(12, layout)
    tables = [np.array([7, 2, 9]), np.array([4, 1, 10])]
    stored = []
    for index, table in enumerate(tables):
        k = np.arange(18).reshape(6, 3) + index * 32
        v = np.arange(30).reshape(6, 5) + index * 32
        for start, stop in ((0, 3), (3, 6)):
            page, first = paged.beacon_indices(layout, table, start, stop - start)
            for i in range(stop - start):
                store[page[i], first[i]:first[i] + 8] = np.concatenate([k[start + i], v[start + i]])
        sink = np.full(8, index + 1.0)
        sink[4:] += 2
        store[table[0], :8] = sink
        stored.append((k, v, sink))
    for table, (k, v, sink) in zip(tables, stored):
        page, first = paged.beacon_indices(layout, table, 0, 6)
        rows = np.stack([store[page[i], first[i]:first[i] + 8] for i in range(6)])
        np.testing.assert_array_equal(rows[:, :3], k)
        np.testing.assert_array_equal(rows[:, 3:], v)
        np.testing.assert_array_equal(store[table[0], :8], sink)
    assert (store[:, layout.page_elements:] == -13).all()
    # exact index values for the first table
    page, first = paged.beacon_indices(layout, tables[0], 0, 6)
    assert page.tolist() == [7, 7, 2, 2, 9, 9] and first.tolist() == [8, 16, 8, 16, 8, 16]


def test_raw_pages_reference_known_answer():
    """tests/test_slimkv_paged_cache.py:69-82: pages [8,4,2,2,3], table
    [5,2,6,1], 7 tokens from absolute position 5."""
    block, offset = paged.raw_indices(4, [5, 2, 6, 1], 5, 7)
    assert block.tolist() == [2, 2, 2, 6, 6, 6, 6]
    assert offset.tolist() == [1, 2, 3, 0, 1, 2, 3]


def test_paged_bookkeeping_formulas():
    assert paged.beacon_block_tokens(1024, 512, 8) == 480      # t8f4 Llama: 60 beacons per page
    assert paged.beacon_block_tokens(1024, 512, 4) == 240
    assert paged.restore_counts(2500, 1024, 4) == (452, 512, 625)
    assert paged.window_roles(7, 4).tolist() == [0, 0, 0, 0, 1, 0, 0, 0]
    assert paged.window_roles(3, 4).tolist() == [0, 0, 0]
    assert paged.flush_raw_start(1000, 1030, 1024) == 1024
    assert paged.flush_raw_start(1025, 1030, 1024) == 1025
    with pytest.raises(ValueError):
        paged.Layout(6, 4, 3, 5, 4)


def test_beacon_indices_brute_force_enumeration():
    layout = paged.Layout(16, 8, 256, 256, 1024)
    table = np.random.default_rng(5).permutation(50)
    page, first = paged.beacon_indices(layout, table, 3, 40)
    for i, logical in enumerate(range(3, 43)):
        assert page[i] == table[logical // 2]
        assert first[i] == 2048 + (logical % 2) * 512


def test_split_count_known_answers():
    for length in [8256, 16448, 32832]:
        assert splits.original_splits(320, length, 32, 78) == 3
        assert splits.original_splits(256, length, 32, 78) == 9
