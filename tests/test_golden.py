"""The golden fixtures (tests/golden/*.npz) against this host's draw and the oracle.

Each case's inputs are drawn again and must carry the fixture's SHA-256
digests; the oracle's results on them must equal the stored ones: bit-exact
results by digest, page and raw-block index vectors exactly, floating-point
results to their float32 storage.  Planted mistakes in the oracle (a RoPE sign,
a key position off by one, swapped page slots) must each move a stored result,
which shows that the fixtures pin those parts.  test_gpu_golden.py runs the
HIP path on the same inputs.
"""
import numpy as np
import pytest

from oracle import paged as opaged
from oracle import rope as orope
from tests.golden import make_golden as mg


def _compare(case, stored, fresh):
    assert set(stored) == set(fresh), f'{case}: fixture keys differ'
    for k, v in fresh.items():
        if isinstance(v, str):
            assert stored[k] == v, f'{case}: {k} differs'
        elif np.asarray(v).dtype.kind == 'f':
            np.testing.assert_allclose(stored[k], v, rtol=1e-6, atol=1e-6, err_msg=f'{case}: {k}')
        else:
            np.testing.assert_array_equal(stored[k], v, err_msg=f'{case}: {k}')


@pytest.mark.parametrize('case', mg.CASES)
def test_fixture_matches_oracle(case):
    stored = mg.load(case)
    _, _, fresh = mg.build(case)
    _compare(case, stored, fresh)


def test_fixture_inputs_are_bf16_exact():
    """Every drawn bf16 input is exactly representable (the digests are of its bits)."""
    from oracle.bf16 import round_bf16
    for case in mg.CASES:
        inp, _ = mg.BUILDERS[case][0]()
        for name, x in inp.items():
            if x.dtype == np.float32 and name not in ('cos', 'sin'):
                assert (round_bf16(x) == x).all(), f'{case}: {name}'


def test_c4_indices_follow_the_page_formulas():
    """Beacon i of a sequence sits in page table[i // slots] at column
    2 * raw_width + (i % slots) * width (paged_cache.py:60-67); raw token t in
    block table[t // 16] at offset t % 16 (paged_cache.py:111-127)."""
    stored = mg.load('c4_paged_decode')
    inp, _ = mg.c4_inputs()
    slots, width, sink = 2, 128, 512
    for b, n in enumerate(inp['lat_len']):
        i = np.arange(n)
        np.testing.assert_array_equal(stored[f'beacon_page_{b}'], inp['tables'][b][i // slots])
        np.testing.assert_array_equal(stored[f'beacon_column_{b}'], sink + (i % slots) * width)
    for b, m in enumerate(inp['raw_len']):
        t = np.arange(m)
        np.testing.assert_array_equal(stored[f'raw_block_{b}'], inp['raw_tables'][b][t // 16])
        np.testing.assert_array_equal(stored[f'raw_offset_{b}'], t % 16)


def test_planted_rope_sign_moves_the_digests(monkeypatch):
    stored = mg.load('c0_latent_decode')
    half = 64
    monkeypatch.setattr(orope, 'rotate_half', lambda x: np.concatenate([x[..., half:], -x[..., :half]], axis=-1))
    inp, meta = mg.c0_inputs()
    fresh = mg.c0_expected(inp, meta)
    assert fresh['sha_q_rot'] != stored['sha_q_rot'] and fresh['sha_k_rot'] != stored['sha_k_rot']
    assert np.abs(fresh['out'] - stored['out']).max() > 2e-2


def test_planted_key_position_moves_the_digest(monkeypatch):
    stored = mg.load('c0_latent_decode')
    inp, meta = mg.c0_inputs()
    meta['history'] += 1
    fresh = mg.c0_expected(inp, meta)
    assert fresh['sha_q_rot'] == stored['sha_q_rot']
    assert fresh['sha_k_rot'] != stored['sha_k_rot']


def test_planted_slot_swap_moves_the_gather(monkeypatch):
    stored = mg.load('c4_paged_decode')
    real = opaged.beacon_indices

    def swapped(layout, table, start, count):
        page, first = real(layout, table, start, count)
        slot = (first - layout.sink_elements) // layout.width
        return page, layout.sink_elements + (layout.slots - 1 - slot) * layout.width

    monkeypatch.setattr(opaged, 'beacon_indices', swapped)
    inp, meta = mg.c4_inputs()
    fresh = mg.c4_expected(inp, meta)
    assert fresh['sha_beacon_rows'] != stored['sha_beacon_rows']
    assert np.abs(fresh['out'] - stored['out']).max() > 2e-2
