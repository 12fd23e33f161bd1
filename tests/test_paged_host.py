"""Host side of the paged drop-in (no GPU): layout geometry, bookkeeping,
constructor checks and the page-size formula, against the oracle and the
reference's own known answers (tests/test_slimkv_paged_cache.py,
slimkv/vllm_plugin/backend.py:108-131)."""
import pytest
import torch

from oracle import paged as opaged


def test_layout_properties_and_errors_match_oracle():
    from slimkv_amd.paged_cache import BeaconPageLayout
    for args in [(4, 2, 3, 5, 4), (16, 8, 256, 256, 1024), (16, 4, 128, 384, 1024), (480, 8, 256, 256, 1024)]:
        ours, ref = BeaconPageLayout(*args), opaged.Layout(*args)
        for name in ('slots', 'width', 'sink_elements', 'page_elements', 'storage_rows'):
            assert getattr(ours, name) == getattr(ref, name), (args, name)
    with pytest.raises(ValueError):
        BeaconPageLayout(6, 4, 3, 5, 4)
    with pytest.raises(ValueError):
        BeaconPageLayout(16, 8, 0, 5, 4)
    # the reference KAT's page: 4 sink elements x2, 2 slots of width 8
    assert BeaconPageLayout(4, 2, 3, 5, 4).page_elements == 24


def test_bookkeeping_matches_oracle():
    from slimkv_amd.paged_model import flush_raw_start, restore_counts, window_roles
    for processed in [0, 1, 3, 7, 1023, 1024, 1025, 2500, 131071]:
        for window, ratio in [(1024, 4), (1024, 8), (16, 4)]:
            assert restore_counts(processed, window, ratio) == opaged.restore_counts(processed, window, ratio)
            raw = processed % window
            assert window_roles(raw, ratio).tolist() == opaged.window_roles(raw, ratio).tolist()
    for prev, cur in [(1000, 1030), (1025, 1030), (0, 3), (3, 10), (2047, 2049)]:
        assert flush_raw_start(prev, cur, 1024) == opaged.flush_raw_start(prev, cur, 1024)


def test_page_geometry_known_answers():
    from slimkv_amd.paged_model import page_geometry
    g = page_geometry(1024, 512, 8)                        # Llama-3.1-8B t8, r 32 per head (rk = rv = 256)
    assert (g.raw_block, g.beacon_block, g.page_bytes) == (16, 480, 65536)
    assert g.beacon_block == opaged.beacon_block_tokens(1024, 512, 8)
    assert page_geometry(1024, 512, 4).beacon_block == 240
    # storage rows: 60 beacons + ceil(2048 / 512) sink rows; page bytes = the raw page's
    assert g.storage_block_size(512) == 64 and g.real_page_size_bytes(512) == 65536
    with pytest.raises(ValueError):
        page_geometry(64, 4096, 8)


def test_pages_constructor_checks_without_gpu():
    from slimkv_amd.paged_cache import BeaconPageLayout, BeaconPages, RawPages
    layout = BeaconPageLayout(4, 2, 3, 5, 4)
    with pytest.raises(ValueError):
        BeaconPages(torch.zeros(3, 24), layout)                                   # not bf16
    with pytest.raises(ValueError):
        BeaconPages(torch.zeros(3, 20, dtype=torch.bfloat16), layout)            # page too small
    with pytest.raises(ValueError):
        BeaconPages(torch.zeros(3, 4, 8, dtype=torch.bfloat16).transpose(1, 2), layout)  # not page-contiguous
    pages = BeaconPages(torch.zeros(3, 3, 8, dtype=torch.bfloat16), layout)      # [pages, rows, width]
    assert pages.pages.shape == (3, 24)
    with pytest.raises(ValueError):
        RawPages(torch.zeros(8, 4, 3, 2, 3, dtype=torch.bfloat16))
    with pytest.raises(ValueError):                                              # no CPU compute path
        pages.read(torch.tensor([0, 1, 2]), 4)


def test_paged_step_plan_matches_oracle():
    """plan_paged_step's per-request counts and slot positions against the
    oracle's restatement of restore_memory (paged_model.py:12-35), the decode
    key positions of fa2_decode.decode (fa2_decode.py:122-126), the insertion
    rule (memory.py:122-124: a beacon after every `ratio` raw tokens, so at
    (P + 1) % ratio == 0) and flush_memory's raw start (paged_model.py:58-59)."""
    import numpy as np
    from oracle import rope as orope
    from slimkv_amd.paged_step import plan_paged_step
    for window, ratio, sink in [(32, 4, 1), (1024, 8, 1), (64, 16, 0)]:
        for P in [1, 2, 3, 7, 15, 16, window - 1, window, window + 1, 3 * window - 1, 5 * window + 7, 100_001]:
            (g,) = plan_paged_step([P], window, ratio, sink, 'cpu')
            t = {k: v[0] for k, v in g.tensors.items()}
            rc, hist, beacons = opaged.restore_counts(P, window, ratio)
            roles = opaged.window_roles(rc, ratio)
            size = int((P + 1) % ratio == 0)
            mem = sink + hist + roles.size
            keys = sink + rc + 1
            want = orope.decode_key_positions(keys, sink, hist, np.nonzero(roles == 0)[0], mem)
            assert g.size == size, (window, ratio, P)
            assert t['raw_positions'][:keys].tolist() == want.tolist(), (window, ratio, P)
            assert t['q_positions'].tolist() == list(range(mem, mem + 1 + size))
            assert (int(t['raw_lengths']), int(t['raw_count']), int(t['window_start'])) == (keys, rc, P - rc)
            assert (int(t['beacon_start']), int(t['lat_lengths'])) == (beacons, beacons + size)
            raw_start = opaged.flush_raw_start(P, P + 1, window)
            assert int(t['raw_write_end']) == (P + 1 if P + 1 > raw_start else P)
            assert bool(t['sink_update']) == (sink > 0 and hist == 0)
            assert (g.max_raw, g.max_beacons, g.rows_total) == (keys, beacons + size, beacons + size)
    with pytest.raises(ValueError):
        plan_paged_step([5], 24, 4, 1, 'cpu')                  # window not a multiple of 16
    with pytest.raises(ValueError):
        plan_paged_step([0], 32, 4, 1, 'cpu')                  # a decode step follows a prefill
