"""Paged cache I/O on the GPU: bit-exact against the oracle's index math
(slimkv/vllm_plugin/paged_cache.py:11-127) and the reference's own known-answer
cases (tests/test_slimkv_paged_cache.py:45-82), at the reference KAT shapes
(odd widths, single-element path) and at the serving page shape
(BeaconPageLayout(16, 8, 256, 256, 1024), raw blocks [*, 16, 2, 8, 128],
16-byte path)."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import paged as opaged
from tests.helpers import bits

pytestmark = pytest.mark.gpu


def test_reference_kat_shuffled_pages_partial_appends(device):
    """tests/test_slimkv_paged_cache.py:45-67 on device tensors."""
    from slimkv_amd.paged_cache import BeaconPageLayout, BeaconPages
    layout = BeaconPageLayout(4, 2, 3, 5, 4)
    backing = torch.full((12, layout.page_elements + 7), -13, dtype=torch.bfloat16, device=device)
    pages = BeaconPages(backing[:, :layout.page_elements], layout)
    tables = [torch.tensor([7, 2, 9]), torch.tensor([4, 1, 10])]
    stored = []
    for index, table in enumerate(tables):
        k = (torch.arange(18).reshape(1, 1, 6, 3) + index * 32).to(torch.bfloat16).to(device)
        v = (torch.arange(30).reshape(1, 1, 6, 5) + index * 32).to(torch.bfloat16).to(device)
        pages.append(table, 0, k[:, :, :3], v[:, :, :3])
        pages.append(table, 3, k[:, :, 3:], v[:, :, 3:])
        sink = torch.full((1, 1, 1, 4), index + 1, dtype=torch.bfloat16, device=device)
        pages.write_sink(table[0], sink, sink + 2)
        stored.append((k, v, sink))
    for table, (k, v, sink) in zip(tables, stored):
        actual_k, actual_v = pages.read(table, 6)
        assert torch.equal(actual_k, k) and torch.equal(actual_v, v)
        sk, sv = pages.read_sink(table[0], 1, 4)
        assert torch.equal(sk, sink) and torch.equal(sv, sink + 2)
    assert (backing[:, layout.page_elements:] == -13).all()
    assert pages.read(tables[0], 0) == (None, None)
    # every page element equals what the oracle's index math places there
    want = np.full((12, layout.page_elements + 7), -13.0)
    for index, (table, (k, v, sink)) in enumerate(zip(tables, stored)):
        page, first = opaged.beacon_indices(opaged.Layout(4, 2, 3, 5, 4), table.numpy(), 0, 6)
        rows = np.concatenate([k[0, 0].float().cpu().numpy(), v[0, 0].float().cpu().numpy()], axis=1)
        for i in range(6):
            want[page[i], first[i]:first[i] + 8] = rows[i]
        want[int(table[0]), :8] = [index + 1] * 4 + [index + 3] * 4
    untouched = backing.float().cpu().numpy()
    np.testing.assert_array_equal(untouched, want)


def test_reference_kat_raw_window_absolute_positions(device):
    """tests/test_slimkv_paged_cache.py:69-82 on device tensors."""
    from slimkv_amd.paged_cache import RawPages
    raw = RawPages(torch.zeros(8, 4, 2, 2, 3, dtype=torch.bfloat16, device=device))
    table = torch.tensor([5, 2, 6, 1])
    key = torch.arange(42).reshape(1, 2, 7, 3).to(torch.bfloat16).to(device)
    value = -key
    raw.write(table, 5, key, value)
    actual = raw.read(table, 5, 7)
    assert torch.equal(actual[0], key) and torch.equal(actual[1], value)
    other = torch.tensor([5, 2, 6, 1])
    raw.write(other, 5, key + 1, value - 1)
    actual = raw.read(other, 5, 7)
    assert torch.equal(actual[0], key + 1) and torch.equal(actual[1], value - 1)
    block, offset = opaged.raw_indices(4, table.numpy(), 5, 7)
    got = raw.pages.float().cpu().numpy()
    for t in range(7):
        np.testing.assert_array_equal(got[block[t], offset[t], 0], (key + 1)[0, :, t].float().cpu().numpy())


def _serving_pool(device, n_pages, layout, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    data = torch.randn(n_pages, layout.page_elements, generator=gen, device=device).to(torch.bfloat16)
    return data


@pytest.mark.parametrize('start,count', [(0, 37), (5, 40), (1, 1), (0, 512)])
def test_serving_layout_read_append_bit_exact(device, start, count):
    from slimkv_amd.paged_cache import BeaconPageLayout, BeaconPages
    layout = BeaconPageLayout(16, 8, 256, 256, 1024)
    olayout = opaged.Layout(16, 8, 256, 256, 1024)
    n_pages = 600
    pool = _serving_pool(device, n_pages, layout, 11)
    table = torch.randperm(n_pages, generator=torch.Generator().manual_seed(start + count))[:300]
    pages = BeaconPages(pool, layout)
    snapshot = bits(pool)
    gen = torch.Generator(device=device).manual_seed(count)
    k = torch.randn(1, 1, count, 256, generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn(1, 1, count, 256, generator=gen, device=device).to(torch.bfloat16)
    pages.append(table, start, k, v)
    after = bits(pool)
    page, first = opaged.beacon_indices(olayout, table.numpy(), start, count)
    want = snapshot.copy()
    rows = np.concatenate([bits(k[0, 0]), bits(v[0, 0])], axis=1)
    for i in range(count):
        want[page[i], first[i]:first[i] + 512] = rows[i]
    np.testing.assert_array_equal(after, want)                # exactly those bytes changed
    rk, rv = pages.read(table, start + count)
    np.testing.assert_array_equal(bits(rk[0, 0, start:]), bits(k[0, 0]))
    np.testing.assert_array_equal(bits(rv[0, 0, start:]), bits(v[0, 0]))
    pg, fc = opaged.beacon_indices(olayout, table.numpy(), 0, start + count)
    gathered = np.stack([after[pg[i], fc[i]:fc[i] + 512] for i in range(start + count)])
    np.testing.assert_array_equal(bits(rk[0, 0]), gathered[:, :256])
    np.testing.assert_array_equal(bits(rv[0, 0]), gathered[:, 256:])


def test_batched_read_with_lengths_and_negative_entries(device):
    """Batched reads past each request's length stay zero; a negative entry in
    [-n, 0) counts from the end of the pool (torch indexing, as the
    reference's pages[page, column] does)."""
    from slimkv_amd.paged_cache import BeaconPageLayout, BeaconPages
    layout = BeaconPageLayout(16, 8, 256, 256, 1024)
    olayout = opaged.Layout(16, 8, 256, 256, 1024)
    n_pages, B, T = 2000, 9, 120
    pool = _serving_pool(device, n_pages, layout, 5)
    perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(2))[:B * T].reshape(B, T)
    lengths = torch.tensor([0, 1, 2, 3, 77, 128, 239, 240, 17], dtype=torch.int32)
    tables = perm.clone()
    tables[4, 10] = -1                                         # beacons 20, 21 of request 4: the last page
    tables[5, 3] = -n_pages                                    # beacons 6, 7 of request 5: page 0
    tables[2, 5:] = n_pages + 99                               # past request 2's length: never read
    pages = BeaconPages(pool, layout)
    k, v = pages.read_batch(tables.to(device), lengths.to(device))
    assert k.shape == (B, 240, 256) and v.shape == (B, 240, 256)
    host = bits(pool)
    kb, vb = bits(k), bits(v)
    for b in range(B):
        n = int(lengths[b])
        page, first = opaged.beacon_indices(olayout, tables[b].numpy(), 0, n)
        for i in range(240):
            if i >= n:
                assert not kb[b, i].any() and not vb[b, i].any(), (b, i)
            else:   # numpy indexing wraps negative page ids the way torch's does
                np.testing.assert_array_equal(kb[b, i], host[page[i], first[i]:first[i] + 256])
                np.testing.assert_array_equal(vb[b, i], host[page[i], first[i] + 256:first[i] + 512])
    # a batched append of the same rows back into fresh pages round-trips
    fresh = torch.zeros_like(pool)
    again = BeaconPages(fresh, layout)
    again.append_batch(tables.to(device), 0, k, v, lengths.to(device))
    k2, v2 = again.read_batch(tables.to(device), lengths.to(device), count=240)
    assert torch.equal(k2, k) and torch.equal(v2, v)


def test_index_errors_raise_or_report_and_move_nothing(device):
    """An entry outside [-n, n) that a row needs is an index error: the
    reference's indexing raises IndexError; here the copy of that row does not
    happen and the call raises IndexError, or, given a status word, leaves
    SLIMKV_STATUS_BAD_PAGE in it.  A table too short for the rows is the same
    error."""
    from slimkv_amd import _lib
    from slimkv_amd.paged_cache import BeaconPageLayout, BeaconPages, RawPages
    layout = BeaconPageLayout(16, 8, 256, 256, 1024)
    n_pages = 50
    pool = _serving_pool(device, n_pages, layout, 6)
    pages = BeaconPages(pool, layout)
    table = torch.arange(10, dtype=torch.long)[None].repeat(2, 1)
    table[1, 3] = n_pages                                      # beacons 6, 7 of request 1
    lengths = torch.tensor([20, 20], dtype=torch.int32, device=device)
    with pytest.raises(IndexError):
        pages.read_batch(table.to(device), lengths)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    k, v = pages.read_batch(table.to(device), lengths, status=status)
    assert int(status.item()) == _lib.STATUS_BAD_PAGE
    assert not k[1, 6:8].any() and not v[1, 6:8].any() and k[1, 5].any() and k[1, 8].any()
    with pytest.raises(IndexError):                            # single-request read past the table
        pages.read(torch.arange(3), 7)
    before = pool.clone()
    with pytest.raises(IndexError):                            # append: nothing written for the bad rows
        pages.append(torch.tensor([1, -51]), 0, k[:1, None, :4], v[:1, None, :4])
    assert torch.equal(pool[2:], before[2:]) and torch.equal(pool[0], before[0])
    raw = RawPages(torch.zeros(6, 4, 2, 2, 8, dtype=torch.bfloat16, device=device))
    with pytest.raises(IndexError):
        raw.read(torch.tensor([0, 6]), 0, 8)
    assert raw.read(torch.tensor([0, -6]), 0, 8)[0].shape == (1, 2, 8, 8)


def test_raw_pages_serving_shape_batched(device):
    from slimkv_amd.paged_cache import RawPages
    blocks, B = 700, 6
    gen = torch.Generator(device=device).manual_seed(9)
    pool = torch.randn(blocks, 16, 2, 8, 128, generator=gen, device=device).to(torch.bfloat16)
    raw = RawPages(pool)
    tables = torch.randperm(blocks, generator=torch.Generator().manual_seed(4))[:B * 40].reshape(B, 40)
    lengths = torch.tensor([4, 133, 200, 640, 16, 17], dtype=torch.int32)
    k, v = raw.read_batch(tables.to(device), 0, 640, lengths.to(device))
    host = bits(pool)
    for b in range(B):
        n = int(lengths[b])
        block, offset = opaged.raw_indices(16, tables[b].numpy(), 0, n)
        np.testing.assert_array_equal(bits(k[b, :, :n]).transpose(1, 0, 2), host[block, offset, 0])
        np.testing.assert_array_equal(bits(v[b, :, :n]).transpose(1, 0, 2), host[block, offset, 1])
        assert not bits(k[b, :, n:]).any()
    # B1 write at an unaligned start changes exactly the oracle's rows
    snap = bits(pool)
    key = torch.randn(1, 8, 45, 128, generator=gen, device=device).to(torch.bfloat16)
    value = torch.randn(1, 8, 45, 128, generator=gen, device=device).to(torch.bfloat16)
    raw.write(tables[2], 131, key, value)
    block, offset = opaged.raw_indices(16, tables[2].numpy(), 131, 45)
    snap[block, offset, 0] = bits(key[0]).transpose(1, 0, 2)
    snap[block, offset, 1] = bits(value[0]).transpose(1, 0, 2)
    np.testing.assert_array_equal(bits(pool), snap)


class _Memory:
    """The memory attributes restore_memory/flush_memory drive
    (slimkv/vllm_plugin/paged_model.py:7-89)."""

    def __init__(self, layers):
        self.config = SimpleNamespace(num_hidden_layers=layers)
        self._cpu = torch.device('cpu')
        self.reset()

    def reset(self):
        n = self.config.num_hidden_layers
        for name in ('sink_activations', 'raw_activations', 'beacon_activations', 'window_beacon_activations'):
            setattr(self, name, [(None, None) for _ in range(n)])

    def _select_cache_mode(self):
        self.selected = True


def _model(device, layers=2, heads=8, head_dim=128, ranks=((256, 256), (128, 384))):
    attn = [SimpleNamespace(num_key_value_heads=heads, head_dim=head_dim,
                            beacon_k_up_proj=SimpleNamespace(in_features=rk),
                            beacon_v_up_proj=SimpleNamespace(in_features=rv)) for rk, rv in ranks[:layers]]
    return SimpleNamespace(
        memory=_Memory(layers),
        config=SimpleNamespace(beacon_window=64, beacon_ratio=[8], beacon_sink_size=1),
        model=SimpleNamespace(layers=[SimpleNamespace(self_attn=a) for a in attn],
                              embed_tokens=SimpleNamespace(weight=torch.zeros(1, device=device))))


def test_flush_then_restore_round_trips_through_pages(device):
    """flush_memory writes a request's beacons, sink and raw tail; restore_memory
    rebuilds the same tensors and the reference's counts and roles."""
    from slimkv_amd.paged_model import flush_memory, restore_memory, release_workspace_views
    model = _model(device)
    gen = torch.Generator(device=device).manual_seed(3)
    rnd = lambda *s: torch.randn(*s, generator=gen, device=device).to(torch.bfloat16)
    raw_layers = [SimpleNamespace(kv_cache=torch.zeros(64, 16, 2, 8, 128, dtype=torch.bfloat16, device=device))
                  for _ in range(2)]
    beacon_layers = [SimpleNamespace(spec=SimpleNamespace(block_size=16),
                                     kv_cache=torch.zeros(64, 6, 512, dtype=torch.bfloat16, device=device))
                     for _ in range(2)]
    raw_table = torch.randperm(64, generator=torch.Generator().manual_seed(1))[:20]
    beacon_table = [torch.randperm(64, generator=torch.Generator().manual_seed(2 + i))[:20] for i in range(2)]
    # state after 150 tokens (window 64, ratio 8): 16 history + 2 window beacons, raw 128..149 open
    expected = []
    for index, (rk, rv) in enumerate(((256, 256), (128, 384))):
        hist = (rnd(1, 1, 16, rk), rnd(1, 1, 16, rv))
        win = (rnd(1, 1, 2, rk), rnd(1, 1, 2, rv))
        sink = (rnd(1, 8, 1, 128), rnd(1, 8, 1, 128))
        rawkv = (rnd(1, 8, 22, 128), rnd(1, 8, 22, 128))
        model.memory.beacon_activations[index] = hist
        model.memory.window_beacon_activations[index] = win
        model.memory.sink_activations[index] = sink
        model.memory.raw_activations[index] = rawkv
        expected.append([hist, win, sink, rawkv])
    flush_memory(model, 0, 150, raw_layers, beacon_layers, raw_table, beacon_table)
    # ten more tokens: two more window beacons, raw 150..159 -- only those are appended
    for index, (rk, rv) in enumerate(((256, 256), (128, 384))):
        hist, win, sink, rawkv = expected[index]
        win = tuple(torch.cat([w, rnd(1, 1, 2, w.shape[-1])], dim=2) for w in win)
        rawkv = tuple(torch.cat([r, rnd(1, 8, 10, 128)], dim=2) for r in rawkv)
        model.memory.window_beacon_activations[index] = win
        model.memory.raw_activations[index] = rawkv
        expected[index] = [hist, win, sink, rawkv]
    flush_memory(model, 150, 160, raw_layers, beacon_layers, raw_table, beacon_table)
    release_workspace_views(model.memory)
    assert model.memory.beacon_activations[0] == (None, None)
    current = 160
    restore_memory(model, current, raw_layers, beacon_layers, raw_table, beacon_table)
    mem = model.memory
    raw_count, history, beacons = opaged.restore_counts(current, 64, 8)
    assert (mem._start_idx, mem._end_idx, mem._step_idx) == (current - raw_count, current, 3)
    assert mem._beacon_indices.tolist() == opaged.window_roles(raw_count, 8).tolist()
    assert mem._window_raw_indices.tolist() == [i for i, r in enumerate(opaged.window_roles(raw_count, 8)) if not r]
    for index, (hist, win, sink, rawkv) in enumerate(expected):
        for kind in (0, 1):
            assert torch.equal(mem.beacon_activations[index][kind], hist[kind])
            assert torch.equal(mem.window_beacon_activations[index][kind], win[kind])
            assert torch.equal(mem.sink_activations[index][kind], sink[kind])
            assert torch.equal(mem.raw_activations[index][kind], rawkv[kind][:, :, -raw_count:])
    assert (raw_count, history, beacons) == (32, 16, 20)
