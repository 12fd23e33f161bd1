"""Paged latent decode (slimkv_paged_latent_decode): the fused latent decode
reading beacon rows straight out of BeaconPageLayout pages through the block
table, instead of restore_memory's gather (slimkv/vllm_plugin/paged_model.py:
36-52 via BeaconPages.read, paged_cache.py:60-87) followed by the decode.

Index handling is checked bit-exactly: with the same key splits the paged
decode equals gather + dense decode bit for bit (same rows, same arithmetic),
for power-of-two and other slot counts (pages of 2 to 60 rows, both
addressing modes of the kernel), ragged lengths including empty
sequences, and table entries past a sequence's pages that hold garbage.  The
automatic compact schedule (splits sized from the total row count, only
non-empty splits launched) is checked against the oracle's float64 attention
within the bf16 bar.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from slimkv_amd.workloads import block_diagonal, orthonormal_columns
from tests.helpers import assert_close, to_np

pytestmark = pytest.mark.gpu

HQ, HKV, D = 32, 8, 128


def _case(device, layout_args, lengths, raw_lengths, seed=0, pool_extra=7, garbage=True, heads=HQ):
    from slimkv_amd.paged_cache import BeaconPageLayout
    layout = BeaconPageLayout(*layout_args)
    gen = torch.Generator(device=device).manual_seed(seed)
    cpu = torch.Generator().manual_seed(seed + 1)
    B = len(lengths)
    pages_needed = [(n + layout.slots - 1) // layout.slots for n in lengths]
    width = max(max(pages_needed), 1) + 2
    pool = sum(pages_needed) + pool_extra
    pages = torch.randn(pool, layout.page_elements, generator=gen, device=device).to(torch.bfloat16)
    perm = torch.randperm(pool, generator=cpu)
    tables = torch.full((B, width), -1, dtype=torch.long)
    if garbage:   # entries past each sequence's pages hold ids far outside the pool
        tables = torch.randint(-(1 << 40), 1 << 40, (B, width), generator=cpu)
    off = 0
    for b, n in enumerate(pages_needed):
        tables[b, :n] = perm[off:off + n]
        off += n
    r_k, r_v = layout.key_rank // HKV, layout.value_rank // HKV
    up_k = block_diagonal([orthonormal_columns(D, r_k, cpu) for _ in range(HKV)]).to(device, torch.bfloat16)
    up_v = block_diagonal([orthonormal_columns(D, r_v, cpu) for _ in range(HKV)]).to(device, torch.bfloat16)
    max_raw = max(raw_lengths)
    raw_k = torch.randn(B, max_raw, HKV, D, generator=gen, device=device).to(torch.bfloat16)
    raw_v = torch.randn(B, max_raw, HKV, D, generator=gen, device=device).to(torch.bfloat16)
    q = torch.randn(B, 1, heads, D, generator=gen, device=device).to(torch.bfloat16)
    return dict(layout=layout, pages=pages, tables=tables.to(device), up_k=up_k, up_v=up_v, raw_k=raw_k,
                raw_v=raw_v, q=q, lengths=torch.tensor(lengths, dtype=torch.int32, device=device),
                raw_lengths=torch.tensor(raw_lengths, dtype=torch.int32, device=device), lat_keys=max(lengths))


def _dense(c):
    from slimkv_amd.paged_cache import BeaconPages
    return BeaconPages(c['pages'], c['layout']).read_batch(c['tables'], c['lengths'], count=c['lat_keys'])


@pytest.mark.parametrize('layout_args,lengths', [
    ((16, 8, 256, 256, 1024), [1000, 0, 37, 1, 777, 16, 15, 1024]),     # 2 slots per page (t8)
    ((16, 4, 256, 256, 1024), [333, 1024, 5, 0, 64, 900]),              # 4 slots per page (t4)
    ((12, 4, 256, 256, 1024), [301, 2, 299, 150]),                      # 3 slots: non-power-of-two
    ((16, 8, 128, 384, 1024), [513, 77, 1, 240]),                       # rank 16 K, rank 48 V
    # pages of at least 16 rows: a tile reads its two pages' ids once
    ((480, 8, 256, 256, 1024), [1000, 0, 37, 1, 777, 59, 60, 61, 1024]),  # 60 slots (the plugin's t8 pages)
    ((256, 8, 256, 256, 1024), [513, 31, 32, 33, 0, 2000]),             # 32 slots: power of two
    ((128, 8, 128, 384, 1024), [513, 77, 1, 240, 15, 16, 17]),          # 16 slots: tiles on page boundaries
])
@pytest.mark.parametrize('splits', [3, 8])
def test_paged_equals_gather_then_decode_bitwise(device, layout_args, lengths, splits):
    from slimkv_amd import kernels
    raw_lengths = [5 + (7 * i) % 40 for i in range(len(lengths))]
    c = _case(device, layout_args, lengths, raw_lengths, seed=len(lengths) + splits)
    lat_k, lat_v = _dense(c)
    scale = D ** -0.5
    # the same split plan on both sides (the automatic plans differ: paged rows
    # take a compact schedule and longer raw splits)
    want, want_lse = kernels.latent_decode(c['q'], c['raw_k'], c['raw_v'], lat_k, lat_v, c['up_k'], c['up_v'],
                                           scale, block_diagonal=True, raw_lengths=c['raw_lengths'],
                                           lat_lengths=c['lengths'], lat_splits=splits, raw_splits=2)
    got, got_lse = kernels.paged_latent_decode(c['q'], c['raw_k'], c['raw_v'], c['pages'], c['tables'],
                                               c['lengths'], c['lat_keys'], c['layout'], c['up_k'], c['up_v'],
                                               scale, block_diagonal=True, raw_lengths=c['raw_lengths'],
                                               lat_splits=splits, raw_splits=2)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(got_lse, want_lse)


@pytest.mark.parametrize('layout_args', [(16, 8, 256, 256, 1024), (480, 8, 256, 256, 1024)])
@pytest.mark.parametrize('rows_total', ['exact', 0, 'low', 'high'])
def test_compact_schedule_matches_oracle(device, rows_total, layout_args):
    """Automatic splits: rows_total only sizes them, so an exact, unknown,
    too-low or too-high hint gives the same (correct) result, with 2-row and
    60-row pages."""
    from slimkv_amd import kernels
    lengths = [4100, 0, 1, 2047, 16, 3000, 255, 8191]
    raw_lengths = [1, 133, 64, 17, 4, 100, 2, 129]
    c = _case(device, layout_args, lengths, raw_lengths, seed=11)
    hint = {'exact': sum(lengths), 0: 0, 'low': 100, 'high': 10 * sum(lengths)}[rows_total]
    scale = D ** -0.5
    got, lse = kernels.paged_latent_decode(c['q'], c['raw_k'], c['raw_v'], c['pages'], c['tables'], c['lengths'],
                                           c['lat_keys'], c['layout'], c['up_k'], c['up_v'], scale,
                                           rows_total=hint, block_diagonal=True, raw_lengths=c['raw_lengths'])
    lat_k, lat_v = _dense(c)
    torch.cuda.synchronize()
    q = to_np(c['q'].transpose(1, 2))                                  # [B, H, 1, D]
    raw_k, raw_v = to_np(c['raw_k'].transpose(1, 2)), to_np(c['raw_v'].transpose(1, 2))
    up_k, up_v = to_np(c['up_k']), to_np(c['up_v'])
    for b, (n, nr) in enumerate(zip(lengths, raw_lengths)):
        ref, ref_lse = oa.latent_layer(q[b:b + 1], raw_k[b:b + 1, :, :nr], raw_v[b:b + 1, :, :nr],
                                       to_np(lat_k)[b:b + 1, None, :n], to_np(lat_v)[b:b + 1, None, :n],
                                       up_k, up_v, scale, HKV)
        assert_close(to_np(got.transpose(1, 2))[b:b + 1], ref, what=f'sequence {b}')
        np.testing.assert_allclose(to_np(lse)[b:b + 1], ref_lse, atol=2e-3, rtol=1e-4)


@pytest.mark.parametrize('heads', [40, 64, 16])
def test_compact_schedule_other_gqa_groups(device, heads):
    """Query heads 40, 64 and 16 on the 8 KV heads of the page layout (GQA
    groups of five, eight and two: the latent tiles hold whole KV heads),
    beacon and raw rows from their pages' dense gather, against the oracle."""
    from slimkv_amd import kernels
    lengths = [3000, 1, 0, 2047, 777]
    raw_lengths = [133, 1, 7, 64, 100]
    c = _case(device, (16, 8, 256, 256, 1024), lengths, raw_lengths, seed=heads, heads=heads)
    scale = D ** -0.5
    got, lse = kernels.paged_latent_decode(c['q'], c['raw_k'], c['raw_v'], c['pages'], c['tables'], c['lengths'],
                                           c['lat_keys'], c['layout'], c['up_k'], c['up_v'], scale,
                                           rows_total=sum(lengths), block_diagonal=True, raw_lengths=c['raw_lengths'])
    lat_k, lat_v = _dense(c)
    torch.cuda.synchronize()
    q = to_np(c['q'].transpose(1, 2))
    raw_k, raw_v = to_np(c['raw_k'].transpose(1, 2)), to_np(c['raw_v'].transpose(1, 2))
    up_k, up_v = to_np(c['up_k']), to_np(c['up_v'])
    for b, (n, nr) in enumerate(zip(lengths, raw_lengths)):
        ref, ref_lse = oa.latent_layer(q[b:b + 1], raw_k[b:b + 1, :, :nr], raw_v[b:b + 1, :, :nr],
                                       to_np(lat_k)[b:b + 1, None, :n], to_np(lat_v)[b:b + 1, None, :n],
                                       up_k, up_v, scale, HKV)
        assert_close(to_np(got.transpose(1, 2))[b:b + 1], ref, what=f'sequence {b}')
        np.testing.assert_allclose(to_np(lse)[b:b + 1], ref_lse, atol=2e-3, rtol=1e-4)


def test_rejects_tables_narrower_than_the_beacon_count(device):
    from slimkv_amd import kernels
    c = _case(device, (16, 8, 256, 256, 1024), [100, 40], [3, 3], seed=3)
    with pytest.raises(ValueError, match='block table'):
        kernels.paged_latent_decode(c['q'], c['raw_k'], c['raw_v'], c['pages'], c['tables'][:, :10], c['lengths'],
                                    c['lat_keys'], c['layout'], c['up_k'], c['up_v'], D ** -0.5,
                                    block_diagonal=True, raw_lengths=c['raw_lengths'])


@pytest.mark.parametrize('layout_args,start,blocks', [((16, 8, 256, 256, 1024), 3, 8), ((16, 4, 256, 256, 1024), 0, 8),
                                                      ((12, 4, 128, 384, 1024), 5, 1)])
def test_down_projection_into_pages_equals_project_then_append(device, layout_args, start, blocks):
    """The down-projection epilogue writing beacon latents straight into pages
    leaves every page element exactly as projecting to a dense buffer and
    appending it (BeaconPages.append_batch) does, untouched elements included."""
    from slimkv_amd import kernels
    from slimkv_amd.paged_cache import BeaconPageLayout, BeaconPages
    layout = BeaconPageLayout(*layout_args)
    gen = torch.Generator(device=device).manual_seed(start + blocks)
    B, L, K, n = 3, 300, 1024, 70
    x = torch.randn(B, L, K, generator=gen, device=device).to(torch.bfloat16)
    rows = torch.randperm(L, generator=torch.Generator().manual_seed(4))[:n].sort().values.to(device)
    wk = (torch.randn(layout.key_rank, K, generator=gen, device=device) / 32).to(torch.bfloat16)
    wv = (torch.randn(layout.value_rank, K, generator=gen, device=device) / 32).to(torch.bfloat16)
    if blocks > 1:   # block-diagonal per-head bases
        mk = torch.block_diag(*[torch.ones(layout.key_rank // blocks, K // blocks)] * blocks).to(device)
        mv = torch.block_diag(*[torch.ones(layout.value_rank // blocks, K // blocks)] * blocks).to(device)
        wk, wv = (wk * mk).to(torch.bfloat16), (wv * mv).to(torch.bfloat16)
    pages_per_seq = (start + n + layout.slots - 1) // layout.slots
    pool = B * pages_per_seq + 5
    table = torch.randperm(pool, generator=torch.Generator().manual_seed(5))[:B * pages_per_seq]
    table = table.view(B, pages_per_seq).to(device)
    base = torch.randn(pool, layout.page_elements + 8, generator=gen, device=device).to(torch.bfloat16)
    want, got = base.clone(), base.clone()
    k = kernels.down_project(x, wk, rows, blocks=blocks)
    v = kernels.down_project(x, wv, rows, blocks=blocks)
    BeaconPages(want[:, :layout.page_elements], layout).append_batch(table, start, k, v)
    kernels.down_project_to_pages(x, wk, got, table, layout, start, 'k', rows, blocks=blocks)
    kernels.down_project_to_pages(x, wv, got, table, layout, start, 'v', rows, blocks=blocks)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize('layout_args', [(16, 8, 256, 256, 1024), (480, 8, 256, 256, 1024)])
def test_negative_entries_wrap_and_index_errors_are_reported(device, layout_args):
    """Table entries follow torch's indexing rules (the reference reads the
    pages with pages[page, column], paged_cache.py:60-73): an entry in
    [-n, 0) is page entry + n -- bit-identical output to the positive ids --
    and an entry outside [-n, n) that a beacon needs raises IndexError, or,
    given a status word, is reported there (garbage past the beacons a
    sequence has is never read, as every other test here checks)."""
    from slimkv_amd import _lib, kernels
    lengths = [700, 37, 0, 121]
    c = _case(device, layout_args, lengths, [9, 17, 3, 40], seed=91)
    scale = D ** -0.5
    args = (c['q'], c['raw_k'], c['raw_v'], c['pages'])
    kw = dict(block_diagonal=True, raw_lengths=c['raw_lengths'], lat_splits=4)

    def run(table, **extra):
        return kernels.paged_latent_decode(*args, table, c['lengths'], c['lat_keys'], c['layout'], c['up_k'],
                                           c['up_v'], scale, **kw, **extra)
    want = run(c['tables'])
    pool = c['pages'].shape[0]
    slots = c['layout'].slots
    neg = c['tables'].clone()
    for b, n in enumerate(lengths):
        used = (n + slots - 1) // slots
        neg[b, :used:2] -= pool                                # every other page by its negative id
    got = run(neg)
    torch.cuda.synchronize()
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
    bad = c['tables'].clone()
    bad[3, (120 // slots)] = pool                              # the page of beacon 120 of sequence 3
    with pytest.raises(IndexError):
        run(bad)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    run(bad, status=status)
    assert int(status.item()) == _lib.STATUS_BAD_PAGE
    status.zero_()
    run(neg, status=status)
    assert int(status.item()) == 0


def _raw_pages_of(c, device, block, seed, garbage=True):
    """The case's dense raw rows written into RawPages-format pages [blocks,
    block, 2, Hkv, D] at a seeded permutation, with a block table (entries
    past a sequence's blocks hold ids outside the pool)."""
    gen = torch.Generator().manual_seed(seed)
    B, max_raw = c['raw_k'].shape[:2]
    per = (max_raw + block - 1) // block
    nblocks = B * per + 3
    pool = torch.randn(nblocks, block, 2, HKV, D, generator=torch.Generator(device=device).manual_seed(seed),
                       device=device).to(torch.bfloat16)
    perm = torch.randperm(nblocks, generator=gen)
    table = torch.randint(-(1 << 40), 1 << 40, (B, per + 1), generator=gen) if garbage \
        else torch.zeros(B, per + 1, dtype=torch.long)
    lengths = c['raw_lengths'].tolist()
    for b in range(B):
        used = (lengths[b] + block - 1) // block
        table[b, :used] = perm[b * per:b * per + used]
        for t in range(lengths[b]):
            blk, off = int(table[b, t // block]), t % block
            pool[blk, off, 0] = c['raw_k'][b, t]
            pool[blk, off, 1] = c['raw_v'][b, t]
    return pool, table.to(device)


@pytest.mark.parametrize('layout_args,lengths,block', [
    ((16, 8, 256, 256, 1024), [1000, 3, 37, 1, 777, 16, 15, 1024], 16),
    ((480, 8, 256, 256, 1024), [513, 31, 32, 33, 1, 2000], 16),
    ((16, 4, 256, 256, 1024), [333, 1024, 5, 64], 32),
])
def test_raw_rows_through_raw_pages_equal_dense_raw_rows(device, layout_args, lengths, block):
    """The raw rows read through raw pages and the block table (no dense
    gather) give the bits of the decode over the same rows held densely, with
    the same split plan; raw row counts 1 to 45 cover partial blocks."""
    from slimkv_amd import kernels
    raw_lengths = [1 + (11 * i) % 45 for i in range(len(lengths))]
    c = _case(device, layout_args, lengths, raw_lengths, seed=len(lengths) + block)
    pool, table = _raw_pages_of(c, device, block, seed=block)
    scale = D ** -0.5
    common = dict(block_diagonal=True, raw_lengths=c['raw_lengths'], lat_splits=5, raw_splits=2)
    want, want_lse = kernels.paged_latent_decode(c['q'], c['raw_k'], c['raw_v'], c['pages'], c['tables'],
                                                 c['lengths'], c['lat_keys'], c['layout'], c['up_k'], c['up_v'],
                                                 scale, **common)
    got, got_lse = kernels.paged_latent_decode(c['q'], None, None, c['pages'], c['tables'], c['lengths'],
                                               c['lat_keys'], c['layout'], c['up_k'], c['up_v'], scale,
                                               raw_pages=pool, raw_tables=table, raw_keys=c['raw_k'].shape[1],
                                               **common)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(got_lse, want_lse)


def test_raw_page_index_errors_are_reported(device):
    """A raw block-table entry outside the pool that a raw row needs raises
    IndexError after the call, as the reference's indexing does; the kernel
    reads block 0 for it and every access stays in bounds."""
    from slimkv_amd import kernels
    c = _case(device, (16, 8, 256, 256, 1024), [64, 32], [20, 9], seed=3)
    pool, table = _raw_pages_of(c, device, 16, seed=4, garbage=False)
    table[1, 0] = pool.shape[0] + 5
    with pytest.raises(IndexError):
        kernels.paged_latent_decode(c['q'], None, None, c['pages'], c['tables'], c['lengths'], c['lat_keys'],
                                    c['layout'], c['up_k'], c['up_v'], D ** -0.5, block_diagonal=True,
                                    raw_lengths=c['raw_lengths'], raw_pages=pool, raw_tables=table)
