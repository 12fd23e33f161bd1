"""Lossless bf16 cache I/O over engine-owned physical pages, on the GPU.

Drop-in for slimkv/vllm_plugin/paged_cache.py:11-127 (BeaconPageLayout,
BeaconPages, RawPages): same constructor checks, error types and results.
The index math (page = table[i // slots], column = sink_elements +
(i % slots) * width) and the copies run in one HIP kernel per call instead of
torch advanced indexing; pages and dense tensors must live on the GPU.

Beyond the reference's one-request calls, `read_batch`/`append_batch` move
the rows of many requests (one block-table row each) in one launch.
"""
from dataclasses import dataclass

import torch

from . import kernels


@dataclass(frozen=True)
class BeaconPageLayout:
    """Geometry of one beacon page (paged_cache.py:11-44)."""
    raw_block_size: int
    token_ratio: int
    key_rank: int
    value_rank: int
    raw_width: int

    def __post_init__(self):
        if min(self.raw_block_size, self.token_ratio, self.key_rank, self.value_rank, self.raw_width) <= 0:
            raise ValueError('Cache dimensions must be positive.')
        if self.raw_block_size % self.token_ratio:
            raise ValueError('Raw block size must be divisible by the token ratio.')

    @property
    def slots(self):
        return self.raw_block_size // self.token_ratio

    @property
    def width(self):
        return self.key_rank + self.value_rank

    @property
    def sink_elements(self):
        return 2 * self.raw_width

    @property
    def page_elements(self):
        return self.sink_elements + self.slots * self.width

    @property
    def storage_rows(self):
        return (self.page_elements + self.width - 1) // self.width


class BeaconPages:
    """Read and append compact rows without owning or allocating KV pages
    (paged_cache.py:47-99)."""

    def __init__(self, pages, layout):
        if pages.dtype != torch.bfloat16:
            raise ValueError('SlimKV pages must retain BF16 checkpoint precision.')
        self.pages = pages.flatten(1)
        if self.pages.data_ptr() != pages.data_ptr():
            raise ValueError('Each physical page must have contiguous feature storage.')
        if self.pages.shape[1] < layout.page_elements:
            raise ValueError('Physical page is too small for the declared ranks.')
        self.layout = layout

    def _move(self, table, start, key, value, to_pages, lengths=None, status=None):
        """Block-table entries follow torch's indexing rules; an entry outside
        the pool that a row needs raises IndexError (as the reference's indexing
        does, paged_cache.py:60-67), or with a caller `status` word is left there."""
        L = self.layout
        kernels.beacon_pages(self.pages, table, key, value, slots=L.slots, key_rank=L.key_rank,
                             value_rank=L.value_rank, sink_elements=L.sink_elements, start=start,
                             count=key.shape[1], to_pages=to_pages, lengths=lengths, status=status)

    def read(self, block_table, count):
        """(k [1,1,count,key_rank], v [1,1,count,value_rank]) of beacons 0..count-1."""
        if count == 0:
            return None, None
        L = self.layout
        k = torch.empty(1, count, L.key_rank, dtype=self.pages.dtype, device=self.pages.device)
        v = torch.empty(1, count, L.value_rank, dtype=self.pages.dtype, device=self.pages.device)
        self._move(block_table, 0, k, v, False)
        return k[None], v[None]

    def append(self, block_table, start, key, value):
        """Store key [1,1,n,key_rank] / value [1,1,n,value_rank] as beacons start..start+n-1."""
        if key.dtype != self.pages.dtype or value.dtype != self.pages.dtype:
            raise ValueError('Cache writes must not change dtype.')
        if (key.ndim != 4 or value.ndim != 4 or key.shape[:2] != (1, 1)
                or value.shape[:3] != key.shape[:3]
                or key.shape[-1] != self.layout.key_rank
                or value.shape[-1] != self.layout.value_rank):
            raise ValueError('Expected independent B1 global-rank K/V tensors.')
        if key.shape[2] == 0:
            return
        self._move(block_table, start, key[0], value[0], True)

    def read_batch(self, tables, lengths, count=None, status=None):
        """Dense latents of many requests: tables [B, T] (one block-table row per
        request), lengths [B] beacon counts.  Returns k [B, count, key_rank] and
        v [B, count, value_rank]; rows at or past a request's length are zero.
        `status`: an optional device int32 word that receives index errors
        instead of an IndexError (then rows with an index error stay zero)."""
        L = self.layout
        count = int(lengths.max()) if count is None else count
        B = tables.shape[0]
        k = torch.zeros(B, count, L.key_rank, dtype=self.pages.dtype, device=self.pages.device)
        v = torch.zeros(B, count, L.value_rank, dtype=self.pages.dtype, device=self.pages.device)
        if count:
            self._move(tables, 0, k, v, False, lengths, status)
        return k, v

    def append_batch(self, tables, start, key, value, lengths=None, status=None):
        """Store key [B, n, key_rank] / value [B, n, value_rank] of many requests
        as their beacons start..start+n-1 (rows past lengths[b] are skipped;
        `status` as read_batch)."""
        if key.shape[1]:
            self._move(tables, start, key, value, True, lengths, status)

    def write_sink(self, root_block, key, value):
        rows = torch.cat([key.flatten(), value.flatten()])
        if rows.numel() != self.layout.sink_elements or rows.dtype != self.pages.dtype:
            raise ValueError('Sink cache must retain the original raw K/V dimensions.')
        self.pages[root_block, :self.layout.sink_elements].copy_(rows)

    def read_sink(self, root_block, heads, head_dim):
        if heads * head_dim != self.layout.raw_width:
            raise ValueError('Sink head dimensions differ from the page layout.')
        rows = self.pages[root_block, :self.layout.sink_elements]
        return tuple(x.reshape(1, heads, 1, head_dim) for x in rows.split(self.layout.raw_width))


class RawPages:
    """Read current-window raw KV using absolute raw-token positions
    (paged_cache.py:102-127)."""

    def __init__(self, pages):
        if pages.dtype != torch.bfloat16 or pages.ndim != 5 or pages.shape[2] != 2:
            raise ValueError('Expected BF16 pages in block/token/KV/head/dim order.')
        self.pages = pages
        self.block_size = pages.shape[1]

    def read(self, block_table, start, count):
        """(K, V) as [1, Hkv, count, D] of raw positions start..start+count-1."""
        if count == 0:
            return None, None
        _, _, _, H, D = self.pages.shape
        k = torch.empty(1, H, count, D, dtype=self.pages.dtype, device=self.pages.device)
        v = torch.empty_like(k)
        kernels.raw_pages(self.pages, block_table, k, v, start=start, count=count, to_pages=False)
        return k, v

    def write(self, block_table, start, key, value):
        """Store key/value [1, Hkv, n, D] at raw positions start..start+n-1."""
        if key.dtype != self.pages.dtype or value.dtype != self.pages.dtype:
            raise ValueError('Raw cache writes must retain BF16 values.')
        key, value = key[:1], value[:1]                       # the reference writes key[0]
        if (key.ndim != 4 or value.shape != key.shape
                or (key.shape[1], key.shape[3]) != tuple(self.pages.shape[3:])):
            raise ValueError('Raw cache dimensions differ from the engine allocation.')
        if key.shape[2] == 0:
            return
        kernels.raw_pages(self.pages, block_table, key.contiguous(), value.contiguous(), start=start,
                          count=key.shape[2], to_pages=True)

    def read_batch(self, tables, start, count, lengths=None):
        """K, V [B, Hkv, count, D] of positions start..start+count-1 of many requests."""
        _, _, _, H, D = self.pages.shape
        k = torch.zeros(tables.shape[0], H, count, D, dtype=self.pages.dtype, device=self.pages.device)
        v = torch.zeros_like(k)
        if count:
            kernels.raw_pages(self.pages, tables, k, v, start=start, count=count, to_pages=False, lengths=lengths)
        return k, v
