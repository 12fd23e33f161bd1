"""Paged-cache index math (oracle), exact integers.

BeaconPageLayout properties  slimkv/vllm_plugin/paged_cache.py:11-44
BeaconPages._indices         slimkv/vllm_plugin/paged_cache.py:60-67
RawPages.read/write indices  slimkv/vllm_plugin/paged_cache.py:111-127
restore_memory counts        slimkv/vllm_plugin/paged_model.py:13-15, 29-35
flush_memory raw start       slimkv/vllm_plugin/paged_model.py:58-59
create_page_layers formula   slimkv/vllm_plugin/backend.py:108-116
"""
import numpy as np


class Layout:
    def __init__(self, raw_block_size, token_ratio, key_rank, value_rank, raw_width):
        if min(raw_block_size, token_ratio, key_rank, value_rank, raw_width) <= 0:
            raise ValueError('Cache dimensions must be positive.')
        if raw_block_size % token_ratio:
            raise ValueError('Raw block size must be divisible by the token ratio.')
        self.raw_block_size, self.token_ratio = raw_block_size, token_ratio
        self.key_rank, self.value_rank, self.raw_width = key_rank, value_rank, raw_width

    slots = property(lambda s: s.raw_block_size // s.token_ratio)
    width = property(lambda s: s.key_rank + s.value_rank)
    sink_elements = property(lambda s: 2 * s.raw_width)
    page_elements = property(lambda s: s.sink_elements + s.slots * s.width)
    storage_rows = property(lambda s: (s.page_elements + s.width - 1) // s.width)


def beacon_indices(layout, block_table, start, count):
    """(physical page [count], first column [count]) of logical beacons start..start+count.
    Columns of beacon i are first[i] + arange(width) (K rank first, then V rank)."""
    logical = np.arange(start, start + count, dtype=np.int64)
    table = np.asarray(block_table, dtype=np.int64)
    page = table[logical // layout.slots]
    first = layout.sink_elements + (logical % layout.slots) * layout.width
    return page, first


def raw_indices(block_size, block_table, start, count):
    """(physical block, offset) of raw tokens start..start+count."""
    pos = np.arange(start, start + count, dtype=np.int64)
    table = np.asarray(block_table, dtype=np.int64)
    return table[pos // block_size], pos % block_size


def restore_counts(processed, window, ratio):
    """raw_count, history_count, beacon_count of a request (paged_model.py:13-15)."""
    raw_count = processed % window
    return raw_count, processed // window * (window // ratio), processed // ratio


def window_roles(raw_count, ratio):
    """Roles of the open window: one beacon after every `ratio` raw tokens
    (paged_model.py:29-31): roles[ratio::ratio+1] = 1."""
    count = raw_count + raw_count // ratio
    roles = np.zeros(count, dtype=np.int64)
    roles[ratio::ratio + 1] = 1
    return roles


def flush_raw_start(previous, current, window):
    return max(previous, current - current % window)


def beacon_block_tokens(raw_width, max_width, ratio, raw_block=16):
    """Raw tokens per beacon page (backend.py:112-116)."""
    page_bytes = raw_block * 2 * raw_width * 2
    return (((page_bytes // 2 - 2 * raw_width) // max_width) * ratio // raw_block) * raw_block
