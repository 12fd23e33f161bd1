"""Restore transient attention workspaces from engine-owned KV pages and flush
new rows back, with the page copies done by the HIP page kernels.

Drop-in for slimkv/vllm_plugin/paged_model.py:7-89 (restore_memory,
flush_memory, release_workspace_views) and for the page-geometry arithmetic of
create_page_layers / BeaconSpec (slimkv/vllm_plugin/backend.py:12-28,108-131).
The functions drive the model's memory object through the same attributes the
reference sets, so they work with any memory that has them.
"""
from dataclasses import dataclass

import torch

from .paged_cache import BeaconPageLayout, BeaconPages, RawPages


def restore_counts(processed, window, ratio):
    """(raw_count, history_count, beacon_count) of a request that has processed
    `processed` raw tokens (paged_model.py:12-15)."""
    raw_count = processed % window
    return raw_count, processed // window * (window // ratio), processed // ratio


def window_roles(raw_count, ratio, device=None):
    """Roles of the open window: a beacon (1) after every `ratio` raw tokens
    (paged_model.py:29-31)."""
    roles = torch.zeros(raw_count + raw_count // ratio, dtype=torch.long, device=device)
    roles[ratio::ratio + 1] = 1
    return roles


def flush_raw_start(previous, current, window):
    """First raw position a flush writes (paged_model.py:58-59)."""
    return max(previous, current - current % window)


def _layer_pages(model, index, raw_layers, beacon_layers, raw_table, beacon_table, ratio):
    attn = model.model.layers[index].self_attn
    raw_blocks = raw_table[index] if isinstance(raw_table, list) else raw_table
    beacon_blocks = beacon_table[index] if isinstance(beacon_table, list) else beacon_table
    layout = BeaconPageLayout(beacon_layers[index].spec.block_size, ratio, attn.beacon_k_up_proj.in_features,
                              attn.beacon_v_up_proj.in_features, attn.num_key_value_heads * attn.head_dim)
    return attn, raw_blocks, beacon_blocks, BeaconPages(beacon_layers[index].kv_cache, layout)


def restore_memory(model, processed, raw_layers, beacon_layers, raw_table, beacon_table):
    """Rebuild the model memory of one request from its pages (paged_model.py:7-52)."""
    memory = model.memory
    memory.reset()
    if processed == 0:
        return
    window, ratio = model.config.beacon_window, model.config.beacon_ratio[0]
    raw_count, history_count, beacon_count = restore_counts(processed, window, ratio)
    memory.all_input_ids = torch.zeros(1, processed, dtype=torch.long, device=memory._cpu)
    memory.all_attention_mask = torch.ones_like(memory.all_input_ids)
    memory._start_idx = processed - raw_count
    memory._end_idx = processed
    memory._step_idx = max(1, (processed + window - 1) // window)
    memory._is_full_window = raw_count == 0
    memory._interleave_remainder = raw_count % ratio
    memory._interleave_compression_ratio = ratio
    memory._compression_ratio = ratio
    memory._select_cache_mode()
    device = model.model.embed_tokens.weight.device
    if raw_count:
        roles = window_roles(raw_count, ratio, device)
        memory._beacon_indices = roles
        memory._window_roles = roles.bool()
        memory._window_raw_indices = (roles == 0).nonzero().flatten()
    for index in range(len(model.model.layers)):
        attn, raw_blocks, beacon_blocks, beacon = _layer_pages(model, index, raw_layers, beacon_layers, raw_table,
                                                               beacon_table, ratio)
        key, value = beacon.read(beacon_blocks, beacon_count)
        memory.beacon_activations[index] = tuple(x[:, :, :history_count] if history_count else None
                                                 for x in (key, value))
        memory.window_beacon_activations[index] = tuple(
            x[:, :, history_count:] if beacon_count > history_count else None for x in (key, value))
        if model.config.beacon_sink_size:
            memory.sink_activations[index] = beacon.read_sink(beacon_blocks[0], attn.num_key_value_heads,
                                                              attn.head_dim)
        memory.raw_activations[index] = RawPages(raw_layers[index].kv_cache).read(
            raw_blocks, processed - raw_count, raw_count)


def flush_memory(model, previous, current, raw_layers, beacon_layers, raw_table, beacon_table):
    """Append the beacons and raw tokens produced since `previous` to the pages
    (paged_model.py:55-84)."""
    memory = model.memory
    ratio, window = model.config.beacon_ratio[0], model.config.beacon_window
    old_beacons = previous // ratio
    raw_start = flush_raw_start(previous, current, window)
    for index in range(len(model.model.layers)):
        _, raw_blocks, beacon_blocks, pages = _layer_pages(model, index, raw_layers, beacon_layers, raw_table,
                                                           beacon_table, ratio)
        if current // ratio > old_beacons:
            tensors = []
            for kind in (0, 1):
                parts = [group[index][kind] for group in (memory.beacon_activations, memory.window_beacon_activations)
                         if group[index][kind] is not None]
                if sum(p.shape[2] for p in parts) != current // ratio:
                    raise RuntimeError('Beacon count does not match the raw-token cursor.')
                tensors.append(_suffix(parts, old_beacons))
            pages.append(beacon_blocks, old_beacons, *tensors)
        if model.config.beacon_sink_size:
            pages.write_sink(beacon_blocks[0], *memory.sink_activations[index])
        if current > raw_start:
            key, value = memory.raw_activations[index]
            RawPages(raw_layers[index].kv_cache).write(raw_blocks, raw_start, key[:, :, -(current - raw_start):],
                                                       value[:, :, -(current - raw_start):])


def _suffix(parts, start):
    """Rows start.. of the concatenation of `parts` along dim 2, concatenating
    only the parts that hold them."""
    kept, offset = [], 0
    for part in parts:
        n = part.shape[2]
        if offset + n > start:
            kept.append(part[:, :, max(start - offset, 0):])
        offset += n
    return kept[0] if len(kept) == 1 else torch.cat(kept, dim=2)


def release_workspace_views(memory):
    """Retain no request KV in the model after it is committed to pages
    (paged_model.py:87-89)."""
    for name in ('sink_activations', 'raw_activations', 'beacon_activations', 'window_beacon_activations'):
        setattr(memory, name, [(None, None) for _ in range(memory.config.num_hidden_layers)])


@dataclass(frozen=True)
class PageGeometry:
    """Page sizes create_page_layers allocates (backend.py:108-131)."""
    raw_block: int
    beacon_block: int
    page_bytes: int
    raw_width: int
    max_width: int
    token_ratio: int

    def storage_block_size(self, width):
        """Rows of `width` elements per beacon page (BeaconSpec.storage_block_size,
        backend.py:17-19)."""
        return self.beacon_block // self.token_ratio + (2 * self.raw_width + width - 1) // width

    def real_page_size_bytes(self, width):
        return self.storage_block_size(width) * width * 2


def page_geometry(raw_width, max_width, ratio, raw_block=16):
    """Raw block 16 tokens; a beacon page has the raw page's byte size and holds
    beacon_block raw tokens' worth of beacons (backend.py:108-118)."""
    page_bytes = raw_block * 2 * raw_width * 2
    beacon_block = (((page_bytes // 2 - 2 * raw_width) // max_width) * ratio // raw_block) * raw_block
    if beacon_block < raw_block or beacon_block % ratio:
        raise ValueError('Cannot represent the selected token ratio in compact pages.')
    return PageGeometry(raw_block, beacon_block, page_bytes, raw_width, max_width, ratio)


def model_page_geometry(model):
    """page_geometry for a model's layers (backend.py:108-116)."""
    first = model.model.layers[0].self_attn
    max_width = max(layer.self_attn.beacon_k_up_proj.in_features + layer.self_attn.beacon_v_up_proj.in_features
                    for layer in model.model.layers)
    return page_geometry(first.num_key_value_heads * first.head_dim, max_width, model.config.beacon_ratio[0])
