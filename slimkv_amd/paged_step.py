"""One decode step of a Llama attention layer for a batch of requests whose
KV lives in vLLM's pages, on gfx950.

The reference serves every request of a decode batch on its own
(SlimKVLlamaForCausalLM._paged_forward, slimkv/vllm_plugin/model.py:114-142):
restore_memory rebuilds the request's memory from its pages
(vllm_plugin/paged_model.py:7-52), the batch-1 model runs the step -- in every
layer fa2_decode.decode (slimkv/llama3/fa2_decode.py:77-166) over
[sink | raw window rows | new token] and [history beacons | window beacons |
new beacon] -- and flush_memory appends what the step produced
(paged_model.py:55-84).  paged_decode_layer runs one layer of that step for all
requests at once and touches the pages in place:

1. the step's q / new K / new V (and, on an insertion step, the new beacon's
   latents) from the module's own projections, as fa2_decode.decode makes them;
2. the new beacon's latents appended to the beacon pages at beacon P // ratio
   (P = tokens the request had processed), where flush_memory appends them;
3. the raw set gathered into a dense buffer -- the sink from the root page,
   the open window's raw rows from the raw pages (positions
   P - P % window .. P - 1), the new token -- and its keys rotated at the
   memory's slot positions (sink 0, raw row j of the window at
   sink + history + j + j // ratio, the new token at the slot after the
   memory), the bf16 RoPE of the reference; the same launch
   (slimkv_paged_step_rows) makes step 5's writes;
4. the fused latent decode with the beacon rows read through their pages
   (slimkv_paged_latent_decode; queries rotated in the kernel at the new
   token's slots, the raw query of an insertion step not seeing the new
   beacon);
5. flush_memory's writes: the new token's K (before RoPE) and V at raw
   position P unless the step completes the window (its raw rows are then
   dropped), and, while a request has no history yet, the new token as its
   sink (update_memory, slimkv/llama3/memory.py:248-253).

Requests are grouped by whether the step inserts a beacon (one query row or
two); plan_paged_step gives the groups and paged_decode_layer runs one group.
The page formats are the reference's (BeaconPageLayout, raw pages
[blocks, 16, 2, Hkv, D]); the configuration is the one the reference's native
paged mode admits (model.py:52-61): aligned windows of a multiple of 16
tokens, interleaved full-coverage beacons, at most one sink token, beacon K
without RoPE.
"""
from dataclasses import dataclass, field

import torch

from . import kernels
from .memory import is_block_diagonal
from .paged_cache import BeaconPageLayout


@dataclass
class PagedStepGroup:
    """The requests of a decode step that insert `size` beacons (0 or 1).
    Host integers per request and the device tensors the layer reads."""
    size: int
    index: list                      # positions of these requests in the step's batch
    processed: list                  # tokens processed before the step (P)
    window: int
    ratio: int
    sink: int
    raw_counts: list = field(default_factory=list)
    histories: list = field(default_factory=list)
    max_raw: int = 0                 # rows of the dense raw set (sink, longest window, new token)
    max_beacons: int = 0             # beacon rows the decode reads for the longest request
    rows_total: int = 0              # beacon rows over the group
    tensors: dict = field(default_factory=dict)


def step_size(processed, window, ratio):
    """Beacons the decode step of a request inserts after its token: one when
    the token completes a group of `ratio` raw tokens of the window
    (slimkv/llama3/memory.py:122-124, interleave remainder (P % window) % ratio)."""
    return ((processed % window) % ratio + 1) // ratio


def plan_paged_step(processed, window, ratio, sink, device):
    """Groups of one decode step (by inserted beacons), with the memory's slot
    positions and the page offsets of every request (restore_memory's counts,
    paged_model.py:12-15)."""
    if window % 16 or window % ratio or sink not in (0, 1):
        raise ValueError('paged decode needs windows of a multiple of 16 and of the ratio, and at most one sink')
    groups = []
    for size in (0, 1):
        idx = [i for i, p in enumerate(processed) if step_size(p, window, ratio) == size]
        if not idx:
            continue
        P = [int(processed[i]) for i in idx]
        if min(P) <= 0:
            raise ValueError('paged decode follows a prefill: every request has processed tokens')
        g = PagedStepGroup(size, idx, P, window, ratio, sink)
        g.raw_counts = [p % window for p in P]
        g.histories = [p // window * (window // ratio) for p in P]
        L = 1 + size
        max_raw = sink + max(g.raw_counts) + 1
        raw_pos = torch.zeros(len(P), max_raw, dtype=torch.int64)
        q_pos = torch.zeros(len(P), L, dtype=torch.int64)
        for b, (p, rc, hist) in enumerate(zip(P, g.raw_counts, g.histories)):
            beacons_in_window = rc // ratio
            mem = sink + hist + rc + beacons_in_window        # memory slots before the new token
            j = torch.arange(rc)
            raw_pos[b, sink:sink + rc] = sink + hist + j + j // ratio
            raw_pos[b, sink + rc] = mem
            q_pos[b] = mem + torch.arange(L)
        completes = [(p + 1) % window == 0 for p in P]
        t = dict(
            q_positions=q_pos, raw_positions=raw_pos,
            raw_lengths=torch.tensor([sink + rc + 1 for rc in g.raw_counts], dtype=torch.int32),
            window_start=torch.tensor([p - rc for p, rc in zip(P, g.raw_counts)], dtype=torch.int64),
            raw_count=torch.tensor(g.raw_counts, dtype=torch.int32),
            beacon_start=torch.tensor([p // ratio for p in P], dtype=torch.int64),
            lat_lengths=torch.tensor([p // ratio + size for p in P], dtype=torch.int32),
            raw_write_end=torch.tensor([p + (0 if c else 1) for p, c in zip(P, completes)], dtype=torch.int32),
            sink_update=torch.tensor([sink > 0 and h == 0 for h in g.histories], dtype=torch.uint8),
            index=torch.tensor(idx, dtype=torch.int64))
        g.tensors = {k: v.to(device) for k, v in t.items()}
        g.max_raw = max_raw
        g.max_beacons = max(p // ratio + size for p in P)
        g.rows_total = sum(p // ratio + size for p in P)
        groups.append(g)
    return groups


def _tables(rope, device):
    cos, sin = rope.cos_cached, rope.sin_cached
    if cos.device != device or cos.dtype != torch.float32:
        cos, sin = cos.to(device, torch.float32), sin.to(device, torch.float32)
    return cos, sin


def paged_decode_layer(attention, hidden, group, raw_pages, beacon_pages, raw_tables, beacon_tables, block_size,
                       status=None, raw_splits=0, lat_splits=0):
    """Attention output [B, 1 + size, hidden] of one layer's decode step for a
    group of requests (plan_paged_step), their pages read and written in
    place.  hidden [B, 1 + size, hidden_size] (the raw token, then the new
    beacon); raw_pages [blocks, 16, 2, Hkv, D]; beacon_pages [pages,
    page_elements] in BeaconPageLayout(block_size, ratio, key_rank,
    value_rank, Hkv * D); raw_tables / beacon_tables [B, T] int64 block tables
    of the group's requests.  Index errors land in `status` (device int32) or
    raise IndexError after the step (one host synchronisation).  raw_splits /
    lat_splits: key splits of the decode (0: the library's plan)."""
    config = attention.config
    size = group.size
    B, L, _ = hidden.shape
    if L != 1 + size or B != len(group.index):
        raise ValueError('hidden must be [requests of the group, 1 + size, hidden]')
    heads, kv_heads, dim = attention.num_heads, attention.num_key_value_heads, attention.head_dim
    # projections of the step (fa2_decode.py:88-100)
    raw_hidden = hidden[:, :1]
    q = attention.q_proj(hidden)
    if size and 'q' in config.beacon_param:
        q = torch.cat([q[:, :1], attention.beacon_q_proj(hidden[:, 1:])], dim=1)
    q = q.reshape(B, L, heads, dim)
    new_k = attention.k_proj(raw_hidden).reshape(B, kv_heads, dim)
    new_v = attention.v_proj(raw_hidden).reshape(B, kv_heads, dim)
    kl = vl = None
    if size:
        kl, vl = _beacon_latents(attention, hidden[:, 1:])
    own_status = status is None
    if own_status:
        status = torch.zeros(1, dtype=torch.int32, device=hidden.device)
    out = _attend(attention, q, new_k, new_v, kl, vl, group, raw_pages, beacon_pages, raw_tables, beacon_tables,
                  block_size, status, raw_splits, lat_splits)
    if own_status:
        kernels.check_status(status)
    output = out.reshape(B, L, attention.hidden_size)
    # roles of the step's rows (raw token, then its beacon) for the beacon O projection
    roles = torch.arange(L, device=hidden.device) if size else None
    return attention.o_proj_with_beacon(output, size, roles)


def _beacon_latents(attention, beacon_hidden):
    """The new beacons' K/V latents [B, 1, rank] (the module's down projections)."""
    shared = attention._use_shared_kv_down_proj()
    kd = attention.beacon_kv_down_proj if shared else attention.beacon_k_down_proj
    vd = attention.beacon_kv_down_proj if shared else attention.beacon_v_down_proj
    return kd(beacon_hidden).contiguous(), vd(beacon_hidden).contiguous()


def _attend(attention, q, new_k, new_v, kl, vl, group, raw_pages, beacon_pages, raw_tables, beacon_tables,
            block_size, status, raw_splits, lat_splits):
    """Steps 2-5 of the module docstring for one group: q [B, L, Hq, D],
    new_k / new_v [B, Hkv, D], kl / vl [B, 1, rank] on an insertion step.
    Returns the attention output [B, L, Hq, D]."""
    config = attention.config
    size, t = group.size, group.tensors
    if not getattr(config, 'beacon_skip_rope_for_beacon_k', False):
        raise ValueError('paged latent decode reads beacon K without RoPE (model.py:45-46)')
    uk, uv = attention.beacon_k_up_proj, attention.beacon_v_up_proj
    kv_heads, dim = attention.num_key_value_heads, attention.head_dim
    layout = BeaconPageLayout(block_size, group.ratio, uk.in_features, uv.in_features, kv_heads * dim)
    device = q.device
    raw_tables = raw_tables.to(device=device, dtype=torch.long)
    beacon_tables = beacon_tables.to(device=device, dtype=torch.long)

    # 2. the new beacon's latents appended at beacon P // ratio
    if size:
        kernels.beacon_pages(beacon_pages, beacon_tables, kl, vl, slots=layout.slots, key_rank=layout.key_rank,
                             value_rank=layout.value_rank, sink_elements=layout.sink_elements, start=0, count=1,
                             to_pages=True, lengths=t['lat_lengths'], status=status, starts=t['beacon_start'])

    # 3. the raw set -- sink (root page), the window's raw rows (raw pages), the
    # new token -- with K rotated at the memory's slots, and flush_memory's raw
    # and sink writes (paged_model.py:55-84, memory.py:248-253), in one launch:
    # the decode reads the dense raw set, not the pages it writes
    cos, sin = _tables(attention.rotary_emb, device)
    raw_k_rot, raw_v = kernels.paged_step_rows(
        raw_pages, raw_tables, beacon_pages, beacon_tables, new_k, new_v, t['window_start'],
        t['raw_count'], t['raw_positions'], cos, sin, group.max_raw, group.sink, flush=True,
        raw_write_end=t['raw_write_end'], sink_update=t['sink_update'], status=status)

    # 4. the fused latent decode, beacon rows through their pages
    bd = is_block_diagonal(uk.weight, kv_heads) and is_block_diagonal(uv.weight, kv_heads)
    out, _ = kernels.paged_latent_decode(
        q, raw_k_rot, raw_v, beacon_pages, beacon_tables, t['lat_lengths'], group.max_beacons,
        layout, uk.weight, uv.weight, 1.0 / dim ** 0.5, up_k_bias=uk.bias, up_v_bias=uv.bias, block_diagonal=bd,
        lat_causal=bool(size), q_positions=t['q_positions'], cos=cos, sin=sin, raw_lengths=t['raw_lengths'],
        rows_total=group.rows_total, status=status, raw_splits=raw_splits, lat_splits=lat_splits)
    return out
