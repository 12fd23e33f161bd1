"""Append-only decode state of the latent cache, kept on the GPU.

The decode step of the reference re-concatenates the raw window and the
window latents every token (LlamaMemory.update_memory, slimkv/llama3/memory.py:233-278,
through cat_tensor) and rebuilds roles and raw indices on the host
(LlamaMemory._step fast path, :101-162).  Here the same schedule drives
preallocated per-layer buffers instead:

  raw rows     [B, raw_capacity, Hkv, D]: sink | window raw tokens | current token,
               K stored already rotated at its key position (rotated once, when
               appended, as StaticDecode keeps `rotated_k`, static_decode.py:150-160)
  latent rows  [B, latent_capacity, R]: history beacons | window beacons

A window rollover only relabels counts (the window's beacons become history,
its raw rows are dropped); nothing is copied.  The per-batch row counts also
live in device int32 tensors, so a captured HIP graph of the decode step
stays valid as the cache grows.
"""
from dataclasses import dataclass

import torch

from . import kernels


@dataclass
class StepPlan:
    size: int                 # beacons inserted after the raw token (0 or 1)
    full: bool                # the step completes the window
    raw_slot: int             # raw row of the new token
    latent_slot: int          # latent row of the new beacon (when size)
    position: int             # key position of the new raw token
    key_length: int           # keys the step attends over, as the reference counts them


class DecodeSchedule:
    """Window bookkeeping of one decode step (slimkv/llama3/memory.py:101-162)
    with a single compression ratio and stride == window."""

    def __init__(self, window, ratio, sink, *, processed, start, roles=(), remainder=0, full=True, history=0):
        if ratio <= 0 or window % ratio:
            raise ValueError('the window must hold a whole number of beacons')
        self.window, self.ratio, self.sink = window, ratio, sink
        self.processed, self.start = processed, start
        self.roles = list(roles)
        self.remainder, self.is_full = remainder, full
        self.history = history

    @classmethod
    def after_prefill(cls, window, ratio, sink, processed):
        """State after prefilling `processed` tokens (paged_model.py:13-35
        restores the same counts): full windows are history, the open window
        holds processed % window raw tokens with a beacon after every `ratio`."""
        raw = processed % window
        roles = []
        for i in range(raw):
            roles.append(0)
            if (i + 1) % ratio == 0:
                roles.append(1)
        return cls(window, ratio, sink, processed=processed, start=processed - raw, roles=roles,
                   remainder=raw % ratio, full=raw == 0, history=processed // window * (window // ratio))

    @property
    def window_raw(self):
        return 0 if self.is_full else self.roles.count(0)

    @property
    def window_beacons(self):
        return 0 if self.is_full else self.roles.count(1)

    def step(self):
        end = self.processed + 1
        full = end >= self.start + self.window
        roles = [] if self.is_full else list(self.roles)
        past_keys = self.sink + self.history + len(roles)
        raw_rows = self.sink + roles.count(0)
        latent_rows = self.history + roles.count(1)
        size = (self.remainder + 1) // self.ratio
        self.remainder = (self.remainder + 1) % self.ratio
        roles += [0] + [1] * size
        plan = StepPlan(size, full, raw_rows, latent_rows, past_keys, past_keys + 1 + size)
        self.roles = roles
        self.is_full = full
        if full:
            self.start += self.window
            self.history += roles.count(1)
        self.processed = end
        return plan


class LatentDecodeCache:
    """Preallocated raw and latent rows of one layer for a batch of sequences
    that advance in lockstep.  `prepare` (host, before a step or a graph
    replay) publishes the step's slots and lengths into device tensors;
    `write` and `attend` read only those, so a captured step stays valid."""

    def __init__(self, batch, kv_heads, head_dim, key_rank, value_rank, raw_capacity, latent_capacity, device,
                 dtype=torch.bfloat16):
        self.kv_heads, self.head_dim = kv_heads, head_dim
        self.raw_k = torch.zeros(batch, raw_capacity, kv_heads, head_dim, dtype=dtype, device=device)
        self.raw_v = torch.zeros_like(self.raw_k)
        self.lat_k = torch.zeros(batch, max(latent_capacity, 1), key_rank, dtype=dtype, device=device)
        self.lat_v = torch.zeros(batch, max(latent_capacity, 1), value_rank, dtype=dtype, device=device)
        self.plain_k = torch.zeros_like(self.raw_k)     # the same rows unrotated (the reference's raw K)
        self.sink = 0
        self.raw = 0            # window raw rows after the sink
        self.history = 0
        self.window = 0         # window beacon rows after the history
        self.raw_index = torch.zeros(1, dtype=torch.long, device=device)
        self.latent_index = torch.zeros(1, dtype=torch.long, device=device)
        self.raw_lengths = torch.zeros(batch, dtype=torch.int32, device=device)
        self.lat_lengths = torch.zeros(batch, dtype=torch.int32, device=device)
        # slot errors of kernels.decode_qkv appends (prepare() already refuses
        # a step past the capacity on the host)
        self.status = torch.zeros(1, dtype=torch.int32, device=device)

    def load(self, sink_k, sink_v, raw_k, raw_v, history_k, history_v, window_k, window_v, cos=None, sin=None,
             positions=None):
        """Fill from a prefilled cache: K/V rows BSHD [B, n, Hkv, D] unrotated,
        latents [B, n, R]; any part may be None.  K is rotated here at
        `positions` [B, sink + raw] (int64) when `cos`/`sin` are given."""
        def put(dst, start, src):
            if src is not None and src.shape[1]:
                dst[:, start:start + src.shape[1]].copy_(src)
            return 0 if src is None else src.shape[1]
        self.sink = put(self.plain_k, 0, sink_k)
        put(self.raw_v, 0, sink_v)
        self.raw = put(self.plain_k, self.sink, raw_k)
        put(self.raw_v, self.sink, raw_v)
        n = self.sink + self.raw
        if n:
            plain = self.plain_k[:, :n]
            if cos is not None:
                q = plain.new_zeros(plain.shape[0], self.kv_heads, 1, self.head_dim)
                # rows rotate at their own positions: every row is a "tail" slot
                _, rot = kernels.rope_decode(q, plain.transpose(1, 2), cos, sin, positions[:, n - 1:n].contiguous(),
                                             positions[0, :n - 1].contiguous(), 0, 0)
                self.raw_k[:, :n].copy_(rot.transpose(1, 2))
            else:
                self.raw_k[:, :n].copy_(plain)
        self.history = put(self.lat_k, 0, history_k)
        put(self.lat_v, 0, history_v)
        self.window = put(self.lat_k, self.history, window_k)
        put(self.lat_v, self.history, window_v)

    def prepare(self, plan):
        """Slots and attention lengths of the step (raw rows incl. the new token,
        latents incl. the new beacon); called outside any captured graph."""
        if plan.raw_slot + 1 > self.raw_k.shape[1] or plan.latent_slot + plan.size > self.lat_k.shape[1]:
            raise ValueError('decode cache capacity exceeded')
        self.raw_index.fill_(plan.raw_slot)
        self.latent_index.fill_(plan.latent_slot)
        self.raw_lengths.fill_(plan.raw_slot + 1)
        self.lat_lengths.fill_(plan.latent_slot + plan.size)

    def write(self, raw_k_rot, raw_k, raw_v, lat_k=None, lat_v=None):
        """Store the step's rows at the prepared slots (device indices):
        K rotated and unrotated [B, 1, Hkv, D], V, latents [B, n, R]."""
        self.raw_k.index_copy_(1, self.raw_index, raw_k_rot)
        self.plain_k.index_copy_(1, self.raw_index, raw_k)
        self.raw_v.index_copy_(1, self.raw_index, raw_v)
        if lat_k is not None:
            self.write_latents(lat_k, lat_v)

    def write_latents(self, lat_k, lat_v):
        """Store the step's beacon latents [B, n, R] at the prepared slots
        (when the raw rows were appended by kernels.decode_qkv)."""
        self.lat_k.index_copy_(1, self.latent_index, lat_k)
        self.lat_v.index_copy_(1, self.latent_index, lat_v)

    def commit(self, plan, refresh_sink=False, cos=None, sin=None):
        """update_memory (memory.py:233-278): keep the raw row and beacons, or
        roll the window over (its beacons become history, its raw rows go).
        `refresh_sink`: the first-window sink update (memory.py:248-253) -- the
        sink becomes the newest raw token, its K rotated at key position 0."""
        if refresh_sink and self.sink:
            slot = plan.raw_slot
            self.plain_k[:, :1].copy_(self.plain_k[:, slot:slot + 1])
            self.raw_v[:, :1].copy_(self.raw_v[:, slot:slot + 1])
            zero = torch.zeros(self.raw_k.shape[0], 1, dtype=torch.long, device=self.raw_k.device)
            q = self.plain_k.new_zeros(self.raw_k.shape[0], self.kv_heads, 1, self.head_dim)
            _, k0 = kernels.rope_decode(q, self.plain_k[:, :1].transpose(1, 2), cos, sin, zero, None, 0, 0)
            self.raw_k[:, :1].copy_(k0.transpose(1, 2))
        if plan.full:
            self.history += self.window + plan.size
            self.window = 0
            self.raw = 0
        else:
            self.raw += 1
            self.window += plan.size

    def cache_bytes(self):
        """Logical persistent K/V bytes per group (memory.py:280-287)."""
        b = self.raw_k.shape[0]
        row = 2 * self.kv_heads * self.head_dim * self.raw_k.element_size()
        lat = (self.lat_k.shape[-1] + self.lat_v.shape[-1]) * self.lat_k.element_size()
        return {'sink': b * self.sink * row, 'raw': b * self.raw * row,
                'beacon': b * self.history * lat, 'window_beacon': b * self.window * lat}

    def attend(self, q, up_k, up_v, scale, *, q_positions, cos, sin, size, up_k_bias=None, up_v_bias=None,
               out=None, lse=None, workspace=None):
        """The decode attention of the step over the full-capacity views, the
        lengths bounding each sequence (graph-capturable)."""
        return kernels.latent_decode(q, self.raw_k, self.raw_v, self.lat_k, self.lat_v, up_k, up_v, scale,
                                     up_k_bias=up_k_bias, up_v_bias=up_v_bias,
                                     block_diagonal=_block_diagonal(up_k, up_v, self.kv_heads),
                                     lat_causal=bool(size), q_positions=q_positions, cos=cos, sin=sin,
                                     raw_lengths=self.raw_lengths, lat_lengths=self.lat_lengths,
                                     out=out, lse=lse, workspace=workspace)


def _block_diagonal(up_k, up_v, kv_heads):
    from .memory import is_block_diagonal
    return is_block_diagonal(up_k, kv_heads) and is_block_diagonal(up_v, kv_heads)
