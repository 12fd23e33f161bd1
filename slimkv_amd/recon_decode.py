"""Drop-in for the decode step of the Llama attention classes over a latent
cache with the reconstruction backend, on gfx950: LlamaAttention.forward
(slimkv/llama3/modeling_llama.py:1402-1406), LlamaSdpaAttention.forward
(:1536-1541) and LlamaFlashAttention2.forward (:1648-1653) each materialise the
cache and run their own attention there (eager softmax, SDPA, flash_attn); the
same `eligible` / `forward` pair serves all three.

The reference (slimkv/llama3/modeling_llama.py:1384-1483) materialises the
whole past K/V from the latents (ReconstructionCache.materialize), appends the
step's rows, applies beacon-aware RoPE to every key (_apply_rotary_with_beacon,
:1108-1216; beacon keys rotated at their slot positions unless
beacon_skip_rope_for_beacon_k) and runs eager softmax attention.  Here one
slimkv_recon_decode call rebuilds each beacon's K tile by tile inside the
attention kernel (rotated at its slot position), keeps V latent until after the
weighted sum, and never writes the full-dimensional cache:

* raw set    [sinks ; raw tail ; the step's raw token], full-dim, K rotated at
             its slot positions by the decode RoPE kernel;
* beacon set [history ; window beacons ; the step's new beacon], latents, with
             slot positions: sinks + i for history row i, sinks + history + j
             for the window beacon at row j of the open window, and the new
             beacon's own position; on an insertion step the raw query does not
             see the new beacon (bottom-right causal over the beacon set).

Projections follow qkv_proj_with_beacon (:1291-1345) with the module's own
layers, and the returned cache update follows _incremental_cache (:1347-1367).
"""
import math

import torch

from . import kernels
from .latent_decode import uses_latent_decode
from .memory import ReconstructionCache, ReconstructionCacheUpdate, is_block_diagonal

_ROPE_TYPES = ('RotaryEmbedding', 'LinearScalingRotaryEmbedding', 'Llama3RotaryEmbedding')


def eligible(attention, hidden_states, past_key_value, output_attentions):
    """A decode step (one raw token, optionally followed by its beacon) over a
    latent cache read with the reconstruction backend."""
    return (getattr(attention.config, '_slimkv_decode_step', False)
            and not uses_latent_decode(attention.config)
            and isinstance(past_key_value[0], ReconstructionCache)
            and not attention.training and not output_attentions
            and hidden_states.shape[0] > 0 and hidden_states.shape[1] in (1, 2))


def _latent_rows(parts, batch, rank, device, dtype):
    """Concatenate latent parts ([B, 1, n, R] global or [B, Hkv, n, r] per-head
    packing) into one [B, N, R] tensor, one copy per part."""
    parts = [p for p in parts if p is not None and p.shape[2] > 0]
    if not parts:
        return None
    total = sum(p.shape[2] for p in parts)
    out = torch.empty(batch, total, rank, dtype=dtype, device=device)
    off = 0
    for p in parts:
        n = p.shape[2]
        if p.shape[1] == 1:
            out[:, off:off + n].copy_(p[:, 0])
        else:
            out[:, off:off + n].view(batch, n, p.shape[1], p.shape[3]).copy_(p.transpose(1, 2))
        off += n
    return out


def _pack(attention, latent):
    """_incremental_cache's packing of the step's beacon latent [B, n, R]."""
    if latent is None:
        return None
    batch, length, rank = latent.shape
    if uses_latent_decode(attention.config):
        return latent.unsqueeze(1).contiguous()
    return latent.reshape(batch, length, attention.num_key_value_heads,
                          rank // attention.num_key_value_heads).transpose(1, 2).contiguous()


def forward(attention, hidden_states, position_ids, past_key_value):
    """(attn_output [B, L, hidden], None, ReconstructionCacheUpdate)."""
    pk, pv, size, indices = past_key_value
    batch, length, _ = hidden_states.shape
    if size not in (0, 1) or length != size + 1:
        raise ValueError('Reconstruction decode expects one raw token followed by at most one Beacon.')
    uk, uv = attention.beacon_k_up_proj, attention.beacon_v_up_proj
    if not isinstance(uk, torch.nn.Linear) or not isinstance(uv, torch.nn.Linear):
        raise ValueError('Reconstruction decode requires Linear beacon up projections.')
    config = attention.config
    heads, kv_heads, dim = attention.num_heads, attention.num_key_value_heads, attention.head_dim
    rope = attention.rotary_emb
    if type(rope).__name__ not in _ROPE_TYPES or position_ids.shape[-1] > rope.max_seq_len_cached:
        raise ValueError('reconstruction decode needs a standard rotary table covering every position')
    cos, sin = rope.cos_cached, rope.sin_cached
    if cos.device != hidden_states.device or cos.dtype != torch.float32:
        cos, sin = cos.to(hidden_states.device, torch.float32), sin.to(hidden_states.device, torch.float32)

    # projections (qkv_proj_with_beacon, decode step: row 0 raw, row 1 beacon)
    raw_hidden = hidden_states[:, :1]
    q = attention.q_proj(hidden_states)
    k = attention.k_proj(hidden_states)
    v = attention.v_proj(hidden_states)
    kl = vl = None
    if size:
        beacon = hidden_states[:, 1:]
        if 'q' in config.beacon_param:
            q = torch.cat([q[:, :1], attention.beacon_q_proj(beacon)], dim=1)
        shared = attention._use_shared_kv_down_proj()
        kd = attention.beacon_kv_down_proj if shared else attention.beacon_k_down_proj
        vd = attention.beacon_kv_down_proj if shared else attention.beacon_v_down_proj
        kl, vl = kd(beacon), vd(beacon)
        k = torch.cat([k[:, :1], uk(kl)], dim=1)
        v = torch.cat([v[:, :1], uv(vl)], dim=1)
    current_k = k.view(batch, length, kv_heads, dim).transpose(1, 2)
    current_v = v.view(batch, length, kv_heads, dim).transpose(1, 2)
    update = ReconstructionCacheUpdate(current_k, current_v, size, indices, _pack(attention, kl),
                                       _pack(attention, vl))

    # raw set: sinks, raw tail, the step's raw token (K rotated at slot positions)
    sink_len = 0 if pk.sink is None else pk.sink.shape[2]
    history_len = 0 if pk.history is None else pk.history.shape[2]
    raw_parts_k = [x for x in (pk.sink, pk.raw, current_k[:, :, :1]) if x is not None]
    raw_parts_v = [x for x in (pv.sink, pv.raw, current_v[:, :, :1]) if x is not None]
    raw_k = torch.cat(raw_parts_k, dim=2) if len(raw_parts_k) > 1 else raw_parts_k[0]
    raw_v = torch.cat(raw_parts_v, dim=2) if len(raw_parts_v) > 1 else raw_parts_v[0]
    q_bhsd = q.view(batch, length, heads, dim).transpose(1, 2)
    q_pos = position_ids[:, -length:]
    if q_pos.shape[0] != batch:
        q_pos = q_pos.expand(batch, -1)
    _, raw_k = kernels.rope_decode(q_bhsd, raw_k, cos, sin, q_pos, pk.window_raw_indices, sink_len, history_len)

    # beacon set: history, window beacons, the step's new beacon (latents)
    rank_k, rank_v = uk.in_features, uv.in_features
    dev, dt = hidden_states.device, hidden_states.dtype
    lat_k = _latent_rows([pk.history, pk.window, None if kl is None else kl[:, None]], batch, rank_k, dev, dt)
    lat_v = _latent_rows([pv.history, pv.window, None if vl is None else vl[:, None]], batch, rank_v, dev, dt)
    beacon_pos = None
    if lat_k is not None and not getattr(config, 'beacon_skip_rope_for_beacon_k', False):
        parts = [sink_len + torch.arange(history_len, device=dev)]
        if pk.window is not None:
            roles = pk.window_roles.to(device=dev, dtype=torch.bool)
            parts.append(sink_len + history_len + roles.nonzero().flatten())
        if size:
            parts.append(position_ids[0, -1:].to(dev))
        beacon_pos = torch.cat(parts).to(torch.int64)[None].expand(batch, -1).contiguous()
    bd = is_block_diagonal(uk.weight, kv_heads) and is_block_diagonal(uv.weight, kv_heads)
    out, _ = kernels.recon_decode(
        q_bhsd.transpose(1, 2), raw_k.transpose(1, 2), raw_v.transpose(1, 2), lat_k, lat_v, uk.weight, uv.weight,
        1.0 / math.sqrt(dim), beacon_positions=beacon_pos, up_k_bias=uk.bias, up_v_bias=uv.bias, block_diagonal=bd,
        lat_causal=bool(size), q_positions=q_pos, cos=cos, sin=sin)
    output = out.reshape(batch, length, attention.hidden_size)
    return attention.o_proj_with_beacon(output, size, indices), None, update
