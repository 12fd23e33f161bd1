"""Window prefill of one attention layer over a latent cache, on gfx950.

Mirrors the latent-cache ("join prefill") branch of LlamaFlashAttention2.forward
(slimkv/llama3/modeling_llama.py:1632-1750) with its helpers
qkv_proj_with_beacon (:1291-1345), _incremental_cache (:1347-1367) and
_apply_rotary_with_beacon (:1108-1216, prefill-metadata case):

1. Q/K/V of the window.  Raw rows use q/k/v_proj; beacon rows use beacon_q_proj
   and the low-rank K/V (latent = down(h), full = up(latent)).  The latents of
   the beacon rows come from the MFMA down-projection kernel (only the beacon
   rows are projected) and their full-dimensional K/V from the MFMA
   reconstruction kernel scattered straight into the window's K/V rows.
2. The cache update carries those latents, packed as the reference packs them.
3. The key/value workspace [sink | up(history) | window | current] is built by
   ReconstructionCache.materialize (reconstruction kernel for the latent parts),
   or -- for a stream of prefill windows with a PrefillHistory attached --
   read from append-only storage that already holds [sink | up(history)]: the
   window is written after it, and once the window is attended only its new
   beacons are rebuilt onto the history (the reference rebuilds the whole
   history every window, modeling_llama.py:1677-1681, from a latent history it
   concatenates anew, slimkv/llama3/memory.py:255-267).
4. bf16-exact RoPE that leaves beacon K unrotated: the keys by the prefill
   RoPE kernel, the queries inside the attention kernel as it loads them
   (the same bits as rotating them first, without writing them out and
   reading them back).
5. Causal attention (MFMA flash-attention kernel), then o_proj_with_beacon.

The module's own q/k/v/o projections are called as they are (model layers);
everything from the latents onwards runs in the HIP library.
"""
import torch

from . import kernels
from .latent_decode import uses_latent_decode
from .memory import ReconstructionCache, ReconstructionCacheUpdate, is_block_diagonal


def _rows_where(current, role):
    return (current == role).nonzero().flatten()


def _beacon_rows(metadata, current):
    return metadata.beacon_indices if metadata is not None else (current != 0).nonzero().flatten()


def _blocks(weight, kv_heads):
    """Diagonal block count of a down-projection weight [R, K] whose input
    features are per KV head (every off-diagonal [R/Hk, K/Hk] block zero), else
    1.  Cached on the tensor per (version, kv_heads)."""
    cached = getattr(weight, '_slimkv_down_blocks', None)
    if cached is not None and cached[:2] == (weight._version, kv_heads):
        return cached[2]
    out_features, in_features = weight.shape
    result = 1
    if kv_heads > 1 and out_features % kv_heads == 0 and in_features % kv_heads == 0:
        blocks = weight.detach().reshape(kv_heads, out_features // kv_heads, kv_heads, in_features // kv_heads)
        mask = ~torch.eye(kv_heads, dtype=torch.bool, device=weight.device)[:, None, :, None]
        if not bool((blocks.abs() * mask).amax() > 0):
            result = kv_heads
    weight._slimkv_down_blocks = (weight._version, kv_heads, result)
    return result


def _low_rank(attention, hidden, rows, down, up, dest, heads):
    """latent = down(h[rows]) [B, n, R]; dest[:, rows] = up(latent) (BSHD view)."""
    latent = kernels.down_project(hidden, down.weight, rows, blocks=_blocks(down.weight, heads))
    kernels.reconstruct(latent, up.weight, up.bias, kv_heads=heads, out=dest, dst_rows=rows,
                        block_diagonal=is_block_diagonal(up.weight, heads))
    return latent


def _low_rank_pair(hidden, rows, downs, ups, dests, heads):
    """_low_rank for K and V together: both down-projections in one launch,
    then both reconstructions in one (the same bits as one at a time)."""
    latents = kernels.down_project_pair(
        *({'x': hidden, 'weight': d.weight, 'rows': rows, 'blocks': _blocks(d.weight, heads)} for d in downs))
    kernels.reconstruct_pair(
        *({'latent': lat, 'weight': u.weight, 'bias': u.bias, 'kv_heads': heads, 'out': dst, 'dst_rows': rows,
           'block_diagonal': is_block_diagonal(u.weight, heads)} for lat, u, dst in zip(latents, ups, dests)))
    return latents


def project_with_beacon(attention, hidden, beacon_size, beacon_indices, metadata):
    """(q [B,L,Hq*D], k [B,L,Hk,D], v [B,L,Hk,D], key latents, value latents);
    qkv_proj_with_beacon with return_latents (modeling_llama.py:1291-1345)."""
    config = attention.config
    B, L, _ = hidden.shape
    Hk, D = attention.num_key_value_heads, attention.head_dim
    q = attention.q_proj(hidden)
    k = attention.k_proj(hidden).view(B, L, Hk, D)
    v = attention.v_proj(hidden).view(B, L, Hk, D)
    if beacon_size <= 0:
        return q, k, v, None, None
    current = beacon_indices[-L:]
    rows = _beacon_rows(metadata, current)
    replicas = metadata.replicas if metadata is not None else bool((current == 2).any())
    shared = attention._use_shared_kv_down_proj()
    if 'q' in config.beacon_param and rows.numel():
        q[:, rows] = attention.beacon_q_proj(hidden[:, rows])
    key_latent = value_latent = None
    k_down = attention.beacon_kv_down_proj if shared else getattr(attention, 'beacon_k_down_proj', None)
    v_down = attention.beacon_kv_down_proj if shared else getattr(attention, 'beacon_v_down_proj', None)
    if 'k' in config.beacon_param and 'v' in config.beacon_param:
        key_latent, value_latent = _low_rank_pair(hidden, rows, (k_down, v_down),
                                                  (attention.beacon_k_up_proj, attention.beacon_v_up_proj), (k, v), Hk)
    elif 'k' in config.beacon_param:
        key_latent = _low_rank(attention, hidden, rows, k_down, attention.beacon_k_up_proj, k, Hk)
    elif 'v' in config.beacon_param:
        value_latent = _low_rank(attention, hidden, rows, v_down, attention.beacon_v_up_proj, v, Hk)
    if replicas:
        # role 2 rows replicate the window's first beacons (parallel encoding)
        firsts, copies = _rows_where(current, 1), _rows_where(current, 2)
        for t in (q, k, v):
            t[:, copies] = t[:, firsts[:copies.numel()]]
    return q, k, v, key_latent, value_latent


def _pack(attention, latent):
    """_incremental_cache packing (modeling_llama.py:1355-1363) of the beacon
    rows' latents: [B, 1, n, R] for latent decode, else [B, Hk, n, r]."""
    if latent is None:
        return None
    batch, length, rank = latent.shape
    if uses_latent_decode(attention.config):
        return latent.unsqueeze(1)
    return latent.reshape(batch, length, attention.num_key_value_heads,
                          rank // attention.num_key_value_heads).transpose(1, 2).contiguous()


class PrefillHistory:
    """Append-only attention K/V of one layer for a stream of prefill windows:
    rows [0, sink + history) hold [sink | up(history beacons)] in the order
    the memory keeps them, keys as the attention reads them, and each window
    is written right after them.

    It replaces the per-window rebuild and rotation of the whole key set: the
    memory hands every window the sink and the latents of all earlier
    windows' beacons (ReconstructionCache), ReconstructionCache.materialize
    up-projects all of them again (modeling_llama.py:1677-1681) and the
    prefill RoPE then runs over every key (:1685-1690).  Here a window costs
    the rotation of its own rows and one reconstruction of its new beacons:
    history keys are beacon keys, which the prefill RoPE leaves unrotated
    (beacon_skip_rope_for_beacon_k), and the sink keeps the rotation it got
    in the first window, at positions 0 .. sink - 1, which full-coverage
    prefill positions (arange over the memory and the window,
    slimkv/memory.py:616) give it in every window.  The store follows the
    memory's update rules (slimkv/llama3/memory.py:233-278): the first
    window's first `sink` rows become the sink, and every window's beacon
    latents are appended to the history.  `capacity` bounds sink + history +
    window rows; BHSD buffers [batch, kv_heads, capacity, head_dim]."""

    def __init__(self, batch, kv_heads, head_dim, capacity, device, dtype=torch.bfloat16):
        self.k = torch.empty(batch, kv_heads, capacity, head_dim, dtype=dtype, device=device)
        self.v = torch.empty_like(self.k)
        self.sink = 0
        self.history = 0

    def reset(self):
        self.sink = self.history = 0

    def follows(self, past_key, past_value):
        """Whether the store holds exactly the memory's sink and history for
        this window (and the memory has no open window rows).  An empty past
        restarts the stream."""
        lengths = [0 if x is None else x.shape[2] for x in (past_key.sink, past_key.history)]
        if past_key.raw is not None or past_key.window is not None or past_value.raw is not None or \
                past_value.window is not None:
            return False
        if lengths == [0, 0]:
            self.reset()
            return True
        return lengths == [self.sink, self.history]

    def reserve(self, batch, length):
        """(base, key rows, value rows) of a window of `length` rows written
        after the held ones: BHSD views [B, Hk, length, D] at row `base`."""
        base = self.sink + self.history
        if base + length > self.k.shape[2] or batch != self.k.shape[0]:
            raise ValueError('prefill history capacity exceeded')
        return base, self.k[:, :, base:base + length], self.v[:, :, base:base + length]

    def sets(self, length):
        """The key and value sets [sink | history | window] as views."""
        end = self.sink + self.history + length
        return self.k[:, :, :end], self.v[:, :, :end]

    def append(self, attention, key_latent, value_latent, sink_size):
        """After the window is attended: the first window's leading rows stay
        as the sink, and the window's new beacons -- up(latents), the rows the
        memory appends to its history -- are rebuilt onto the history, over
        the window's own rows."""
        if self.history == 0 and self.sink == 0:
            self.sink = sink_size
        n = 0 if key_latent is None else key_latent.shape[1]
        if n:
            if value_latent is None or value_latent.shape[1] != n:
                raise ValueError('prefill history needs key and value latents of the same rows')
            heads = attention.num_key_value_heads
            base = self.sink + self.history
            if base + n > self.k.shape[2] or key_latent.shape[0] != self.k.shape[0]:
                raise ValueError('prefill history capacity exceeded')
            kernels.reconstruct_pair(
                *({'latent': lat, 'weight': up.weight, 'bias': up.bias, 'kv_heads': heads,
                   'out': dst[:, :, base:base + n].transpose(1, 2), 'block_diagonal': is_block_diagonal(up.weight, heads)}
                  for lat, up, dst in ((key_latent, attention.beacon_k_up_proj, self.k),
                                       (value_latent, attention.beacon_v_up_proj, self.v))))
            self.history += n


def _rope_tables(rope, query, keys, metadata, n):
    """fp32 (cos, sin) of the module's rotary table for the prefill RoPE of
    [B, n] keys; ValueError where the kernels do not apply (the conditions of
    fused_prefill_rope, prefill_ops.py:48-73)."""
    B = query.shape[0]
    if (not query.is_cuda or query.dtype != torch.bfloat16 or keys.dtype != query.dtype or query.shape[-1] % 16
            or type(rope).__name__ not in ('RotaryEmbedding', 'LinearScalingRotaryEmbedding', 'Llama3RotaryEmbedding')
            or metadata.positions.shape != (B, n) or n > rope.max_seq_len_cached
            or metadata.roles.numel() > keys.shape[2] or query.stride(-1) != 1 or keys.stride(-1) != 1):
        raise ValueError('prefill RoPE needs bf16 device tensors and a standard rotary table')
    cos, sin = rope.cos_cached, rope.sin_cached
    if cos.device != query.device or cos.dtype != torch.float32:
        cos, sin = cos.to(query.device, torch.float32), sin.to(query.device, torch.float32)
    return cos, sin


def prefill_forward(attention, hidden_states, position_ids, past_key_value, history=None):
    """(attn_output [B, L, hidden], None, cache update) for a prefill window
    over a ReconstructionCache (modeling_llama.py:1632-1750, join_prefill).
    `history` (or the module's `_slimkv_prefill_history`): a PrefillHistory
    kept across the stream's windows; it must follow the memory (an empty
    past restarts it), else ValueError."""
    past_key, past_value, beacon_size, beacon_indices = past_key_value
    if not isinstance(past_key, ReconstructionCache):
        raise ValueError('prefill_forward expects a latent (ReconstructionCache) past')
    B, L, _ = hidden_states.shape
    Hq, Hk, D = attention.num_heads, attention.num_key_value_heads, attention.head_dim
    metadata = getattr(attention, '_prefill_metadata', None)
    store = history if history is not None else getattr(attention, '_slimkv_prefill_history', None)
    if store is not None and not store.follows(past_key, past_value):
        raise ValueError('the prefill history store does not hold the memory\'s sink and history')
    q, k, v, key_latent, value_latent = project_with_beacon(attention, hidden_states, beacon_size, beacon_indices,
                                                            metadata)
    current_k, current_v = k.transpose(1, 2), v.transpose(1, 2)           # BHSD views
    update = current_k, current_v, beacon_size, beacon_indices
    if key_latent is not None or value_latent is not None:
        update = ReconstructionCacheUpdate(current_k, current_v, beacon_size, beacon_indices,
                                           _pack(attention, key_latent), _pack(attention, value_latent))
        if metadata is not None:
            update.raw_indices = metadata.raw_indices
    query = q.view(B, L, Hq, D)                                           # BSHD
    if metadata is None:
        raise ValueError('prefill_forward needs the prefill metadata (prefill_ops.prepare_metadata)')
    positions, roles = metadata.positions, metadata.roles
    # The queries are rotated inside the attention kernel as it loads them;
    # the keys by the prefill RoPE (beacon keys copied unrotated).
    if store is not None:
        base, key_rows, value_rows = store.reserve(B, L)
        cos, sin = _rope_tables(attention.rotary_emb, query, current_k, metadata, base + L)
        if roles.numel() != L:
            raise ValueError('the prefill history rotates the window\'s keys: roles must cover the window')
        # the window's keys rotated into the key set, its values copied into
        # the value set, in one launch
        kernels.rope_keys(current_k, cos, sin, positions[:, base:], roles, 0, out_k=key_rows, v=current_v,
                          out_v=value_rows)
        k_rot, value_states = store.sets(L)
    else:
        key_states = past_key.materialize(attention, current_k)
        value_states = past_value.materialize(attention, current_v)
        cos, sin = _rope_tables(attention.rotary_emb, query, key_states, metadata, key_states.shape[2])
        k_rot = kernels.rope_keys(key_states, cos, sin, positions, roles, attention.config.beacon_sink_size)
    scale = getattr(attention, 'softmax_scale', None) or D ** -0.5
    out, _ = kernels.prefill_attention(query, k_rot.transpose(1, 2), value_states.transpose(1, 2), scale,
                                       causal=True, q_positions=positions[:, -L:], cos=cos, sin=sin)
    out = out.reshape(B, L, Hq * D)
    if store is not None:
        store.append(attention, key_latent, value_latent, getattr(attention.config, 'beacon_sink_size', 0))
    return attention.o_proj_with_beacon(out, beacon_size, beacon_indices), None, update
