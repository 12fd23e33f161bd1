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
   ReconstructionCache.materialize (reconstruction kernel for the latent parts).
4. bf16-exact RoPE that leaves beacon K unrotated (prefill RoPE kernel).
5. Causal attention (MFMA flash-attention kernel), then o_proj_with_beacon.

The module's own q/k/v/o projections are called as they are (model layers);
everything from the latents onwards runs in the HIP library.
"""
import torch

from . import kernels
from .latent_decode import uses_latent_decode
from .memory import ReconstructionCache, ReconstructionCacheUpdate, is_block_diagonal
from .prefill_ops import fused_prefill_rope


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
    if 'k' in config.beacon_param:
        down = attention.beacon_kv_down_proj if shared else attention.beacon_k_down_proj
        key_latent = _low_rank(attention, hidden, rows, down, attention.beacon_k_up_proj, k, Hk)
    if 'v' in config.beacon_param:
        down = attention.beacon_kv_down_proj if shared else attention.beacon_v_down_proj
        value_latent = _low_rank(attention, hidden, rows, down, attention.beacon_v_up_proj, v, Hk)
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


def prefill_forward(attention, hidden_states, position_ids, past_key_value):
    """(attn_output [B, L, hidden], None, cache update) for a prefill window
    over a ReconstructionCache (modeling_llama.py:1632-1750, join_prefill)."""
    past_key, past_value, beacon_size, beacon_indices = past_key_value
    if not isinstance(past_key, ReconstructionCache):
        raise ValueError('prefill_forward expects a latent (ReconstructionCache) past')
    B, L, _ = hidden_states.shape
    Hq, Hk, D = attention.num_heads, attention.num_key_value_heads, attention.head_dim
    metadata = getattr(attention, '_prefill_metadata', None)
    q, k, v, key_latent, value_latent = project_with_beacon(attention, hidden_states, beacon_size, beacon_indices,
                                                            metadata)
    current_k, current_v = k.transpose(1, 2), v.transpose(1, 2)           # BHSD views
    update = current_k, current_v, beacon_size, beacon_indices
    if key_latent is not None or value_latent is not None:
        update = ReconstructionCacheUpdate(current_k, current_v, beacon_size, beacon_indices,
                                           _pack(attention, key_latent), _pack(attention, value_latent))
        if metadata is not None:
            update.raw_indices = metadata.raw_indices
    key_states = past_key.materialize(attention, current_k)
    value_states = past_value.materialize(attention, current_v)
    query_states = q.view(B, L, Hq, D).transpose(1, 2)
    if metadata is None:
        raise ValueError('prefill_forward needs the prefill metadata (prefill_ops.prepare_metadata)')
    rotated = fused_prefill_rope(query_states, key_states, attention.rotary_emb, metadata,
                                 attention.config.beacon_sink_size)
    if rotated is None:
        raise ValueError('prefill RoPE needs bf16 device tensors and a standard rotary table')
    q_rot, k_rot = rotated
    scale = getattr(attention, 'softmax_scale', None) or D ** -0.5
    out, _ = kernels.prefill_attention(q_rot.transpose(1, 2), k_rot.transpose(1, 2), value_states.transpose(1, 2),
                                       scale, causal=True)
    out = out.reshape(B, L, Hq * D)
    return attention.o_proj_with_beacon(out, beacon_size, beacon_indices), None, update
