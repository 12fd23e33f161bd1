"""Drop-in for the attention core of slimkv/qwen2/modeling_qwen2.py on gfx950.

forward
    Qwen2FlashAttention2.forward (slimkv/qwen2/modeling_qwen2.py:887-978)
    with its Python signature, for batches without padding: the reference's
    memory drops the mask for flash_attention_2 when no token is padded
    (slimkv/memory.py:618-622) and this forward takes exactly that call.  The
    eager Qwen2Attention.forward (:699-779) always receives the memory's 4-D
    mask (slimkv/memory.py:626-633), which this forward refuses (ValueError),
    so it is not a drop-in there.  The module's own projections
    (qkv_proj_with_beacon) and output
    projection (o_proj_with_beacon) as they are; the beacon-aware RoPE of
    _apply_rotary_with_beacon (:602-635) in the bf16-exact prefill RoPE kernel;
    causal GQA attention over [past ; current] in the split-K decode kernel
    (one or two query rows) or the MFMA prefill kernel (longer windows).
flash_attention_forward
    Qwen2FlashAttention2._flash_attention_forward (:980-1040) for batches
    without padding (no mask, as above): bottom-right causal attention, BSHD
    in and out.

The past K/V stay pre-RoPE as the reference keeps them (the returned cache
holds the current step's keys before RoPE), so every step rotates the whole
key set at its slot positions, as the reference does.
"""
import math

import torch

from . import kernels

_ROPE_TYPES = ('RotaryEmbedding', 'LinearScalingRotaryEmbedding', 'Llama3RotaryEmbedding')


def _rope_tables(attention, rows, device):
    rope = attention.rotary_emb
    if type(rope).__name__ not in _ROPE_TYPES:
        return None
    if rows > rope.max_seq_len_cached:
        rope._set_cos_sin_cache(seq_len=rows, device=device, dtype=torch.float32)
    cos, sin = rope.cos_cached, rope.sin_cached
    if cos.device != device or cos.dtype != torch.float32:
        cos, sin = cos.to(device, torch.float32), sin.to(device, torch.float32)
    return cos, sin


def apply_rotary_with_beacon(attention, query_states, key_states, position_ids, beacon_size, beacon_indices):
    """_apply_rotary_with_beacon (modeling_qwen2.py:602-635): RoPE on every
    query and key at position_ids (queries take the last q_len positions);
    with beacon_skip_rope_for_beacon_k and beacon_size > 0 the beacon keys --
    the history prefix after the sinks and the window rows whose role is 1 or
    2 -- stay unrotated.  q [B, Hq, L, D], k [B, Hk, N, D] (BHSD)."""
    batch, _, keys, dim = key_states.shape
    tables = _rope_tables(attention, max(keys, position_ids.shape[-1]), key_states.device)
    if tables is None:
        # other RoPE variants keep the module's own rotary embedding
        return attention._apply_rotary_with_beacon(query_states, key_states, position_ids, beacon_size,
                                                    beacon_indices)
    skip = getattr(attention.config, 'beacon_skip_rope_for_beacon_k', False) and beacon_size > 0
    positions = position_ids if position_ids.shape[0] == batch else position_ids.expand(batch, -1)
    if skip:
        roles, sink = beacon_indices, getattr(attention.config, 'beacon_sink_size', 0)
    else:
        roles, sink = torch.zeros(keys, dtype=torch.long, device=key_states.device), 0
    return kernels.prefill_rope(query_states, key_states, tables[0], tables[1], positions, roles, sink)


def flash_attention_forward(attention, query_states, key_states, value_states, attention_mask, query_length,
                            dropout=0.0, softmax_scale=None):
    """BSHD q [B, L, Hq, D], k/v [B, N, Hk, D] -> out [B, L, Hq, D]; bottom-right
    causal (flash-attn >= 2.1 semantics, the module's is_causal)."""
    if attention_mask is not None:
        raise ValueError('padded batches (an attention mask) are not supported by the gfx950 attention')
    if dropout:
        raise ValueError('attention dropout is not supported (inference only)')
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(query_states.shape[-1])
    causal = bool(getattr(attention, 'is_causal', True))
    if query_length <= 2:
        out, _ = kernels.attention_forward(query_states, key_states, value_states, scale, causal)
    else:
        out, _ = kernels.prefill_attention(query_states, key_states, value_states, scale, causal)
    return out


def forward(attention, hidden_states, attention_mask=None, position_ids=None, past_key_value=None,
            output_attentions=False, use_cache=False, **kwargs):
    """(attn_output [B, L, hidden], None, (key, value, beacon_size, beacon_indices))
    with the current step's key/value before RoPE as the returned cache."""
    bsz, q_len, _ = hidden_states.size()
    past_key, past_value, beacon_size, beacon_indices = past_key_value
    heads, kv_heads, dim = attention.num_heads, attention.num_key_value_heads, attention.head_dim
    q, k, v = attention.qkv_proj_with_beacon(hidden_states, beacon_size, beacon_indices)
    q = q.view(bsz, q_len, heads, dim).transpose(1, 2)
    k = k.view(bsz, q_len, kv_heads, dim).transpose(1, 2)
    v = v.view(bsz, q_len, kv_heads, dim).transpose(1, 2)
    cache = (k, v, beacon_size, beacon_indices)
    if past_key is not None:
        k = torch.cat([past_key, k], dim=2)
        v = torch.cat([past_value, v], dim=2)
    if position_ids is None:
        position_ids = torch.arange(k.shape[2], device=k.device)[None]
    q, k = apply_rotary_with_beacon(attention, q, k, position_ids, beacon_size, beacon_indices)
    out = flash_attention_forward(attention, q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                  attention_mask, q_len)
    out = out.reshape(bsz, q_len, attention.hidden_size)
    return attention.o_proj_with_beacon(out, beacon_size, beacon_indices), None, cache
