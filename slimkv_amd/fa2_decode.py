"""Drop-in for slimkv.llama3.fa2_decode: reconstruction-free latent decode on gfx950.

Same names, arguments and return values as the reference module
(slimkv/llama3/fa2_decode.py); the attention work runs in the HIP library.
`decode` fuses query RoPE, absorption, both branches, the V lift, bias folding
and the merge into one call of slimkv_latent_decode; when a caller passes its
own `forward` (the reference tests substitute flash_forward this way) the
two-branch composition of the reference is used with that forward.
"""
import math

import torch
import torch.nn.functional as F

from . import kernels
from .latent_decode import eager_forward, uses_fa2_decode, uses_latent_decode  # noqa: F401
from .memory import ReconstructionCache, ReconstructionCacheUpdate, cat_tensor, is_block_diagonal

MAX_WIDTH = 384


def flash_forward(q, k, v, scale, causal=False):
    """BSHD q [B,Lq,H,Wq], k [B,N,Hk,Wq], v [B,N,Hk,Wv] -> (out BSHD, lse [B,H,Lq]).

    slimkv/llama3/fa2_decode.py:15-38.  Widths are padded to a multiple of 8
    (as the reference pads) with the original scale; K and V widths may differ,
    so no 320-wide padding is needed.  Rows that see no key get LSE -inf.
    """
    width = max(q.shape[-1], k.shape[-1], v.shape[-1])
    if width > MAX_WIDTH:
        raise ValueError(f'Latent decode supports global ranks up to {MAX_WIDTH}, found {width}')
    wk = (max(q.shape[-1], k.shape[-1]) + 7) // 8 * 8
    wv = (v.shape[-1] + 7) // 8 * 8
    if q.shape[-1] != wk:
        q = F.pad(q, (0, wk - q.shape[-1]))
    if k.shape[-1] != wk:
        k = F.pad(k, (0, wk - k.shape[-1]))
    if v.shape[-1] != wv:
        v = F.pad(v, (0, wv - v.shape[-1]))
    return kernels.attention_forward(q, k, v, scale, causal)


def project_query(q, weight, kv_heads):
    """Q in BHQD; global U_K slices follow the GQA grouping (fa2_decode.py:41-46)."""
    batch, heads, length, dim = q.shape
    rank = weight.shape[-1]
    grouped = q.reshape(batch, kv_heads, heads // kv_heads * length, dim)
    return (grouped @ weight.reshape(kv_heads, dim, rank)).reshape(batch, heads, length, rank)


def project_value(output, weight, kv_heads):
    """Latent PV in BHQR; each KV head's U_V slice (fa2_decode.py:49-54)."""
    batch, heads, length, rank = output.shape
    dim = weight.shape[0] // kv_heads
    grouped = output.reshape(batch, kv_heads, heads // kv_heads * length, rank)
    return (grouped @ weight.reshape(kv_heads, dim, rank).transpose(-1, -2)).reshape(batch, heads, length, dim)


def merge_attention(raw_out, raw_lse, latent_out, latent_lse):
    """Outputs BHQD, LSE BHQ; merged in fp32, rounded once (fa2_decode.py:57-66).

    Where the reference's fused merge does not apply (fp32 outputs) it merges
    with torch arithmetic; here every dtype (bf16, fp16, fp32) runs the HIP
    merge.  CPU tensors and autograd raise: this library has no CPU or
    gradient path."""
    from .decode_ops import fused_merge
    fused = fused_merge(raw_out, raw_lse, latent_out, latent_lse)
    if fused is not None:
        return fused
    if not (raw_out.is_cuda and latent_out.is_cuda):
        raise ValueError('slimkv_amd merges on the GPU; CPU tensors are not supported')
    if torch.is_grad_enabled() and (raw_out.requires_grad or latent_out.requires_grad):
        raise ValueError('slimkv_amd merge is inference-only (no autograd)')
    if latent_out.dtype != raw_out.dtype:
        latent_out = latent_out.to(raw_out.dtype)
    return kernels.merge(raw_out, raw_lse, latent_out, latent_lse)


def eligible(attention, hidden_states, past_key_value, output_attentions):
    """Latent decode gate (fa2_decode.py:69-74)."""
    return (getattr(attention.config, '_slimkv_decode_step', False)
            and uses_latent_decode(attention.config)
            and isinstance(past_key_value[0], ReconstructionCache)
            and not attention.training and not output_attentions
            and hidden_states.shape[0] > 0 and hidden_states.shape[1] in (1, 2))


def _positions(position_ids, length, sink_len, history_len, raw_indices):
    positions = [position_ids[0, :sink_len]]
    if raw_indices is not None:
        positions.append(raw_indices.to(position_ids.device) + sink_len + history_len)
    positions.append(position_ids[0, -length:][:1])
    return torch.cat(positions)


def _rotate(attention, q, raw_k, position_ids, length, pk, sink_len, history_len):
    """RoPE on q (BHSD) and raw K (BHSD) with the decode position rule."""
    rope = attention.rotary_emb
    if (type(rope).__name__ in ('RotaryEmbedding', 'LinearScalingRotaryEmbedding', 'Llama3RotaryEmbedding')
            and position_ids.shape[-1] <= rope.max_seq_len_cached):
        cos, sin = rope.cos_cached, rope.sin_cached
        if cos.device != q.device or cos.dtype != torch.float32:
            cos, sin = cos.to(q.device, torch.float32), sin.to(q.device, torch.float32)
        return kernels.rope_decode(q, raw_k, cos, sin, position_ids[:, -length:], pk.window_raw_indices,
                                   sink_len, history_len)
    # Other RoPE variants keep their own module (query temperature, other
    # frequencies): dummy keys carry the query positions (fa2_decode.py:127-142).
    batch = q.shape[0]
    raw_positions = _positions(position_ids, length, sink_len, history_len, pk.window_raw_indices)
    raw_positions = raw_positions.unsqueeze(0).expand(batch, -1)
    rope_positions = torch.cat([raw_positions, position_ids[:, -length:]], dim=1)
    dummy = raw_k.new_zeros(batch, raw_k.shape[1], length, raw_k.shape[-1])
    q, rotated = rope(q, torch.cat([raw_k, dummy], dim=2), rope_positions)
    return q, rotated[:, :, :-length]


def decode(attention, hidden, position_ids, past_key_value, forward=None):
    """One raw token, optionally followed by its newly inserted beacon
    (slimkv/llama3/fa2_decode.py:77-166).  Returns (attn_out, None, update)."""
    pk, pv, size, indices = past_key_value
    batch, length, _ = hidden.shape
    if size not in (0, 1) or length != size + 1:
        raise ValueError('Latent decode expects one raw token followed by at most one Beacon.')
    uk, uv = attention.beacon_k_up_proj, attention.beacon_v_up_proj
    if not isinstance(uk, torch.nn.Linear) or not isinstance(uv, torch.nn.Linear):
        raise ValueError('Latent decode currently requires globally coupled Linear up projections.')
    heads, kv_heads, dim = attention.num_heads, attention.num_key_value_heads, attention.head_dim
    raw_hidden = hidden[:, :1]
    q = attention.q_proj(hidden)
    new_k = attention.k_proj(raw_hidden).reshape(batch, 1, kv_heads, dim).transpose(1, 2)
    new_v = attention.v_proj(raw_hidden).reshape(batch, 1, kv_heads, dim).transpose(1, 2)
    kl = vl = None
    if size:
        if 'q' in attention.config.beacon_param:
            q = torch.cat([q[:, :1], attention.beacon_q_proj(hidden[:, 1:])], dim=1)
        shared = attention._use_shared_kv_down_proj()
        kd = attention.beacon_kv_down_proj if shared else attention.beacon_k_down_proj
        vd = attention.beacon_kv_down_proj if shared else attention.beacon_v_down_proj
        kl, vl = kd(hidden[:, 1:]).unsqueeze(1), vd(hidden[:, 1:]).unsqueeze(1)
    update = ReconstructionCacheUpdate(new_k, new_v, size, indices, kl, vl)
    update.raw_only = True
    q = q.reshape(batch, length, heads, dim).transpose(1, 2)
    raw_k = cat_tensor([pk.sink, pk.raw, new_k], dim=2)
    raw_v = cat_tensor([pv.sink, pv.raw, new_v], dim=2)
    sink_len = 0 if pk.sink is None else pk.sink.shape[2]
    history_len = 0 if pk.history is None else pk.history.shape[2]
    q, raw_k = _rotate(attention, q, raw_k, position_ids, length, pk, sink_len, history_len)
    scale = 1.0 / math.sqrt(dim)
    if forward is None:
        # The history's latent rows are read where they lie (first segment);
        # only the current window and the new beacon are joined (second).
        window_k = cat_tensor([pk.window, kl], dim=2)
        window_v = cat_tensor([pv.window, vl], dim=2)
        hist_k = None if pk.history is None else pk.history[:, 0]
        hist_v = None if pv.history is None else pv.history[:, 0]
        out, _ = kernels.latent_decode(
            q.transpose(1, 2), raw_k.transpose(1, 2), raw_v.transpose(1, 2), hist_k, hist_v,
            uk.weight, uv.weight, scale, up_k_bias=uk.bias, up_v_bias=uv.bias,
            block_diagonal=is_block_diagonal(uk.weight, kv_heads) and is_block_diagonal(uv.weight, kv_heads),
            lat_causal=bool(size), lat_k2=None if window_k is None else window_k[:, 0],
            lat_v2=None if window_v is None else window_v[:, 0])
        output = out.reshape(batch, length, attention.hidden_size)
        return attention.o_proj_with_beacon(output, size, indices), None, update
    latent_k = cat_tensor([pk.history, pk.window, kl], dim=2)
    latent_v = cat_tensor([pv.history, pv.window, vl], dim=2)
    # Two-branch composition with a caller-supplied attention forward.
    raw_out, raw_lse = forward(q.transpose(1, 2), raw_k.transpose(1, 2), raw_v.transpose(1, 2), scale, False)
    raw_out = raw_out[..., :dim].transpose(1, 2)
    if latent_k is None:
        output = raw_out
    else:
        latent_q = project_query(q, uk.weight, kv_heads)
        latent_out, latent_lse = forward(latent_q.transpose(1, 2), latent_k.transpose(1, 2),
                                         latent_v.transpose(1, 2), scale, bool(size))
        latent_out = project_value(latent_out[..., :uv.in_features].transpose(1, 2), uv.weight, kv_heads)
        groups = heads // kv_heads
        if uk.bias is not None:
            bias = uk.bias.reshape(kv_heads, dim).repeat_interleave(groups, dim=0)
            latent_lse = latent_lse + (q.float() * bias[None, :, None].float()).sum(-1) * scale
        if uv.bias is not None:
            bias = uv.bias.reshape(kv_heads, dim).repeat_interleave(groups, dim=0)
            latent_out = latent_out + bias[None, :, None]
        output = merge_attention(raw_out, raw_lse, latent_out, latent_lse)
    output = output.transpose(1, 2).reshape(batch, length, attention.hidden_size)
    return attention.o_proj_with_beacon(output, size, indices), None, update
