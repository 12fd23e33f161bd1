"""Drop-in for slimkv.llama3.prefill_ops: prefill index metadata and RoPE.

PrefillMetadata / prepare_metadata restate slimkv/llama3/prefill_ops.py:8-36
(host bookkeeping shared by all layers); fused_prefill_rope (:48-73) runs the
bf16-exact HIP kernel that leaves beacon K unrotated.
"""
from dataclasses import dataclass

import torch

from . import kernels


@dataclass
class PrefillMetadata:
    raw_indices: torch.Tensor
    beacon_indices: torch.Tensor
    roles: torch.Tensor
    positions: torch.Tensor
    replicas: bool


def prepare_metadata(model, ids, mask, positions, past, labels):
    config = model.config
    if (not getattr(config, 'beacon_prefill_fast', True) or model.training
            or torch.is_grad_enabled() or labels is not None or not ids.is_cuda
            or ids.shape[1] <= 1 or getattr(config, '_slimkv_decode_step', False)
            or config._attn_implementation != 'flash_attention_2' or mask is not None
            or config.beacon_pos != 'interleave' or config.beacon_parallel_window != 1
            or config.beacon_window != config.beacon_stride
            or not model.memory.latent_cache_active or past[0][2] < 0
            or not getattr(config, 'beacon_skip_rope_for_beacon_k', False)
            or getattr(config, 'beacon_chunk_fixed_rope_for_beacon_k', False)
            or getattr(config, 'beacon_enhance_k_pos_residual', False)
            or getattr(config, 'raw_nokrope', False)
            or getattr(config, 'beacon_skip_rope_for_raw_k', False)):
        return None
    roles = past[0][3]
    current = roles[-ids.shape[1]:]
    return PrefillMetadata((current == 0).nonzero().flatten(), (current != 0).nonzero().flatten(), roles,
                           positions, bool((current == 2).any()))


def fused_prefill_rope(q, k, rope, metadata, sink):
    """q [B,Hq,Lq,D], k [B,Hk,N,D] -> (q, k) rotated; beacon K copied unchanged."""
    if (not q.is_cuda or not k.is_cuda or q.dtype != torch.bfloat16 or k.dtype != q.dtype
            or q.shape[-1] != k.shape[-1] or q.shape[-1] % 16
            or type(rope).__name__ not in ('RotaryEmbedding', 'LinearScalingRotaryEmbedding', 'Llama3RotaryEmbedding')
            or metadata.positions.shape != (q.shape[0], k.shape[2])
            or k.shape[2] > rope.max_seq_len_cached
            or metadata.roles.numel() > k.shape[2]
            or q.stride(-1) != 1 or k.stride(-1) != 1):
        return None
    cos, sin = rope.cos_cached, rope.sin_cached
    if cos.device != q.device or cos.dtype != torch.float32:
        cos, sin = cos.to(q.device, torch.float32), sin.to(q.device, torch.float32)
    return kernels.prefill_rope(q, k, cos, sin, metadata.positions, metadata.roles, sink)
