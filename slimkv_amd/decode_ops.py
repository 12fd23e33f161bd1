"""Drop-in for slimkv.llama3.decode_ops: fused decode RoPE and LSE merge.

Same contract as slimkv/llama3/decode_ops.py:14-48: the functions return None
(the caller's torch path) only where the reference does -- tensors off the GPU,
a dtype other than bf16, or autograd in use.  Device bf16 tensors always run
the HIP kernels (bit-exact RoPE, fp32 merge).
"""
import torch

from . import kernels


def _skip(x, *others):
    return (not x.is_cuda or x.dtype != torch.bfloat16
            or (torch.is_grad_enabled() and any(t.requires_grad for t in (x, *others))))


def fused_rope(q, k, rope, query_positions, raw_indices, sink, history):
    """q [B,Hq,L,D], raw K [B,Hk,N,D] (BHSD) -> rotated (q, k), contiguous."""
    if _skip(q, k):
        return None
    cos, sin = rope.cos_cached, rope.sin_cached
    if cos.device != q.device or cos.dtype != torch.float32:
        cos, sin = cos.to(q.device, torch.float32), sin.to(q.device, torch.float32)
    return kernels.rope_decode(q, k, cos, sin, query_positions, raw_indices, sink, history)


def fused_merge(raw, raw_lse, latent, latent_lse):
    """raw/latent [B,H,L,D], LSEs [B,H,L] -> merged [B,H,L,D] in raw.dtype."""
    if _skip(raw, latent):
        return None
    return kernels.merge(raw, raw_lse, latent, latent_lse)
