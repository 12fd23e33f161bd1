"""Drop-in for slimkv.llama3.decode_ops: fused decode RoPE and LSE merge.

Contract of slimkv/llama3/decode_ops.py:14-48: the functions return None (the
caller's torch path) for tensors off the GPU, a dtype other than bf16 / fp16,
or autograd in use.  The merge runs the HIP kernel for device bf16 and fp16
tensors (fp32 arithmetic, one rounding), as the reference's fused merge does.
The RoPE kernel is bf16-exact only: fp16 RoPE returns None, and the caller
rotates with its own module, as it does where the reference lacks Triton.
"""
import torch

from . import kernels


def _skip(x, *others, dtypes=(torch.bfloat16,)):
    return (not x.is_cuda or x.dtype not in dtypes
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
    if _skip(raw, latent, dtypes=(torch.bfloat16, torch.float16)) or latent.dtype != raw.dtype:
        return None
    return kernels.merge(raw, raw_lse, latent, latent_lse)
