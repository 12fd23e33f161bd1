"""Drop-in for slimkv.llama3.latent_decode: backend selection and eager attention.

uses_latent_decode / uses_fa2_decode follow slimkv/llama3/latent_decode.py:7-13.
eager_forward keeps the reference signature and arithmetic (latent_decode.py:
16-41): inputs of any model dtype (bf16, fp16, fp32) meet in fp32 in the HIP
eager attention kernel, the output is cast once to q's dtype, the LSE stays
fp32.  It computes on the GPU only: CPU tensors raise, as does autograd (the
reference's function is the CPU/gradient baseline of the fused kernels, which
this library does not provide).
"""
import torch


def uses_latent_decode(config):
    return getattr(config, 'beacon_decode_backend', 'reconstruct') in ('latent', 'fa2')


def uses_fa2_decode(config):
    backend = getattr(config, 'beacon_decode_backend', 'reconstruct')
    return backend == 'fa2' or (backend == 'latent' and config._attn_implementation == 'flash_attention_2')


def eager_forward(q, k, v, scale, causal=False):
    """BSHD inputs, BSHD output and BHQ log-sum-exp; K/V ranks may differ."""
    batch, queries, heads, rank = q.shape
    keys, kv_heads = k.shape[1:3]
    if (k.shape[0] != batch or k.shape[-1] != rank or v.shape[:3] != k.shape[:3]
            or kv_heads < 1 or heads % kv_heads or keys < 1):
        raise ValueError('Invalid eager attention shapes or GQA head counts.')
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError('slimkv_amd computes eager attention on the GPU; CPU tensors are not supported')
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        raise ValueError('slimkv_amd eager attention is inference-only (no autograd)')
    from . import kernels
    if k.dtype != q.dtype or v.dtype != q.dtype:       # mixed dtypes meet in fp32 as well
        out, lse = kernels.eager_attention(q.float(), k.float(), v.float(), scale, causal)
        return out.to(q.dtype), lse
    return kernels.eager_attention(q, k, v, scale, causal)
