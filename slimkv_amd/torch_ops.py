"""torch.library operators over the HIP library.

Importing this module registers, in namespace `slimkv`, custom operators for
the decode path's entry points, each with a fake (meta) implementation that
gives the output shapes, so torch.compile callers trace through the decode
instead of breaking the graph at every call.  The reference wraps its
extension the same way for its benchmark runtime
(tools/benchmark/context_decode_runtime.py:44-80: `attention` over the
extension's forward, `paired_attention`); its kernels themselves are called
through pybind.  Every operator launches the gfx950 kernels through
slimkv_amd.kernels and has no CPU implementation.

    slimkv::attention(q, k, v, scale, causal, splits, lengths) -> (out, lse)
        the forward320 split-K attention (kernels/fa2_decode/binding.cpp:123-130)
    slimkv::paired_attention(q, k, v, lengths, scale, splits) -> (out, lse)
        context_decode_runtime.py:71-80 (q holds both queries of a step)
    slimkv::latent_decode(...) -> (out, lse)      fused latent beacon decode
        (slimkv/llama3/fa2_decode.py:77-166 in one call)
    slimkv::recon_decode(...) -> (out, lse)       reconstruction decode
        (slimkv/llama3/modeling_llama.py:1405-1483)
    slimkv::rope_decode(q, k, cos, sin, query_positions, raw_indices, sink,
        history) -> (q_rot, k_rot)                 (decode_kernels.py:7-51)
    slimkv::merge(raw, raw_lse, latent, latent_lse) -> out
        (fa2_decode.py:57-66)
"""
from typing import Optional

import torch

from . import kernels

Tensor = torch.Tensor
_NS = 'slimkv'


def _lse_like(q, B, H, L):
    return q.new_empty((B, H, L), dtype=torch.float32)


@torch.library.custom_op(f'{_NS}::attention', mutates_args=(), device_types='cuda')
def attention(q: Tensor, k: Tensor, v: Tensor, scale: float, causal: bool, splits: int,
              lengths: Optional[Tensor]) -> tuple[Tensor, Tensor]:
    """BSHD q [B,Lq,Hq,W], k/v [B,N,Hk,W] -> (out [B,Lq,Hq,Wv], lse [B,Hq,Lq])."""
    return kernels.attention_forward(q, k, v, scale, causal, splits=splits, seqlens=lengths)


@attention.register_fake
def _(q, k, v, scale, causal, splits, lengths):
    B, Lq, Hq, _ = q.shape
    return q.new_empty((B, Lq, Hq, v.shape[-1])), _lse_like(q, B, Hq, Lq)


@torch.library.custom_op(f'{_NS}::paired_attention', mutates_args=(), device_types='cuda')
def paired_attention(q: Tensor, k: Tensor, v: Tensor, lengths: Tensor, scale: float,
                     splits: int) -> tuple[Tensor, Tensor]:
    """Both queries of a two-query step over one K/V (no causal mask)."""
    return kernels.attention_forward(q, k, v, scale, False, splits=splits, seqlens=lengths)


@paired_attention.register_fake
def _(q, k, v, lengths, scale, splits):
    B, Lq, Hq, _ = q.shape
    return q.new_empty((B, Lq, Hq, v.shape[-1])), _lse_like(q, B, Hq, Lq)


@torch.library.custom_op(f'{_NS}::latent_decode', mutates_args=(), device_types='cuda')
def latent_decode(q: Tensor, raw_k: Tensor, raw_v: Tensor, lat_k: Tensor, lat_v: Tensor, up_k: Tensor,
                  up_v: Tensor, scale: float, up_k_bias: Optional[Tensor], up_v_bias: Optional[Tensor],
                  block_diagonal: bool, lat_causal: bool, q_positions: Optional[Tensor], cos: Optional[Tensor],
                  sin: Optional[Tensor], raw_lengths: Optional[Tensor],
                  lat_lengths: Optional[Tensor]) -> tuple[Tensor, Tensor]:
    """kernels.latent_decode: q [B,Lq,Hq,D] -> (out [B,Lq,Hq,D], lse [B,Hq,Lq])."""
    return kernels.latent_decode(q, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale, up_k_bias=up_k_bias,
                                 up_v_bias=up_v_bias, block_diagonal=block_diagonal, lat_causal=lat_causal,
                                 q_positions=q_positions, cos=cos, sin=sin, raw_lengths=raw_lengths,
                                 lat_lengths=lat_lengths)


@latent_decode.register_fake
def _(q, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale, up_k_bias, up_v_bias, block_diagonal, lat_causal,
      q_positions, cos, sin, raw_lengths, lat_lengths):
    B, Lq, Hq, D = q.shape
    return q.new_empty((B, Lq, Hq, D)), _lse_like(q, B, Hq, Lq)


@torch.library.custom_op(f'{_NS}::recon_decode', mutates_args=(), device_types='cuda')
def recon_decode(q: Tensor, raw_k: Tensor, raw_v: Tensor, lat_k: Tensor, lat_v: Tensor, up_k: Tensor,
                 up_v: Tensor, scale: float, beacon_positions: Optional[Tensor], up_k_bias: Optional[Tensor],
                 up_v_bias: Optional[Tensor], block_diagonal: bool, lat_causal: bool,
                 q_positions: Optional[Tensor], cos: Optional[Tensor], sin: Optional[Tensor],
                 raw_lengths: Optional[Tensor], lat_lengths: Optional[Tensor],
                 reference_rounding: bool) -> tuple[Tensor, Tensor]:
    """kernels.recon_decode: q [B,Lq,Hq,D] -> (out [B,Lq,Hq,D], lse [B,Hq,Lq])."""
    return kernels.recon_decode(q, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale,
                                beacon_positions=beacon_positions, up_k_bias=up_k_bias, up_v_bias=up_v_bias,
                                block_diagonal=block_diagonal, lat_causal=lat_causal, q_positions=q_positions,
                                cos=cos, sin=sin, raw_lengths=raw_lengths, lat_lengths=lat_lengths,
                                reference_rounding=reference_rounding)


@recon_decode.register_fake
def _(q, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale, beacon_positions, up_k_bias, up_v_bias, block_diagonal,
      lat_causal, q_positions, cos, sin, raw_lengths, lat_lengths, reference_rounding):
    B, Lq, Hq, D = q.shape
    return q.new_empty((B, Lq, Hq, D)), _lse_like(q, B, Hq, Lq)


@torch.library.custom_op(f'{_NS}::rope_decode', mutates_args=(), device_types='cuda')
def rope_decode(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor, query_positions: Tensor,
                raw_indices: Optional[Tensor], sink: int, history: int) -> tuple[Tensor, Tensor]:
    """kernels.rope_decode: BHSD q, k -> new contiguous (q_rot, k_rot)."""
    return kernels.rope_decode(q, k, cos, sin, query_positions, raw_indices, sink, history)


@rope_decode.register_fake
def _(q, k, cos, sin, query_positions, raw_indices, sink, history):
    return q.new_empty(q.shape), k.new_empty(k.shape)


@torch.library.custom_op(f'{_NS}::merge', mutates_args=(), device_types='cuda')
def merge(raw: Tensor, raw_lse: Tensor, latent: Tensor, latent_lse: Tensor) -> Tensor:
    """kernels.merge: BHSD raw/latent with their LSEs -> merged [B,H,L,D]."""
    return kernels.merge(raw, raw_lse, latent, latent_lse)


@merge.register_fake
def _(raw, raw_lse, latent, latent_lse):
    return raw.new_empty(raw.shape)
