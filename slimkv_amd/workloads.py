"""Seeded synthetic inputs for the latent beacon decode layer.

Shapes follow the Llama-3.1-8B / Qwen2.5-14B attention layer: Hq query heads,
Hkv KV heads, head_dim D.  A decode step sees
  * `sinks` full-dim sink tokens at positions 0..sinks-1,
  * a full-dim raw tail of `tail` tokens ending just before the query,
  * the current token (its K/V belong to the raw set; the reference always
    appends it, slimkv/llama3/fa2_decode.py:103-104),
  * `beacons` latent rows of rank rk (K) / rv (V) per KV head, never RoPE'd.
Latents, K/V and queries are N(0,1); the per-KV-head bases U_k [D x rk] and
U_v [D x rv] have orthonormal columns (QR of a Gaussian) and are assembled into
the block-diagonal nn.Linear weights [Hkv*D, Hkv*r] of the global layout.
"""
from dataclasses import dataclass

import torch


@dataclass
class LatentCase:
    q: torch.Tensor            # [B,1,Hq,D] bf16, before RoPE
    q_positions: torch.Tensor  # [B,1] int64
    raw_k: torch.Tensor        # [B,Nr,Hkv,D] bf16, before RoPE
    raw_v: torch.Tensor        # [B,Nr,Hkv,D] bf16
    raw_positions: torch.Tensor  # [Nr] int64
    lat_k: torch.Tensor        # [B,Nb,Hkv*rk] bf16
    lat_v: torch.Tensor        # [B,Nb,Hkv*rv] bf16
    up_k: torch.Tensor         # [Hkv*D, Hkv*rk] bf16, block diagonal
    up_v: torch.Tensor         # [Hkv*D, Hkv*rv] bf16, block diagonal
    cos: torch.Tensor          # [rows, D] fp32
    sin: torch.Tensor
    scale: float
    sinks: int
    tail: int

    @property
    def kv_heads(self):
        return self.raw_k.shape[2]


def rope_tables(rows, dim, base, device='cpu'):
    """RotaryEmbedding tables in fp32 (slimkv/modeling_utils.py:359-376)."""
    inv = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    t = torch.arange(rows, dtype=torch.float32)
    freqs = torch.outer(t, inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(device), emb.sin().to(device)


def orthonormal_columns(rows, cols, generator):
    """QR of a Gaussian [rows, cols] on the CPU, signs fixed by diag(R) > 0."""
    g = torch.randn(rows, cols, generator=generator, dtype=torch.float32)
    q, r = torch.linalg.qr(g)
    return q * torch.sign(torch.diagonal(r))[None]


def block_diagonal(blocks):
    """Per-KV-head [D, r] blocks -> nn.Linear weight [Hkv*D, Hkv*r]."""
    D, r = blocks[0].shape
    out = torch.zeros(len(blocks) * D, len(blocks) * r, dtype=blocks[0].dtype, device=blocks[0].device)
    for h, blk in enumerate(blocks):
        out[h * D:(h + 1) * D, h * r:(h + 1) * r] = blk
    return out


def latent_case(batch=1, heads=32, kv_heads=8, head_dim=128, context=4096, ratio=4, sinks=4, tail=124,
                rank_k=32, rank_v=32, theta=500000.0, seed=0, device='cpu', dtype=torch.bfloat16):
    """One latent decode layer.  `context` raw tokens precede the query; the
    beacons cover context - sinks - tail of them at `ratio` tokens each.
    Draw order (generator on `device`): lat_k, lat_v, raw_k, raw_v, q; then
    (CPU generator seeded seed+1) U_k and U_v per KV head.
    Positions: sinks 0.., tail context-tail.., query = context."""
    gen = torch.Generator(device=device).manual_seed(seed)
    cpu_gen = torch.Generator().manual_seed(seed + 1)
    beacons = (context - sinks - tail) // ratio
    nr = sinks + tail + 1

    def randn(*shape):
        return torch.randn(*shape, generator=gen, device=device, dtype=torch.float32).to(dtype)

    lat_k = randn(batch, beacons, kv_heads * rank_k)
    lat_v = randn(batch, beacons, kv_heads * rank_v)
    raw_k = randn(batch, nr, kv_heads, head_dim)
    raw_v = randn(batch, nr, kv_heads, head_dim)
    q = randn(batch, 1, heads, head_dim)
    uk = [orthonormal_columns(head_dim, rank_k, cpu_gen) for _ in range(kv_heads)]
    uv = [orthonormal_columns(head_dim, rank_v, cpu_gen) for _ in range(kv_heads)]
    up_k = block_diagonal(uk).to(device=device, dtype=dtype)
    up_v = block_diagonal(uv).to(device=device, dtype=dtype)
    positions = torch.cat([torch.arange(sinks), torch.arange(context - tail, context),
                           torch.tensor([context])]).to(device)
    q_positions = torch.full((batch, 1), context, dtype=torch.int64, device=device)
    cos, sin = rope_tables(context + 1, head_dim, theta, device)
    return LatentCase(q, q_positions, raw_k, raw_v, positions, lat_k, lat_v, up_k, up_v, cos, sin,
                      1.0 / head_dim ** 0.5, sinks, tail)


def decode_rope_layout(case):
    """(raw_indices, history) such that the decode RoPE key-position rule
    (slot s -> raw_indices[s-sinks] + sinks + history) reproduces the tail
    positions of `case`."""
    tail_pos = case.raw_positions[case.sinks:case.sinks + case.tail]
    history = int(tail_pos[0]) - case.sinks if case.tail else 0
    raw_indices = tail_pos - case.sinks - history
    return raw_indices, history
