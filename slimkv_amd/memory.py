"""Latent cache views with the reconstruction done by the HIP up-projection.

Mirrors slimkv/llama3/memory.py:10-61 (ReconstructionCache, ReconstructionCacheUpdate)
and slimkv/memory.py:999-1007 (cat_tensor); `materialize` builds the full-dim
[B, Hkv, n, D] K or V with the MFMA reconstruction kernel, writing each part in
place instead of concatenating.
"""
import torch

from . import kernels


def cat_tensor(tensors, dim):
    """Concatenate the non-None tensors (slimkv/memory.py:999-1007)."""
    tensors = [t for t in tensors if t is not None]
    if not tensors:
        return None
    if len(tensors) == 1:
        return tensors[0]
    return torch.cat(tensors, dim=dim)


def _length(tensor):
    return 0 if tensor is None else tensor.shape[2]


def is_block_diagonal(weight, kv_heads):
    """True when every off-diagonal [D, R/Hkv] block of an up-projection weight
    [Hkv*D, R] is exactly zero (per-KV-head bases).  Cached on the tensor per
    (version, kv_heads), so an in-place weight update re-checks."""
    cached = getattr(weight, '_slimkv_block_diagonal', None)
    if cached is not None and cached[:2] == (weight._version, kv_heads):
        return cached[2]
    out_features, rank = weight.shape
    result = False
    if rank % kv_heads == 0 and out_features % kv_heads == 0:
        blocks = weight.detach().reshape(kv_heads, out_features // kv_heads, kv_heads, rank // kv_heads)
        mask = ~torch.eye(kv_heads, dtype=torch.bool, device=weight.device)[:, None, :, None]
        result = not bool((blocks.abs() * mask).amax() > 0)
    weight._slimkv_block_diagonal = (weight._version, kv_heads, result)
    return result


def _flat_latents(latent):
    """[B, 1, n, R] or [B, Hkv, n, r] -> [B, n, R] (a view for the global layout)."""
    batch, heads, length, dim = latent.shape
    if heads == 1:
        return latent[:, 0]
    return latent.transpose(1, 2).reshape(batch, length, heads * dim)


class ReconstructionCache:
    """A layer-local cache read; materialization is never retained."""

    def __init__(self, sink, history, raw, window, window_roles, num_heads, head_dim, kind,
                 window_raw_indices=None):
        self.sink = sink
        self.history = history
        self.raw = raw
        self.window = window
        self.window_roles = window_roles
        self.kind = kind
        self.window_raw_indices = window_raw_indices
        batch = next((x.shape[0] for x in (sink, history, raw, window) if x is not None), 0)
        length = sum(_length(x) for x in (sink, history, raw, window))
        self.shape = (batch, num_heads, length, head_dim)

    def materialize(self, attention, current=None):
        """[sink ; up(history) ; interleave(up(window), raw) ; current] as BHSD
        (slimkv/llama3/memory.py:26-48)."""
        up = attention.beacon_k_up_proj if self.kind == 'k' else attention.beacon_v_up_proj
        heads, dim = attention.num_key_value_heads, attention.head_dim
        parts = [self.sink, self.history, self.window, self.raw, current]
        ref = next(x for x in parts if x is not None)
        batch = ref.shape[0]
        n_sink, n_hist = _length(self.sink), _length(self.history)
        n_recent = (self.window_roles.numel() if self.window is not None else _length(self.raw))
        total = n_sink + n_hist + n_recent + _length(current)
        out = torch.empty(batch, heads, total, dim, dtype=up.weight.dtype, device=up.weight.device)
        bd = is_block_diagonal(up.weight, heads)
        if self.sink is not None:
            out[:, :, :n_sink] = self.sink
        if self.history is not None:
            kernels.reconstruct(_flat_latents(self.history), up.weight, up.bias, kv_heads=heads,
                                out=out[:, :, n_sink:n_sink + n_hist].transpose(1, 2), block_diagonal=bd)
        base = n_sink + n_hist
        if self.window is None:
            if self.raw is not None:
                out[:, :, base:base + n_recent] = self.raw
        else:
            roles = self.window_roles.to(device=out.device, dtype=torch.bool)
            beacon_rows = roles.nonzero().flatten()
            kernels.reconstruct(_flat_latents(self.window), up.weight, up.bias, kv_heads=heads,
                                out=out[:, :, base:base + n_recent].transpose(1, 2), dst_rows=beacon_rows,
                                block_diagonal=bd)
            if self.raw is not None:
                out[:, :, base + (~roles).nonzero().flatten()] = self.raw
        if current is not None:
            out[:, :, total - current.shape[2]:] = current
        return out


class ReconstructionCacheUpdate(tuple):
    """The legacy four-item cache tuple plus the newly projected latents."""

    def __new__(cls, key, value, beacon_size, beacon_indices, key_latents, value_latents):
        result = super().__new__(cls, (key, value, beacon_size, beacon_indices))
        result.key_latents = key_latents
        result.value_latents = value_latents
        return result
