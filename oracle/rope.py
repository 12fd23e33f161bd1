"""RoPE tables and bf16-exact rotations (oracle).

Tables restate RotaryEmbedding._set_cos_sin_cache (slimkv/modeling_utils.py:354-376)
and Llama3RotaryEmbedding (slimkv/modeling_utils.py:690-731): fp32 inv_freq,
freqs = outer(t, inv_freq), emb = cat(freqs, freqs), cos/sin in fp32.
Rotations restate the decode kernel (slimkv/llama3/decode_kernels.py:7-51), the
prefill kernel (slimkv/llama3/prefill_kernels.py:7-53) and the torch fallback
`x * cos + rotate_half(x) * sin` with bf16 cos/sin
(slimkv/llama3/fa2_decode.py:118-121; rotate_half slimkv/modeling_utils.py:347-351).
"""
import math

import numpy as np

from .bf16 import round_bf16


def inv_freq(dim, base):
    """1 / base^(2i/dim) computed in fp32 as torch does (modeling_utils.py:359)."""
    exponent = (np.arange(0, dim, 2, dtype=np.float32) / np.float32(dim)).astype(np.float32)
    return (np.float32(1.0) / np.power(np.float32(base), exponent, dtype=np.float32)).astype(np.float32)


def llama3_inv_freq(dim, base, scaling_factor, original_max, low_freq_factor, high_freq_factor):
    """Llama-3 wavelength smoothing (modeling_utils.py:702-716)."""
    freqs = inv_freq(dim, base)
    low_wavelen = original_max / low_freq_factor
    high_wavelen = original_max / high_freq_factor
    out = []
    for f in freqs.astype(np.float64):
        f32 = np.float32(f)
        wavelen = 2 * math.pi / float(f32)
        if wavelen < high_wavelen:
            out.append(f32)
        elif wavelen > low_wavelen:
            out.append(np.float32(f32 / scaling_factor))
        else:
            smooth = (original_max / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
            out.append(np.float32((1 - smooth) * f32 / scaling_factor + smooth * f32))
    return np.array(out, dtype=np.float32)


def tables(rows, freqs):
    """cos/sin [rows, dim] fp32 from fp32 angles t * inv_freq (modeling_utils.py:368-376).

    The angle is the fp32 product (torch.outer in fp32); cos/sin of that fp32
    angle are evaluated in float64 and rounded once to fp32.
    """
    t = np.arange(rows, dtype=np.float32)
    angles = np.outer(t, freqs).astype(np.float32)
    emb = np.concatenate([angles, angles], axis=-1).astype(np.float64)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def rotate_half(x):
    half = x.shape[-1] // 2
    return np.concatenate([-x[..., half:], x[..., :half]], axis=-1)


def rotate_bf16(x, cos_rows, sin_rows):
    """bf16(bf16(x*bf16(cos)) + bf16(rotate_half(x)*bf16(sin))), fp32 products.

    x holds bf16 values (float32 array); cos_rows/sin_rows broadcast to x.
    decode_kernels.py:44-51 (and the identical torch bf16 fallback).
    """
    c = round_bf16(cos_rows)
    s = round_bf16(sin_rows)
    first = round_bf16(x.astype(np.float32) * c)
    second = round_bf16(rotate_half(x).astype(np.float32) * s)
    return round_bf16(first + second)


def decode_key_positions(keys, sink, history, raw_indices, current):
    """Positions of the raw K slots (decode_kernels.py:36-40; fa2_decode.py:122-126):
    slot s < sink -> s; last slot -> current; else raw_indices[s-sink]+sink+history."""
    pos = np.empty(keys, dtype=np.int64)
    for s in range(keys):
        if s < sink:
            pos[s] = s
        elif s == keys - 1:
            pos[s] = current
        else:
            pos[s] = int(raw_indices[s - sink]) + sink + history
    return pos


def rope_decode(q, k, cos, sin, query_positions, raw_indices, sink, history):
    """fused_rope semantics.  q [B,Hq,L,D], k [B,Hk,N,D] (bf16 values), positions
    [B,L] int64.  Returns rotated (q, k) as float32 arrays of bf16 values."""
    B, Hq, L, D = q.shape
    N = k.shape[2]
    oq = np.empty_like(q, dtype=np.float32)
    ok = np.empty_like(k, dtype=np.float32)
    for b in range(B):
        qp = np.asarray(query_positions[b], dtype=np.int64)
        oq[b] = rotate_bf16(q[b], cos[qp][None], sin[qp][None])
        kp = decode_key_positions(N, sink, history, raw_indices, int(qp[0]))
        ok[b] = rotate_bf16(k[b], cos[kp][None], sin[kp][None])
    return oq, ok


def prefill_beacon_mask(keys, role_len, roles, sink):
    """Beacon K slots keep unrotated K (prefill_kernels.py:38-41): the history
    prefix [sink, keys-role_len) and window slots whose role is 1 or 2."""
    prefix = keys - role_len
    mask = np.zeros(keys, dtype=bool)
    for s in range(keys):
        if s < prefix:
            mask[s] = s >= sink
        else:
            mask[s] = int(roles[s - prefix]) in (1, 2)
    return mask


def prefill_rope(q, k, cos, sin, positions, roles, sink):
    """fused_prefill_rope semantics.  q [B,Hq,Lq,D], k [B,Hk,N,D], positions [B,N]."""
    B, Hq, Lq, D = q.shape
    N = k.shape[2]
    mask = prefill_beacon_mask(N, len(roles), roles, sink)
    oq = np.empty_like(q, dtype=np.float32)
    ok = np.empty_like(k, dtype=np.float32)
    for b in range(B):
        pos = np.asarray(positions[b], dtype=np.int64)
        qp = pos[N - Lq:]
        oq[b] = rotate_bf16(q[b], cos[qp][None], sin[qp][None])
        rotated = rotate_bf16(k[b], cos[pos][None], sin[pos][None])
        ok[b] = np.where(mask[None, :, None], k[b], rotated)
    return oq, ok
