"""The reference's eager latent decode path restated in torch fp32 on the CPU.

Used only as the CPU baseline leg of bench.py (timed on the host cores) and as a
second, independent restatement checked against the numpy oracle in tests.
Follows slimkv/llama3/latent_decode.py:16-41 (eager_forward),
slimkv/llama3/fa2_decode.py:41-54 (project_query / project_value),
:57-66 (merge) and :145-164 (the branch structure of decode), in fp32 as the
reference eager path computes (latent_decode.py:26-28).
"""
import math

import torch


def eager_forward(q, k, v, scale, causal=False):
    batch, queries, heads, rank = q.shape
    keys, kv_heads = k.shape[1:3]
    groups = heads // kv_heads
    grouped_q = q.transpose(1, 2).reshape(batch, kv_heads, groups * queries, rank)
    scores = (grouped_q.float() @ k.transpose(1, 2).transpose(-1, -2).float()) * scale
    scores = scores.reshape(batch, heads, queries, keys)
    if causal:
        qpos = torch.arange(queries) + keys - queries
        scores = scores.masked_fill(torch.arange(keys)[None, :] > qpos[:, None], -math.inf)
    lse = torch.logsumexp(scores, dim=-1)
    probs = torch.softmax(scores, dim=-1)
    probs = torch.where(torch.isfinite(lse)[..., None], probs, 0.0)
    out = probs.reshape(batch, kv_heads, groups * queries, keys) @ v.transpose(1, 2).float()
    return out.reshape(batch, heads, queries, v.shape[-1]).transpose(1, 2), lse


def project_query(q, weight, kv_heads):
    batch, heads, length, dim = q.shape
    grouped = q.reshape(batch, kv_heads, heads // kv_heads * length, dim)
    return (grouped @ weight.reshape(kv_heads, dim, weight.shape[-1])).reshape(batch, heads, length, -1)


def project_value(out, weight, kv_heads):
    batch, heads, length, rank = out.shape
    dim = weight.shape[0] // kv_heads
    grouped = out.reshape(batch, kv_heads, heads // kv_heads * length, rank)
    return (grouped @ weight.reshape(kv_heads, dim, rank).transpose(-1, -2)).reshape(batch, heads, length, dim)


def latent_layer(q_rot, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale, kv_heads, up_k_bias=None, up_v_bias=None):
    """q_rot [B,H,1,D]; raw_k/raw_v [B,Nr,Hkv,D]; lat_k/lat_v [B,Nl,1,R];
    biases [Hkv*D] or None (fa2_decode.py:157-163: the K bias shifts the latent
    LSE by (q . b_k) * scale, the V bias adds to the lifted output); fp32."""
    raw_out, raw_lse = eager_forward(q_rot.transpose(1, 2), raw_k, raw_v, scale)
    latent_q = project_query(q_rot, up_k, kv_heads)
    lat_out, lat_lse = eager_forward(latent_q.transpose(1, 2), lat_k, lat_v, scale)
    lat_out = project_value(lat_out.transpose(1, 2), up_v, kv_heads)
    heads, dim = q_rot.shape[1], q_rot.shape[-1]
    if up_k_bias is not None:
        bias = up_k_bias.reshape(kv_heads, dim).repeat_interleave(heads // kv_heads, dim=0)
        lat_lse = lat_lse + (q_rot.float() * bias[None, :, None].float()).sum(-1) * scale
    if up_v_bias is not None:
        bias = up_v_bias.reshape(kv_heads, dim).repeat_interleave(heads // kv_heads, dim=0)
        lat_out = lat_out + bias[None, :, None].float()
    total = torch.logaddexp(raw_lse, lat_lse)
    return (torch.exp(raw_lse - total)[..., None] * raw_out.transpose(1, 2)
            + torch.exp(lat_lse - total)[..., None] * lat_out)


def rotate(x, cos, sin):
    """x * cos + rotate_half(x) * sin in fp32 (modeling_utils.py:347-351, 386-389)."""
    half = x.shape[-1] // 2
    return x * cos + torch.cat([-x[..., half:], x[..., :half]], dim=-1) * sin


def recon_layer(q_rot, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale, kv_heads, cos_rows=None, sin_rows=None):
    """The reconstruction route in fp32 (LlamaAttention.forward after
    materialize, slimkv/llama3/modeling_llama.py:1405-1483, upcast as the
    eager softmax does): K = up_k(lat_k), rotated at the beacon positions when
    cos_rows / sin_rows [Nl, D] are given, V = up_v(lat_v), attention over
    [beacons ; raw rows].  q_rot [B,H,L,D]; raw_k/raw_v [B,Nr,Hkv,D];
    lat_k/lat_v [B,Nl,R].  Returns out [B,L,H,D]."""
    batch, n, _ = lat_k.shape
    dim = up_k.shape[0] // kv_heads
    k = (lat_k @ up_k.T).reshape(batch, n, kv_heads, dim)
    if cos_rows is not None:
        k = rotate(k, cos_rows[None, :, None], sin_rows[None, :, None])
    v = (lat_v @ up_v.T).reshape(batch, n, kv_heads, dim)
    out, _ = eager_forward(q_rot.transpose(1, 2), torch.cat([k, raw_k], dim=1), torch.cat([v, raw_v], dim=1), scale)
    return out
