"""Attention algebra of the hot path (oracle, numpy float64 unless stated).

eager_forward     slimkv/llama3/latent_decode.py:16-41
project_query     slimkv/llama3/fa2_decode.py:41-46
project_value     slimkv/llama3/fa2_decode.py:49-54
merge_attention   slimkv/llama3/fa2_decode.py:57-66 (torch branch) and
                  slimkv/llama3/decode_kernels.py:53-75 (fused branch)
latent_layer      slimkv/llama3/fa2_decode.py:143-164 (RoPE'd q and raw K given)
materialize       slimkv/llama3/memory.py:26-48
eager_recon_layer slimkv/llama3/modeling_llama.py:1431-1483 (LlamaAttention.forward
                  after materialize: cat, RoPE, repeat_kv, softmax in fp32)
"""
import numpy as np

from .bf16 import round_bf16


def _logsumexp(x, axis=-1):
    m = np.max(x, axis=axis, keepdims=True)
    finite = np.isfinite(m)
    safe = np.where(finite, m, 0.0)
    with np.errstate(divide='ignore'):
        out = np.log(np.sum(np.exp(x - safe), axis=axis, keepdims=True)) + safe
    out = np.where(finite, out, -np.inf)
    return np.squeeze(out, axis=axis)


def eager_forward(q, k, v, scale, causal=False, dtype=np.float64):
    """q [B,Q,H,R], k [B,N,Hk,R], v [B,N,Hk,Rv] -> (out [B,Q,H,Rv], lse [B,H,Q]).

    Query heads are grouped per KV head without expanding K/V (latent_decode.py:23-25);
    bottom-right causality (:29-33); rows with no visible key get zero output and
    LSE -inf (:36-37).  Output is left in `dtype` (the caller rounds).
    """
    q, k, v = (np.asarray(x, dtype=dtype) for x in (q, k, v))
    B, Q, H, R = q.shape
    N, Hk = k.shape[1], k.shape[2]
    if k.shape[0] != B or k.shape[-1] != R or v.shape[:3] != k.shape[:3] or Hk < 1 or H % Hk or N < 1:
        raise ValueError('Invalid eager attention shapes or GQA head counts.')
    g = H // Hk
    grouped = q.transpose(0, 2, 1, 3).reshape(B, Hk, g * Q, R)
    scores = (grouped @ k.transpose(0, 2, 3, 1)) * scale
    scores = scores.reshape(B, H, Q, N)
    if causal:
        qpos = np.arange(Q) + N - Q
        mask = np.arange(N)[None, :] > qpos[:, None]
        scores = np.where(mask, -np.inf, scores)
    lse = _logsumexp(scores)
    finite = np.isfinite(lse)[..., None]
    probs = np.where(finite, np.exp(scores - np.where(finite, lse[..., None], 0.0)), 0.0)
    out = probs.reshape(B, Hk, g * Q, N) @ v.transpose(0, 2, 1, 3)
    out = out.reshape(B, H, Q, v.shape[-1]).transpose(0, 2, 1, 3)
    return out, lse


def repeat_kv_forward(q, k, v, scale, causal=False):
    """The same attention by explicit K/V head repetition (the reference test
    oracle `reference_forward`, tests/test_llama_fa2_decode.py:14-23)."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    rep = q.shape[2] // k.shape[2]
    k = np.repeat(k, rep, axis=2)
    v = np.repeat(v, rep, axis=2)
    logits = q.transpose(0, 2, 1, 3) @ k.transpose(0, 2, 3, 1) * scale
    if causal:
        mask = np.arange(k.shape[1])[None] > np.arange(q.shape[1])[:, None] + k.shape[1] - q.shape[1]
        logits = np.where(mask, -np.inf, logits)
    lse = _logsumexp(logits)
    with np.errstate(invalid='ignore'):
        probs = np.nan_to_num(np.exp(logits - lse[..., None]))
    return (probs @ v.transpose(0, 2, 1, 3)).transpose(0, 2, 1, 3), lse


def project_query(q, weight, kv_heads):
    """q [B,H,L,D] @ W_k.reshape(Hkv,D,R) per KV group -> [B,H,L,R] (fa2_decode.py:41-46)."""
    B, H, L, D = q.shape
    R = weight.shape[-1]
    grouped = np.asarray(q, dtype=np.float64).reshape(B, kv_heads, H // kv_heads * L, D)
    w = np.asarray(weight, dtype=np.float64).reshape(kv_heads, D, R)
    return (grouped @ w).reshape(B, H, L, R)


def project_value(out, weight, kv_heads):
    """out [B,H,L,Rv] @ W_v.reshape(Hkv,D,Rv)^T per KV group -> [B,H,L,D] (fa2_decode.py:49-54)."""
    B, H, L, Rv = out.shape
    D = weight.shape[0] // kv_heads
    grouped = np.asarray(out, dtype=np.float64).reshape(B, kv_heads, H // kv_heads * L, Rv)
    w = np.asarray(weight, dtype=np.float64).reshape(kv_heads, D, Rv).transpose(0, 2, 1)
    return (grouped @ w).reshape(B, H, L, D)


def merge_attention(raw_out, raw_lse, latent_out, latent_lse):
    """t = logaddexp(r, l); out = e^{r-t} raw + e^{l-t} latent (fa2_decode.py:62-66)."""
    r = np.asarray(raw_lse, dtype=np.float64)
    l = np.asarray(latent_lse, dtype=np.float64)
    with np.errstate(invalid='ignore'):
        total = np.logaddexp(r, l)
        rw = np.exp(r - total)[..., None]
        lw = np.exp(l - total)[..., None]
    return rw * np.asarray(raw_out, np.float64) + lw * np.asarray(latent_out, np.float64)


def merge_fused_form(raw_out, raw_lse, latent_out, latent_lse):
    """The fused kernel's form t = max + log1p(exp(-|r-l|)) (decode_kernels.py:65-68)."""
    r = np.asarray(raw_lse, dtype=np.float64)
    l = np.asarray(latent_lse, dtype=np.float64)
    m = np.maximum(r, l)
    total = m + np.log1p(np.exp(-np.abs(r - l)))
    return (np.exp(r - total)[..., None] * np.asarray(raw_out, np.float64)
            + np.exp(l - total)[..., None] * np.asarray(latent_out, np.float64))


def latent_layer(q_rot, raw_k, raw_v, lat_k, lat_v, up_k, up_v, scale, kv_heads,
                 up_k_bias=None, up_v_bias=None, lat_causal=False, bf16_boundaries=True):
    """Attention core of fa2_decode.decode after RoPE (fa2_decode.py:145-164).

    q_rot [B,H,L,D] (RoPE'd), raw_k/raw_v [B,Hkv,Nr,D] (raw_k RoPE'd),
    lat_k [B,1,Nl,Rk], lat_v [B,1,Nl,Rv] (latent rows, no RoPE; Nl may be 0),
    up_k [Hkv*D,Rk], up_v [Hkv*D,Rv] (nn.Linear weights), biases [Hkv*D].
    With bf16_boundaries the model-dtype roundings of the reference bf16 path are
    applied: branch outputs, project_query/project_value results, bias add and
    the merged output.  Returns out [B,H,L,D] (float64 array of bf16 values when
    bf16_boundaries) and the merged LSE [B,H,L].
    """
    rnd = round_bf16 if bf16_boundaries else (lambda x: np.asarray(x, np.float64))
    B, H, L, D = q_rot.shape
    g = H // kv_heads
    raw_out, raw_lse = eager_forward(q_rot.transpose(0, 2, 1, 3), raw_k.transpose(0, 2, 1, 3),
                                     raw_v.transpose(0, 2, 1, 3), scale, False)
    raw_out = rnd(raw_out).transpose(0, 2, 1, 3)
    if lat_k is None or lat_k.shape[2] == 0:
        return np.asarray(raw_out, np.float64), raw_lse
    latent_q = rnd(project_query(q_rot, up_k, kv_heads))
    lat_out, lat_lse = eager_forward(latent_q.transpose(0, 2, 1, 3), lat_k.transpose(0, 2, 1, 3),
                                     lat_v.transpose(0, 2, 1, 3), scale, bool(lat_causal))
    lat_out = rnd(project_value(rnd(lat_out).transpose(0, 2, 1, 3), up_v, kv_heads))
    if up_k_bias is not None:
        bias = np.repeat(np.asarray(up_k_bias, np.float64).reshape(kv_heads, D), g, axis=0)
        lat_lse = lat_lse + (np.asarray(q_rot, np.float64) * bias[None, :, None]).sum(-1) * scale
    if up_v_bias is not None:
        bias = np.repeat(np.asarray(up_v_bias, np.float64).reshape(kv_heads, D), g, axis=0)
        lat_out = rnd(lat_out + bias[None, :, None])
    out = rnd(merge_attention(raw_out, raw_lse, lat_out, lat_lse))
    with np.errstate(invalid='ignore'):
        lse = np.logaddexp(raw_lse, lat_lse)
    return np.asarray(out, np.float64), lse


def reconstruct(latent, up, bias, kv_heads, head_dim, bf16_boundaries=True):
    """ReconstructionCache.materialize's up-projection (llama3/memory.py:29-36):
    latent [B,1,n,R] -> up(latent) -> [B,Hkv,n,D]."""
    rnd = round_bf16 if bf16_boundaries else (lambda x: np.asarray(x, np.float64))
    B, _, n, R = latent.shape
    full = np.asarray(latent, np.float64).reshape(B, n, R) @ np.asarray(up, np.float64).T
    if bias is not None:
        full = full + np.asarray(bias, np.float64)
    return np.asarray(rnd(full), np.float64).reshape(B, n, kv_heads, head_dim).transpose(0, 2, 1, 3)


def down_project(x, weight, rows=None, bf16_boundaries=True):
    """Beacon latents of the selected rows (modeling_llama.py:383-390 down
    projection, then the role selection of _incremental_cache :1355-1359):
    x [B,L,K] -> x[:, rows] @ weight^T -> [B,n,N]; a row index outside [0, L)
    gives a zero row (the HIP kernel's documented out-of-range behaviour)."""
    rnd = round_bf16 if bf16_boundaries else (lambda a: np.asarray(a, np.float64))
    x = np.asarray(x, np.float64)
    B, L, K = x.shape
    rows = np.arange(L) if rows is None else np.asarray(rows, np.int64)
    valid = (rows >= 0) & (rows < L)
    picked = np.where(valid[None, :, None], x[:, np.clip(rows, 0, L - 1)], 0.0)
    return np.asarray(rnd(picked @ np.asarray(weight, np.float64).T), np.float64)


def materialize(sink, history, raw, window, window_roles, up, bias, kv_heads, head_dim,
                current=None, bf16_boundaries=True):
    """[sink ; up(history) ; interleave(up(window), raw by roles) ; current] along keys
    (llama3/memory.py:26-48).  Tensors [B,Hkv,n,D] for sink/raw/current,
    [B,1,n,R] for history/window; window_roles bool [n_window + n_raw]."""
    parts = []
    if sink is not None:
        parts.append(np.asarray(sink, np.float64))
    if history is not None:
        parts.append(reconstruct(history, up, bias, kv_heads, head_dim, bf16_boundaries))
    if window is None:
        if raw is not None:
            parts.append(np.asarray(raw, np.float64))
    else:
        win = reconstruct(window, up, bias, kv_heads, head_dim, bf16_boundaries)
        roles = np.asarray(window_roles, bool)
        recent = np.empty(win.shape[:2] + (roles.size, head_dim))
        recent[:, :, roles] = win
        if raw is not None:
            recent[:, :, ~roles] = raw
        parts.append(recent)
    if current is not None:
        parts.append(np.asarray(current, np.float64))
    return np.concatenate(parts, axis=2)


def eager_recon_layer(q_rot, k_rot, v, scale, mask=None, bf16_boundaries=True):
    """LlamaAttention.forward's attention after RoPE (modeling_llama.py:1450-1483):
    bf16 QK^T, / sqrt(d) (given as scale), + mask, fp32 softmax cast to bf16,
    bf16 PV.  q_rot [B,H,L,D], k_rot/v [B,Hkv,N,D] -> out [B,H,L,D]."""
    rnd = round_bf16 if bf16_boundaries else (lambda x: np.asarray(x, np.float64))
    H, Hkv = q_rot.shape[1], k_rot.shape[1]
    k = np.repeat(np.asarray(k_rot, np.float64), H // Hkv, axis=1)
    vv = np.repeat(np.asarray(v, np.float64), H // Hkv, axis=1)
    scores = rnd(np.asarray(q_rot, np.float64) @ k.transpose(0, 1, 3, 2))
    scores = rnd(scores * scale) if bf16_boundaries else scores * scale
    if mask is not None:
        scores = scores + mask
    lse = _logsumexp(scores)
    probs = rnd(np.exp(scores - lse[..., None]))
    return np.asarray(rnd(probs @ vv), np.float64), lse
