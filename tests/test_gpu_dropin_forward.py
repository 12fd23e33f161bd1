"""The attention-forward drop-ins against the oracle's restatement of the
reference forwards:

* slimkv_amd.recon_decode.forward -- the decode step of LlamaAttention.forward,
  LlamaSdpaAttention.forward and LlamaFlashAttention2.forward over a latent
  cache with the reconstruction backend (slimkv/llama3/modeling_llama.py:
  1384-1483, 1515-1541, 1641-1653): materialize, append the step's rows,
  beacon-aware RoPE, attention -- reached through each class's dispatch;
* slimkv_amd.qwen2.forward -- Qwen2FlashAttention2.forward / Qwen2Attention.forward
  (slimkv/qwen2/modeling_qwen2.py:699-779, :887-978) for prefill windows and
  decode steps, with and without unrotated beacon keys.

Each output is checked against the float64 attention and against the eager
formulation with the reference's bf16 score/probability roundings, within the
bf16 bar; the returned cache against the module's own projections.
"""
import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import rope as orope
from tests.helpers import assert_close, to_np

pytestmark = pytest.mark.gpu


class RotaryEmbedding:          # the type name the RoPE fusions recognise
    def __init__(self, rows, device):
        from slimkv_amd.workloads import rope_tables
        self.cos_cached, self.sin_cached = rope_tables(rows, 128, 500000.0, device)
        self.max_seq_len_cached = rows


def _linear(i, o, gen, device, bias=False, weight=None):
    lin = torch.nn.Linear(i, o, bias=bias, device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(weight if weight is not None else torch.randn(o, i, generator=gen, device=device) / i ** 0.5)
        if bias:
            lin.bias.copy_(0.2 * torch.randn(o, generator=gen, device=device))
    return lin


def _rope_oracle(q, k, positions, roles, sink, att):
    """Beacon-aware RoPE over the whole key set (prefill rule: queries at the
    last positions; beacon keys of the history prefix and roles 1/2 kept)."""
    c = to_np(att.rotary_emb.cos_cached).astype(np.float32)
    s = to_np(att.rotary_emb.sin_cached).astype(np.float32)
    return orope.prefill_rope(q.astype(np.float32), k.astype(np.float32), c, s, positions, roles, sink)


def _attend(q_rot, k_rot, v, causal):
    """(float64 attention, reference eager bf16 formulation): BHSD in, BSHD out."""
    B, H, L, D = q_rot.shape
    exact, _ = oa.eager_forward(q_rot.transpose(0, 2, 1, 3), k_rot.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3),
                                1 / math.sqrt(D), causal=causal)
    N = k_rot.shape[2]
    mask = None
    if causal and L > 1:
        mask = np.zeros((B, 1, L, N))
        mask[:, :, np.arange(N)[None, :] > (np.arange(L)[:, None] + N - L)] = -np.inf
    eager, _ = oa.eager_recon_layer(q_rot, k_rot, v, 1 / math.sqrt(D), mask)
    return exact, eager.transpose(0, 2, 1, 3)


# ----------------------------------------------------------------------------- reconstruction decode

def _llama_module(device, skip_beacon_rope, seed):
    from slimkv_amd.workloads import block_diagonal, orthonormal_columns
    H, Hk, D, hidden, r = 8, 2, 128, 256, 32
    gen = torch.Generator(device=device).manual_seed(seed)
    up = [block_diagonal([orthonormal_columns(D, r, torch.Generator().manual_seed(seed + 10 * j + i))
                          for i in range(Hk)]).to(device, torch.bfloat16) for j in range(2)]
    config = SimpleNamespace(beacon_param=['q', 'k', 'v'], beacon_decode_backend='reconstruct', beacon_sink_size=1,
                             beacon_skip_rope_for_beacon_k=skip_beacon_rope, _slimkv_decode_step=True,
                             _attn_implementation='eager')
    att = SimpleNamespace(
        config=config, num_heads=H, num_key_value_heads=Hk, head_dim=D, hidden_size=H * D, training=False,
        q_proj=_linear(hidden, H * D, gen, device), k_proj=_linear(hidden, Hk * D, gen, device),
        v_proj=_linear(hidden, Hk * D, gen, device), beacon_q_proj=_linear(hidden, H * D, gen, device),
        beacon_k_down_proj=_linear(hidden, Hk * r, gen, device), beacon_v_down_proj=_linear(hidden, Hk * r, gen, device),
        beacon_k_up_proj=_linear(Hk * r, Hk * D, gen, device, weight=up[0]),
        beacon_v_up_proj=_linear(Hk * r, Hk * D, gen, device, weight=up[1]),
        rotary_emb=RotaryEmbedding(4096, device))
    att._use_shared_kv_down_proj = lambda: False
    att.o_proj_with_beacon = lambda output, size, indices: output
    return att, gen


def _eager_class(att, hidden, positions, past, output_attentions=False):
    """The top of LlamaAttention.forward (modeling_llama.py:1399-1406) with
    the reconstruction-decode hook ahead of the latent-decode branch."""
    from slimkv_amd import fa2_decode, recon_decode
    if recon_decode.eligible(att, hidden, past, output_attentions):
        return recon_decode.forward(att, hidden, positions, past)
    if fa2_decode.eligible(att, hidden, past, output_attentions):
        return fa2_decode.decode(att, hidden, positions, past)
    raise LookupError('the decode step fell through to materialize')


def _sdpa_class(att, hidden, positions, past, output_attentions=False):
    """The top of LlamaSdpaAttention.forward (:1515-1541): with
    output_attentions it runs the eager class's forward; otherwise the same
    hook before its latent-decode branch."""
    from slimkv_amd import fa2_decode, recon_decode
    if output_attentions:
        return _eager_class(att, hidden, positions, past, output_attentions)
    if recon_decode.eligible(att, hidden, past, output_attentions):
        return recon_decode.forward(att, hidden, positions, past)
    if fa2_decode.eligible(att, hidden, past, output_attentions):
        return fa2_decode.decode(att, hidden, positions, past)
    raise LookupError('the decode step fell through to materialize')


def _fa2_class(att, hidden, positions, past, output_attentions=False):
    """The top of LlamaFlashAttention2.forward (:1641-1653): output_attentions
    forced off, the hook for decode steps (q_len <= 2) ahead of the
    latent-decode branch and the join-prefill."""
    from slimkv_amd import fa2_decode, recon_decode
    output_attentions = False
    if recon_decode.eligible(att, hidden, past, output_attentions):
        return recon_decode.forward(att, hidden, positions, past)
    if fa2_decode.eligible(att, hidden, past, output_attentions):
        return fa2_decode.decode(att, hidden, positions, past)
    raise LookupError('the decode step fell through to materialize')


CLASSES = {'eager': _eager_class, 'sdpa': _sdpa_class, 'flash_attention_2': _fa2_class}


@pytest.mark.parametrize('skip_beacon_rope', [False, True])
@pytest.mark.parametrize('size', [0, 1])
@pytest.mark.parametrize('implementation', list(CLASSES))
def test_recon_decode_forward_matches_reference_semantics(device, skip_beacon_rope, size, implementation):
    """The reconstruction backend's decode step through each Llama attention
    class's dispatch (eager, SDPA, FlashAttention-2 -- the reference
    materialises and calls its own attention in each; here every class takes
    the same HIP forward), against the reference semantics."""
    from slimkv_amd.memory import ReconstructionCache
    from slimkv_amd.recon_decode import eligible
    att, gen = _llama_module(device, skip_beacon_rope, seed=11 + size + 2 * skip_beacon_rope)
    att.config._attn_implementation = implementation
    B, Hk, D, r, S, n_hist, L = 3, 2, 128, 32, 1, 300, size + 1
    roles = torch.zeros(45, dtype=torch.bool)
    roles[4::5] = True                                        # 9 window beacons among 36 raw rows
    n_win, n_raw = int(roles.sum()), int((~roles).sum())
    rnd = lambda *s: torch.randn(*s, generator=gen, device=device).to(torch.bfloat16)
    sink = rnd(B, Hk, S, D), rnd(B, Hk, S, D)
    hist = rnd(B, Hk, n_hist, r), rnd(B, Hk, n_hist, r)        # reconstruction backend packing [B, Hk, n, r]
    win = rnd(B, Hk, n_win, r), rnd(B, Hk, n_win, r)
    raw = rnd(B, Hk, n_raw, D), rnd(B, Hk, n_raw, D)
    raw_idx = (~roles).nonzero().flatten().to(device)
    pk = ReconstructionCache(sink[0], hist[0], raw[0], win[0], roles.to(device), Hk, D, 'k', raw_idx)
    pv = ReconstructionCache(sink[1], hist[1], raw[1], win[1], roles.to(device), Hk, D, 'v', raw_idx)
    N = S + n_hist + roles.numel() + L
    positions = torch.arange(N, device=device)[None].expand(B, -1)
    indices = torch.cat([roles.long(), torch.tensor([0] + [1] * size)]).to(device)
    hidden = (0.5 * torch.randn(B, L, 256, generator=gen, device=device)).to(torch.bfloat16)
    assert eligible(att, hidden, (pk, pv, size, indices), False)
    with torch.no_grad():
        out, none, update = CLASSES[implementation](att, hidden, positions, (pk, pv, size, indices))
        torch.cuda.synchronize()
        q = att.q_proj(hidden)
        k, v = att.k_proj(hidden), att.v_proj(hidden)
        if size:
            q[:, 1:] = att.beacon_q_proj(hidden[:, 1:])
            kl, vl = att.beacon_k_down_proj(hidden[:, 1:]), att.beacon_v_down_proj(hidden[:, 1:])
            k[:, 1:], v[:, 1:] = att.beacon_k_up_proj(kl), att.beacon_v_up_proj(vl)
    assert none is None
    # the cache update: the step's pre-RoPE K/V and the new beacon's packed latents
    assert torch.equal(update[0], k.view(B, L, Hk, D).transpose(1, 2))
    assert torch.equal(update[1], v.view(B, L, Hk, D).transpose(1, 2))
    if size:
        assert torch.equal(update.key_latents, kl.view(B, 1, Hk, r).transpose(1, 2))
        assert torch.equal(update.value_latents, vl.view(B, 1, Hk, r).transpose(1, 2))
    else:
        assert update.key_latents is None
    # oracle: the reference forward (materialize, append, RoPE, eager attention)
    glob = lambda t: to_np(t).transpose(0, 2, 1, 3).reshape(B, 1, t.shape[2], Hk * r)
    kw = dict(kv_heads=Hk, head_dim=D)
    K = oa.materialize(to_np(sink[0]), glob(hist[0]), to_np(raw[0]), glob(win[0]), roles.numpy(),
                       to_np(att.beacon_k_up_proj.weight), None, current=to_np(k.view(B, L, Hk, D).transpose(1, 2)), **kw)
    V = oa.materialize(to_np(sink[1]), glob(hist[1]), to_np(raw[1]), glob(win[1]), roles.numpy(),
                       to_np(att.beacon_v_up_proj.weight), None, current=to_np(v.view(B, L, Hk, D).transpose(1, 2)), **kw)
    qn = to_np(q).reshape(B, L, 8, D).transpose(0, 2, 1, 3)
    if skip_beacon_rope:
        q_rot, k_rot = _rope_oracle(qn, K, positions.cpu().numpy(), indices.cpu().numpy(), S, att)
    else:
        q_rot, k_rot = _rope_oracle(qn, K, positions.cpu().numpy(), np.zeros(N, np.int64), 0, att)
    exact, eager = _attend(q_rot.astype(np.float64), k_rot.astype(np.float64), V, causal=bool(size))
    got = to_np(out).reshape(B, L, 8, D)
    assert_close(got, exact, what='vs float64')
    assert_close(got, eager, what='vs eager bf16')


# ----------------------------------------------------------------------------- Qwen2

def _qwen2_module(device, skip_beacon_rope, seed):
    """Qwen2.5-14B head grouping (GQA 5) at a small width, q/k/v biases, full-dim
    beacon projections; qkv_proj_with_beacon picks per row by role."""
    H, Hk, D, hidden = 10, 2, 128, 256
    gen = torch.Generator(device=device).manual_seed(seed)
    lin = lambda i, o, b=False: _linear(i, o, gen, device, bias=b)
    config = SimpleNamespace(beacon_param=['q', 'k', 'v'], beacon_sink_size=1,
                             beacon_skip_rope_for_beacon_k=skip_beacon_rope)
    att = SimpleNamespace(config=config, num_heads=H, num_key_value_heads=Hk, head_dim=D, hidden_size=H * D,
                          is_causal=True, q_proj=lin(hidden, H * D, True), k_proj=lin(hidden, Hk * D, True),
                          v_proj=lin(hidden, Hk * D, True), beacon_q_proj=lin(hidden, H * D, True),
                          beacon_k_proj=lin(hidden, Hk * D, True), beacon_v_proj=lin(hidden, Hk * D, True),
                          rotary_emb=RotaryEmbedding(4096, device))

    def qkv(h, size, indices):
        if size <= 0:
            return att.q_proj(h), att.k_proj(h), att.v_proj(h)
        beacon = (indices[-h.shape[1]:] != 0)[:, None]
        return (torch.where(beacon, att.beacon_q_proj(h), att.q_proj(h)),
                torch.where(beacon, att.beacon_k_proj(h), att.k_proj(h)),
                torch.where(beacon, att.beacon_v_proj(h), att.v_proj(h)))
    att.qkv_proj_with_beacon = qkv
    att.o_proj_with_beacon = lambda output, size, indices: output
    return att, gen


@pytest.mark.parametrize('skip_beacon_rope', [True, False])
@pytest.mark.parametrize('L,n_past', [(64, 70), (1, 300), (2, 301), (40, 0)])
def test_qwen2_forward_matches_reference_semantics(device, skip_beacon_rope, L, n_past):
    from slimkv_amd.qwen2 import forward
    att, gen = _qwen2_module(device, skip_beacon_rope, seed=5 + L)
    B, Hk, D, S = 2, 2, 128, 1
    n_hist = 20 if n_past else 0
    n_raw_past = max(n_past - S - n_hist, 0)
    rnd = lambda *s: torch.randn(*s, generator=gen, device=device).to(torch.bfloat16)
    past_k = rnd(B, Hk, n_past, D) if n_past else None
    past_v = rnd(B, Hk, n_past, D) if n_past else None
    roles = torch.zeros(n_raw_past + L, dtype=torch.long)
    roles[4::5] = 1                                           # beacons among the window's rows
    size = int(roles[-L:].sum())
    N = n_past + L
    positions = torch.arange(N, device=device)[None].expand(B, -1)
    hidden = (0.5 * torch.randn(B, L, 256, generator=gen, device=device)).to(torch.bfloat16)
    indices = roles.to(device)
    with torch.no_grad():
        out, none, cache = forward(att, hidden, None, positions, (past_k, past_v, size, indices))
        torch.cuda.synchronize()
        q, k, v = att.qkv_proj_with_beacon(hidden, size, indices)
    assert none is None and cache[2] == size
    assert torch.equal(cache[0], k.view(B, L, Hk, D).transpose(1, 2))
    K = to_np(k.view(B, L, Hk, D).transpose(1, 2))
    V = to_np(v.view(B, L, Hk, D).transpose(1, 2))
    if n_past:
        K = np.concatenate([to_np(past_k), K], axis=2)
        V = np.concatenate([to_np(past_v), V], axis=2)
    qn = to_np(q).reshape(B, L, 10, D).transpose(0, 2, 1, 3)
    if skip_beacon_rope and size > 0:
        q_rot, k_rot = _rope_oracle(qn, K, positions.cpu().numpy(), roles.numpy(), S, att)
    else:
        q_rot, k_rot = _rope_oracle(qn, K, positions.cpu().numpy(), np.zeros(N, np.int64), 0, att)
    exact, eager = _attend(q_rot.astype(np.float64), k_rot.astype(np.float64), V, causal=True)
    got = to_np(out).reshape(B, L, 10, D)
    assert_close(got, exact, what='vs float64')
    assert_close(got, eager, what='vs eager bf16')


def test_qwen2_rejects_padding_masks(device):
    from slimkv_amd.qwen2 import flash_attention_forward
    att, _ = _qwen2_module(device, False, 3)
    q = torch.zeros(1, 3, 10, 128, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match='mask'):
        flash_attention_forward(att, q, q[:, :, :2], q[:, :, :2], torch.ones(1, 3, device=device), 3)
