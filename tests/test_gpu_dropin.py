"""The drop-in modules on the GPU against the oracle.

decode (slimkv/llama3/fa2_decode.py:77-166) runs with a small attention module
(8 query / 2 KV heads, head_dim 128, block-diagonal or general up-projections,
with and without biases) over a ReconstructionCache holding sinks, history
latents, an open window of raw tokens and window beacons.  The oracle uses the
same projections (computed once by torch), rotates with the bf16-exact rule and
restates the reference branch algebra with its bf16 roundings.
"""
import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import rope as orope
from oracle.bf16 import to_bits
from slimkv_amd.workloads import block_diagonal, orthonormal_columns, rope_tables
from tests.helpers import assert_close, bits, to_np

pytestmark = pytest.mark.gpu

H, HKV, D, RANK = 8, 2, 128, 32
HIDDEN = H * D


class RotaryEmbedding:          # the type name the decode path recognises
    def __init__(self, rows, device):
        self.cos_cached, self.sin_cached = rope_tables(rows, D, 500000.0, device)
        self.max_seq_len_cached = rows


def _linear(i, o, gen, device, bias=False, weight=None):
    lin = torch.nn.Linear(i, o, bias=bias, device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(weight if weight is not None else torch.randn(o, i, generator=gen, device=device) / i ** 0.5)
        if bias:
            lin.bias.copy_(0.3 * torch.randn(o, generator=gen, device=device))
    return lin


def _attention(device, bd=True, bias=False, seed=0):
    gen = torch.Generator(device=device).manual_seed(seed)
    R = HKV * RANK
    if bd:
        uk = block_diagonal([orthonormal_columns(D, RANK, torch.Generator().manual_seed(seed + i)) for i in range(HKV)])
        uv = block_diagonal([orthonormal_columns(D, RANK, torch.Generator().manual_seed(seed + 9 + i))
                             for i in range(HKV)])
        uk, uv = uk.to(device, torch.bfloat16), uv.to(device, torch.bfloat16)
    else:
        uk = uv = None
    att = SimpleNamespace(
        config=SimpleNamespace(beacon_param=['q', 'k', 'v'], _slimkv_decode_step=True, beacon_decode_backend='fa2',
                               _attn_implementation='flash_attention_2'),
        num_heads=H, num_key_value_heads=HKV, head_dim=D, hidden_size=HIDDEN, training=False,
        q_proj=_linear(HIDDEN, H * D, gen, device), k_proj=_linear(HIDDEN, HKV * D, gen, device),
        v_proj=_linear(HIDDEN, HKV * D, gen, device), beacon_q_proj=_linear(HIDDEN, H * D, gen, device),
        beacon_k_down_proj=_linear(HIDDEN, R, gen, device), beacon_v_down_proj=_linear(HIDDEN, R, gen, device),
        beacon_k_up_proj=_linear(R, HKV * D, gen, device, bias, uk),
        beacon_v_up_proj=_linear(R, HKV * D, gen, device, bias, uv),
        rotary_emb=RotaryEmbedding(2048, device))
    att._use_shared_kv_down_proj = lambda: False
    att.o_proj_with_beacon = lambda output, size, indices: output
    return att, gen


def _cache(device, gen, B, n_sink=1, n_hist=40, n_raw=5, n_win=1):
    from slimkv_amd.memory import ReconstructionCache
    R = HKV * RANK
    rnd = lambda *s: torch.randn(*s, generator=gen, device=device).to(torch.bfloat16)
    sink_k, sink_v = rnd(B, HKV, n_sink, D), rnd(B, HKV, n_sink, D)
    hist_k, hist_v = rnd(B, 1, n_hist, R), rnd(B, 1, n_hist, R)
    raw_k, raw_v = rnd(B, HKV, n_raw, D), rnd(B, HKV, n_raw, D)
    win_k, win_v = rnd(B, 1, n_win, R), rnd(B, 1, n_win, R)
    roles = torch.zeros(n_raw + n_win, dtype=torch.bool, device=device)
    roles[4::5] = True                                         # one beacon after every 4 raw tokens
    raw_idx = (~roles).nonzero().flatten()
    pk = ReconstructionCache(sink_k, hist_k, raw_k, win_k, roles, HKV, D, 'k', raw_idx)
    pv = ReconstructionCache(sink_v, hist_v, raw_v, win_v, roles, HKV, D, 'v', raw_idx)
    return pk, pv


def _oracle_decode(att, hidden, position_ids, pk, pv, size):
    B, L, _ = hidden.shape
    with torch.no_grad():
        q = att.q_proj(hidden)
        if size:
            q = torch.cat([q[:, :1], att.beacon_q_proj(hidden[:, 1:])], dim=1)
        new_k = att.k_proj(hidden[:, :1]).reshape(B, 1, HKV, D).transpose(1, 2)
        new_v = att.v_proj(hidden[:, :1]).reshape(B, 1, HKV, D).transpose(1, 2)
        kl = att.beacon_k_down_proj(hidden[:, 1:]).unsqueeze(1) if size else None
        vl = att.beacon_v_down_proj(hidden[:, 1:]).unsqueeze(1) if size else None
    q = to_np(q.reshape(B, L, H, D).transpose(1, 2)).astype(np.float32)
    raw_k = np.concatenate([to_np(pk.sink), to_np(pk.raw), to_np(new_k)], axis=2).astype(np.float32)
    raw_v = np.concatenate([to_np(pv.sink), to_np(pv.raw), to_np(new_v)], axis=2)
    lat_k = np.concatenate([to_np(pk.history), to_np(pk.window)] + ([to_np(kl)] if size else []), axis=2)
    lat_v = np.concatenate([to_np(pv.history), to_np(pv.window)] + ([to_np(vl)] if size else []), axis=2)
    c = to_np(att.rotary_emb.cos_cached).astype(np.float32)
    s = to_np(att.rotary_emb.sin_cached).astype(np.float32)
    sink, hist = pk.sink.shape[2], pk.history.shape[2]
    q_rot, k_rot = orope.rope_decode(q, raw_k, c, s, position_ids[:, -L:].cpu().numpy(),
                                     pk.window_raw_indices.cpu().numpy(), sink, hist)
    uk, uv = att.beacon_k_up_proj, att.beacon_v_up_proj
    out, _ = oa.latent_layer(q_rot, k_rot, raw_v, lat_k, lat_v, to_np(uk.weight), to_np(uv.weight), 1 / math.sqrt(D),
                             HKV, None if uk.bias is None else to_np(uk.bias),
                             None if uv.bias is None else to_np(uv.bias), lat_causal=bool(size))
    return out.transpose(0, 2, 1, 3).reshape(B, L, HIDDEN)


@pytest.mark.parametrize('bd,bias', [(True, False), (True, True), (False, True)])
@pytest.mark.parametrize('size', [0, 1])
def test_decode_matches_oracle(device, bd, bias, size):
    from slimkv_amd import fa2_decode
    att, gen = _attention(device, bd, bias, seed=3 + size)
    B = 3
    pk, pv = _cache(device, gen, B)
    L = 1 + size
    hidden = (torch.randn(B, L, HIDDEN, generator=gen, device=device) * 0.5).to(torch.bfloat16)
    total = 1 + 40 + 6 + L
    position_ids = torch.arange(total, device=device)[None].expand(B, -1)
    indices = torch.zeros(7 + size, dtype=torch.long, device=device)
    with torch.no_grad():
        out, none, update = fa2_decode.decode(att, hidden, position_ids, (pk, pv, size, indices))
        two, _, _ = fa2_decode.decode(att, hidden, position_ids, (pk, pv, size, indices),
                                      forward=fa2_decode.flash_forward)
    torch.cuda.synchronize()
    assert none is None and update.raw_only and update[2] == size
    assert (update.key_latents is None) == (size == 0)
    expected = _oracle_decode(att, hidden, position_ids, pk, pv, size)
    assert_close(to_np(out), expected, what='fused')
    assert_close(to_np(two), expected, what='two-branch')


def test_materialize_matches_oracle(device):
    att, gen = _attention(device, True, True, seed=11)
    pk, _ = _cache(device, gen, 2, n_sink=1, n_hist=23, n_raw=9, n_win=2)
    cur = torch.randn(2, HKV, 1, D, generator=gen, device=device).to(torch.bfloat16)
    got = pk.materialize(att, cur)
    torch.cuda.synchronize()
    uk = att.beacon_k_up_proj
    want = oa.materialize(to_np(pk.sink), to_np(pk.history), to_np(pk.raw), to_np(pk.window),
                          pk.window_roles.cpu().numpy(), to_np(uk.weight), to_np(uk.bias), HKV, D, to_np(cur))
    exact = oa.materialize(to_np(pk.sink), to_np(pk.history), to_np(pk.raw), to_np(pk.window),
                           pk.window_roles.cpu().numpy(), to_np(uk.weight), to_np(uk.bias), HKV, D, to_np(cur),
                           bf16_boundaries=False)
    assert got.shape == want.shape
    mag = np.maximum(np.abs(exact), 1e-30)
    assert (np.abs(to_np(got) - exact) < 2.0 ** (np.floor(np.log2(mag)) - 7) * 1.0001).all()
    assert (to_np(got) == want).mean() > 0.98


def test_extension_forward_and_paired_attention(device):
    import sys
    sys.path.insert(0, 'slimkv_amd/fa2ext')
    import slimkv_fa2_decode_320 as ext
    from slimkv_amd.paired_decode import paired_attention
    gen = torch.Generator(device=device).manual_seed(2)
    q = torch.randn(1, 2, 32, 256, generator=gen, device=device).to(torch.bfloat16)
    # a padded cache buffer: 77 valid rows of 100
    k = torch.randn(1, 100, 1, 256, generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn(1, 100, 1, 256, generator=gen, device=device).to(torch.bfloat16)
    lengths = torch.tensor([76, 77], dtype=torch.int32, device=device)
    out, lse = paired_attention(ext.forward, q, k, v, 0.0625, lengths, 256)
    # the non-paired causal launch (StaticDecode's other branch): the same bits
    uo, ul = ext.forward(q, k, v, 0.0625, True, 0, True, lengths[1:])
    torch.cuda.synchronize()
    assert torch.equal(out, uo) and torch.equal(lse, ul)
    eo, el = oa.eager_forward(to_np(q), to_np(k[:, :77]), to_np(v[:, :77]), 0.0625, True)
    assert_close(to_np(out), eo)
    np.testing.assert_allclose(to_np(lse), el, atol=2e-3)
    # the raw query's row excludes the Beacon key: it equals a one-query launch over 76 keys
    ro, rl = ext.forward(q[:, :1], k[:, :76], v[:, :76], 0.0625, False)
    torch.cuda.synchronize()
    assert_close(to_np(out[:, :1]), to_np(ro))


def test_fused_prefill_rope_through_metadata(device):
    from slimkv_amd.prefill_ops import PrefillMetadata, fused_prefill_rope
    gen = torch.Generator(device=device).manual_seed(4)
    q = torch.randn(2, 8, 6, D, generator=gen, device=device).to(torch.bfloat16)
    k = torch.randn(2, 2, 14, D, generator=gen, device=device).to(torch.bfloat16)
    roles = torch.tensor([0, 0, 0, 0, 1, 0, 0, 2], device=device)
    positions = torch.arange(14, device=device)[None].expand(2, -1)
    meta = PrefillMetadata((roles == 0).nonzero().flatten(), (roles != 0).nonzero().flatten(), roles, positions,
                           True)
    rope = RotaryEmbedding(64, device)
    oq, ok = fused_prefill_rope(q, k, rope, meta, 1)
    torch.cuda.synchronize()
    c, s = to_np(rope.cos_cached).astype(np.float32), to_np(rope.sin_cached).astype(np.float32)
    eq, ek = orope.prefill_rope(to_np(q).astype(np.float32), to_np(k).astype(np.float32), c, s,
                                positions.cpu().numpy(), roles.cpu().numpy(), 1)
    assert (bits(oq) == to_bits(eq)).all() and (bits(ok) == to_bits(ek)).all()
