"""StaticDecode on the GPU (slimkv/llama3/static_decode.py:43-287): a captured
decode step replays bit-identically to the same step run eagerly (the
reference checks graph == eager bitwise, tools/validate_b1_decode.py:56-57),
the step's attention equals the drop-in decode (fa2_decode.decode, itself
checked against the oracle) over the same cache, and commit publishes the
memory views the ordinary path reads next."""
from types import SimpleNamespace

import pytest
import torch

from tests.helpers import assert_close, to_np
from tests.test_gpu_dropin import RotaryEmbedding, _attention

pytestmark = pytest.mark.gpu

H, HKV, D, RANK, HIDDEN, VOCAB = 8, 2, 128, 32, 1024, 64


class _Memory:
    def __init__(self, layers):
        self._static_decode_epoch = 1
        self._is_full_window = False
        self._decode_uncompressed = False
        self._fast_decode_active = True
        self._fast_window_roles = None
        self._fast_window_raw_indices = None
        self.sink_activations = [(None, None)] * layers
        self.beacon_activations = [(None, None)] * layers
        self.raw_activations = [(None, None)] * layers
        self.window_beacon_activations = [(None, None)] * layers


def _model(device, layers=2):
    gen = torch.Generator(device=device).manual_seed(1)
    blocks = []
    for i in range(layers):
        att, _ = _attention(device, True, True, seed=20 + i)
        att.config.beacon_param = ['q', 'k', 'v']
        att.rotary_emb = RotaryEmbedding(4096, device)
        att.o_proj = torch.nn.Identity()
        blocks.append(SimpleNamespace(input_layernorm=torch.nn.Identity(), self_attn=att,
                                      _decode_tail=lambda out, res: res + out))
    embed = torch.nn.Embedding(VOCAB, HIDDEN, device=device, dtype=torch.bfloat16)
    beacon_embed = torch.nn.Embedding(1, HIDDEN, device=device, dtype=torch.bfloat16)
    lm_head = torch.nn.Linear(HIDDEN, VOCAB, bias=False, device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        for p in (embed.weight, beacon_embed.weight, lm_head.weight):
            p.copy_(torch.randn(p.shape, generator=gen, device=device) * 0.05)
    config = SimpleNamespace(beacon_window=16, beacon_sink_size=1, vocab_size=VOCAB, beacon_param=['q', 'k', 'v'])
    return SimpleNamespace(device=device, dtype=torch.bfloat16, config=config, memory=_Memory(layers),
                           model=SimpleNamespace(embed_tokens=embed, beacon_embed_tokens=beacon_embed,
                                                 layers=blocks, norm=torch.nn.Identity()),
                           lm_head=lm_head)


def _past(device, model, n_hist=8, n_raw=5, n_win=1):
    from slimkv_amd.memory import ReconstructionCache
    gen = torch.Generator(device=device).manual_seed(5)
    rnd = lambda *s: torch.randn(*s, generator=gen, device=device).to(torch.bfloat16)
    roles = torch.zeros(n_raw + n_win, dtype=torch.bool, device=device)
    roles[4::5] = True
    raw_idx = (~roles).nonzero().flatten()
    past = []
    for _ in model.model.layers:
        pk = ReconstructionCache(rnd(1, HKV, 1, D), rnd(1, 1, n_hist, HKV * RANK), rnd(1, HKV, n_raw, D),
                                 rnd(1, 1, n_win, HKV * RANK), roles, HKV, D, 'k', raw_idx)
        pv = ReconstructionCache(rnd(1, HKV, 1, D), rnd(1, 1, n_hist, HKV * RANK), rnd(1, HKV, n_raw, D),
                                 rnd(1, 1, n_win, HKV * RANK), roles, HKV, D, 'v', raw_idx)
        past.append((pk, pv, 0, None))
    return past


@pytest.mark.parametrize('size', [0, 1])
def test_graph_replay_equals_eager_and_drop_in_decode(device, size):
    from slimkv_amd import fa2_decode
    from slimkv_amd.static_decode import StaticDecode
    model = _model(device)
    past = _past(device, model)
    keys = 1 + 8 + 6
    ids = torch.tensor([[7] + [VOCAB] * size], device=device)
    positions = torch.arange(keys + 1 + size, device=device)[None]
    static = StaticDecode(model, capacity=64)
    with torch.no_grad():
        logits = static.run(ids, positions, past)
        eager = static.forward(ids, positions[:, -ids.shape[1]:])
        torch.cuda.synchronize()
    assert torch.equal(logits, eager), 'graph replay differs from the eager step'
    # the attention of layer 0 equals the drop-in decode over the same cache
    layer = model.model.layers[0]
    hidden = model.model.embed_tokens(ids[:, :1])
    if size:
        hidden = torch.cat([hidden, model.model.beacon_embed_tokens(ids[:, 1:] - VOCAB)], dim=1)
    att = layer.self_attn
    att.config._slimkv_decode_step = True
    with torch.no_grad():
        want, _, _ = fa2_decode.decode(att, hidden, positions, (past[0][0], past[0][1], size,
                                                                torch.zeros(7 + size, dtype=torch.long, device=device)))
        static_caches = static.caches[0]
        q = att.q_proj(hidden)
        if size:
            q = torch.cat([q[:, :1], att.beacon_q_proj(hidden[:, 1:])], dim=1)
        from slimkv_amd import kernels
        q_rot, _ = kernels.rope_decode(q.view(1, 1 + size, H, D).transpose(1, 2), q.new_zeros(1, HKV, 1, D),
                                       att.rotary_emb.cos_cached, att.rotary_emb.sin_cached,
                                       positions[:, -ids.shape[1]:].contiguous(), None, 0, 0)
        got, _ = static_caches.attend(q_rot.transpose(1, 2), att.beacon_k_up_proj.weight, att.beacon_v_up_proj.weight,
                                      D ** -0.5, q_positions=None, cos=None, sin=None, size=size,
                                      up_k_bias=att.beacon_k_up_proj.bias, up_v_bias=att.beacon_v_up_proj.bias)
    torch.cuda.synchronize()
    assert_close(to_np(got.reshape(1, 1 + size, HIDDEN)), to_np(want))
    mem = model.memory
    assert mem.raw_activations[0][0].shape == (1, HKV, 6, D)              # 5 window raw rows + the new token
    assert mem.window_beacon_activations[0][0].shape[2] == 1 + size
    assert mem.beacon_activations[0][0].shape == (1, 1, 8, HKV * RANK)
    assert static.cache_bytes()['raw'] == 2 * 6 * (2 * HKV * D * 2)        # two layers, 6 raw rows
