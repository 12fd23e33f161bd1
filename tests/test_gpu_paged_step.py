"""Batched paged decode layer (slimkv_amd.paged_step) against the oracle.

The reference runs a decode batch one request at a time: restore_memory
(slimkv/vllm_plugin/paged_model.py:7-52), fa2_decode.decode
(slimkv/llama3/fa2_decode.py:77-166), flush_memory (paged_model.py:55-84).
Here a batch of requests at different points of their windows (no history yet,
window boundary, insertion steps, a step that completes its window, several
pages of beacons) runs through paged_decode_layer, and

* each request's output is checked against the oracle's restatement of that
  sequence -- the memory read out of the pages with the oracle's page index
  math, RoPE at the memory's slot positions, the latent layer with the
  reference's bf16 roundings -- within the bf16 bar;
* the pages afterwards are checked bit for bit against flush_memory's writes:
  the new token's K/V (before RoPE) at raw position P unless the step
  completes the window, the new beacon's latents at beacon P // ratio, the sink
  replaced by the new token while the request has no history
  (slimkv/llama3/memory.py:257-262), nothing else touched;
* steps chained over a window boundary read back what earlier steps wrote;
* a block-table entry outside the pool at the raw write raises IndexError.
"""
import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import paged as op
from oracle import rope as orope
from slimkv_amd.workloads import block_diagonal, orthonormal_columns, rope_tables
from tests.helpers import assert_close, to_np

pytestmark = pytest.mark.gpu

H, HKV, D, RANK = 8, 2, 128, 32
HIDDEN = H * D
WINDOW, RATIO, BLOCK, SINK = 32, 4, 16, 1
DEFAULT = (WINDOW, RATIO, SINK)


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


def _attention(device, bias=False, seed=0):
    gen = torch.Generator(device=device).manual_seed(seed)
    R = HKV * RANK
    uk = block_diagonal([orthonormal_columns(D, RANK, torch.Generator().manual_seed(seed + i)) for i in range(HKV)])
    uv = block_diagonal([orthonormal_columns(D, RANK, torch.Generator().manual_seed(seed + 9 + i))
                         for i in range(HKV)])
    att = SimpleNamespace(
        config=SimpleNamespace(beacon_param=['q', 'k', 'v'], beacon_skip_rope_for_beacon_k=True),
        num_heads=H, num_key_value_heads=HKV, head_dim=D, hidden_size=HIDDEN, training=False,
        q_proj=_linear(HIDDEN, H * D, gen, device), k_proj=_linear(HIDDEN, HKV * D, gen, device),
        v_proj=_linear(HIDDEN, HKV * D, gen, device), beacon_q_proj=_linear(HIDDEN, H * D, gen, device),
        beacon_k_down_proj=_linear(HIDDEN, R, gen, device), beacon_v_down_proj=_linear(HIDDEN, R, gen, device),
        beacon_k_up_proj=_linear(R, HKV * D, gen, device, bias, uk.to(device, torch.bfloat16)),
        beacon_v_up_proj=_linear(R, HKV * D, gen, device, bias, uv.to(device, torch.bfloat16)),
        rotary_emb=RotaryEmbedding(2048, device))
    att._use_shared_kv_down_proj = lambda: False
    att.o_proj_with_beacon = lambda output, size, indices: output
    return att, gen


def _layout(ratio=RATIO):
    from slimkv_amd.paged_cache import BeaconPageLayout
    return BeaconPageLayout(BLOCK, ratio, HKV * RANK, HKV * RANK, HKV * D)


def _pool(device, processed, gen, steps=1, seed=0, cfg=DEFAULT):
    """Random pages and permuted block tables with room for `steps` more
    tokens; table entries past a request's pages hold ids far outside the pool."""
    RATIO = cfg[1]
    layout = _layout(RATIO)
    cpu = torch.Generator().manual_seed(seed)
    last = [p + steps for p in processed]
    raw_need = [(n + BLOCK - 1) // BLOCK for n in last]
    beacon_need = [max(1, (n // RATIO + layout.slots - 1) // layout.slots) for n in last]
    tables = []
    pools = []
    for need in (raw_need, beacon_need):
        pool = sum(need) + 5
        perm = torch.randperm(pool, generator=cpu)
        width = max(need) + 2
        t = torch.randint(1 << 40, 1 << 41, (len(processed), width), generator=cpu)
        off = 0
        for b, n in enumerate(need):
            t[b, :n] = perm[off:off + n]
            off += n
        tables.append(t.to(device))
        pools.append(pool)
    raw = torch.randn(pools[0], BLOCK, 2, HKV, D, generator=gen, device=device).to(torch.bfloat16)
    beacon = torch.randn(pools[1], layout.page_elements, generator=gen, device=device).to(torch.bfloat16)
    return layout, raw, beacon, tables[0], tables[1]


def _projections(att, hidden, size):
    """The step's q / new K / new V and new beacon latents by the module's own
    projections (fa2_decode.py:88-100)."""
    with torch.no_grad():
        q = att.q_proj(hidden)
        if size:
            q = torch.cat([q[:, :1], att.beacon_q_proj(hidden[:, 1:])], dim=1)
        new_k = att.k_proj(hidden[:, :1]).reshape(-1, HKV, D)
        new_v = att.v_proj(hidden[:, :1]).reshape(-1, HKV, D)
        kl = att.beacon_k_down_proj(hidden[:, 1:]) if size else None
        vl = att.beacon_v_down_proj(hidden[:, 1:]) if size else None
    return q, new_k, new_v, kl, vl


def _oracle_request(att, layout, raw_np, beacon_np, raw_table, beacon_table, P, q, new_k, new_v, kl, vl, size,
                    cfg=DEFAULT):
    """Output [L, HIDDEN] of request's decode step: the memory read out of
    the pages before the step (restore_memory), the oracle's RoPE and latent
    layer (fa2_decode.decode)."""
    WINDOW, RATIO, SINK = cfg
    rc, hist, beacons = op.restore_counts(P, WINDOW, RATIO)
    root = beacon_np[int(beacon_table[0])]
    sink_k = root[:layout.raw_width].reshape(HKV, 1, D)[:, :SINK]
    sink_v = root[layout.raw_width:layout.sink_elements].reshape(HKV, 1, D)[:, :SINK]
    blk, off = op.raw_indices(BLOCK, raw_table, P - rc, rc)
    raw_k = raw_np[blk, off, 0].transpose(1, 0, 2)                     # [HKV, rc, D]
    raw_v = raw_np[blk, off, 1].transpose(1, 0, 2)
    page, first = op.beacon_indices(layout, beacon_table, 0, beacons)
    cols_k = first[:, None] + np.arange(layout.key_rank)
    cols_v = first[:, None] + layout.key_rank + np.arange(layout.value_rank)
    lat_k = beacon_np[page[:, None], cols_k]
    lat_v = beacon_np[page[:, None], cols_v]
    if size:
        lat_k = np.concatenate([lat_k, to_np(kl).reshape(1, -1)])
        lat_v = np.concatenate([lat_v, to_np(vl).reshape(1, -1)])
    L = 1 + size
    keys = np.concatenate([sink_k, raw_k, to_np(new_k).reshape(HKV, 1, D)], axis=1)
    values = np.concatenate([sink_v, raw_v, to_np(new_v).reshape(HKV, 1, D)], axis=1)
    raw_idx = np.nonzero(op.window_roles(rc, RATIO) == 0)[0]
    mem = SINK + hist + rc + rc // RATIO
    c = to_np(att.rotary_emb.cos_cached).astype(np.float32)
    s = to_np(att.rotary_emb.sin_cached).astype(np.float32)
    qn = to_np(q).reshape(1, L, H, D).transpose(0, 2, 1, 3).astype(np.float32)
    q_rot, k_rot = orope.rope_decode(qn, keys[None].astype(np.float32), c, s, (mem + np.arange(L))[None], raw_idx,
                                     SINK, hist)
    uk, uv = att.beacon_k_up_proj, att.beacon_v_up_proj
    out, _ = oa.latent_layer(q_rot, k_rot, values[None], lat_k[None, None], lat_v[None, None], to_np(uk.weight),
                             to_np(uv.weight), 1 / math.sqrt(D), HKV,
                             None if uk.bias is None else to_np(uk.bias),
                             None if uv.bias is None else to_np(uv.bias), lat_causal=bool(size))
    return out.transpose(0, 2, 1, 3).reshape(L, HIDDEN)


def _expected_pages(layout, raw, beacon, raw_tables, beacon_tables, processed, proj, cfg=DEFAULT):
    """flush_memory's writes of one decode step on copies of the pages."""
    WINDOW, RATIO, SINK = cfg
    raw, beacon = raw.clone(), beacon.clone()
    for b, P in enumerate(processed):
        new_k, new_v, kl, vl = proj[b]
        if (P + 1) % WINDOW:
            blk = int(raw_tables[b, P // BLOCK])
            raw[blk, P % BLOCK, 0] = new_k
            raw[blk, P % BLOCK, 1] = new_v
        if kl is not None:
            n = P // RATIO
            page = int(beacon_tables[b, n // layout.slots])
            first = layout.sink_elements + (n % layout.slots) * layout.width
            beacon[page, first:first + layout.key_rank] = kl.reshape(-1)
            beacon[page, first + layout.key_rank:first + layout.width] = vl.reshape(-1)
        if SINK and P < WINDOW:                                # no history yet: the new token is the sink
            root = int(beacon_tables[b, 0])
            beacon[root, :layout.sink_elements] = torch.cat([new_k.reshape(-1), new_v.reshape(-1)])
    return raw, beacon


def _step(att, gen, device, layout, raw, beacon, raw_tables, beacon_tables, processed, check_pages=True,
          cfg=DEFAULT):
    """One decode step of every request through paged_decode_layer; outputs
    against the oracle, pages against flush_memory's writes."""
    from slimkv_amd.paged_step import paged_decode_layer, plan_paged_step, step_size
    WINDOW, RATIO, SINK = cfg
    sizes = [step_size(P, WINDOW, RATIO) for P in processed]
    hidden = [(torch.randn(1 + s, HIDDEN, generator=gen, device=device) * 0.5).to(torch.bfloat16) for s in sizes]
    proj = []
    for h, s in zip(hidden, sizes):
        q, nk, nv, kl, vl = _projections(att, h[None], s)
        proj.append((q, nk, nv, kl, vl))
    raw_np = to_np(raw).astype(np.float32)
    beacon_np = to_np(beacon).astype(np.float32)
    expected = [_oracle_request(att, layout, raw_np, beacon_np, to_np(raw_tables[b]), to_np(beacon_tables[b]), P,
                                *proj[b], sizes[b], cfg=cfg) for b, P in enumerate(processed)]
    want_raw, want_beacon = _expected_pages(layout, raw, beacon, raw_tables, beacon_tables, processed,
                                            [p[1:] for p in proj], cfg=cfg)
    groups = plan_paged_step(processed, WINDOW, RATIO, SINK, device)
    assert sorted(i for g in groups for i in g.index) == list(range(len(processed)))
    for g in groups:
        idx = g.tensors['index']
        with torch.no_grad():
            out = paged_decode_layer(att, torch.stack([hidden[i] for i in g.index]), g, raw, beacon,
                                     raw_tables[idx], beacon_tables[idx], BLOCK)
        torch.cuda.synchronize()
        for row, i in enumerate(g.index):
            print(f'request {i}: processed {processed[i]}, size {g.size}', flush=True)
            assert_close(to_np(out[row]), expected[i], what=f'request {i} (P={processed[i]}, size {g.size})')
    if check_pages:
        assert torch.equal(raw.view(torch.int16), want_raw.view(torch.int16)), 'raw pages differ from the flush'
        assert torch.equal(beacon.view(torch.int16), want_beacon.view(torch.int16)), \
            'beacon pages differ from the flush'


@pytest.mark.parametrize('bias', [False, True])
def test_paged_step_mixed_batch(device, bias):
    processed = [1, 3, 7, 31, 32, 45, 63, 64, 100, 131, 200, 255]
    att, gen = _attention(device, bias, seed=5 + bias)
    layout, raw, beacon, raw_tables, beacon_tables = _pool(device, processed, gen, seed=2)
    _step(att, gen, device, layout, raw, beacon, raw_tables, beacon_tables, processed)


def test_paged_step_chained(device):
    """Four consecutive steps across window boundaries (P = 29..32 and
    61..64): each step reads what the previous ones flushed."""
    att, gen = _attention(device, False, seed=17)
    processed = [29, 61, 2]
    layout, raw, beacon, raw_tables, beacon_tables = _pool(device, processed, gen, steps=4, seed=3)
    for step in range(4):
        print(f'step {step}: processed {processed}', flush=True)
        _step(att, gen, device, layout, raw, beacon, raw_tables, beacon_tables, processed)
        processed = [p + 1 for p in processed]


def test_paged_step_bad_write_block(device):
    """A raw block-table entry outside the pool at the new token's position:
    the write moves nothing and the step raises IndexError."""
    from slimkv_amd.paged_step import paged_decode_layer, plan_paged_step
    att, gen = _attention(device, False, seed=23)
    processed = [32, 40]
    layout, raw, beacon, raw_tables, beacon_tables = _pool(device, processed, gen, seed=4)
    raw_tables[0, 32 // BLOCK] = raw.shape[0] + 3
    before = raw.clone()
    (g,) = plan_paged_step(processed, WINDOW, RATIO, SINK, device)
    hidden = (torch.randn(2, 1, HIDDEN, generator=gen, device=device) * 0.5).to(torch.bfloat16)
    with torch.no_grad(), pytest.raises(IndexError):
        paged_decode_layer(att, hidden, g, raw, beacon, raw_tables, beacon_tables, BLOCK)
    torch.cuda.synchronize()
    blk = int(raw_tables[1, 40 // BLOCK])
    changed = (raw.view(torch.int16) != before.view(torch.int16)).flatten(1).any(1).nonzero().flatten().tolist()
    assert changed == [blk]


def test_paged_step_rows_bounds(device):
    """A dense raw set too short for a request's sink + window rows + new
    token raises IndexError after the launch; per-request tensors shorter than
    the batch are refused before it."""
    from slimkv_amd import kernels
    from slimkv_amd.paged_step import plan_paged_step
    att, gen = _attention(device, False, seed=29)
    processed = [9, 20]
    layout, raw, beacon, raw_tables, beacon_tables = _pool(device, processed, gen, seed=7)
    (g,) = plan_paged_step(processed, WINDOW, RATIO, SINK, device)
    t = g.tensors
    new_k = torch.randn(2, HKV, D, generator=gen, device=device).to(torch.bfloat16)
    new_v = torch.randn_like(new_k)
    cos, sin = att.rotary_emb.cos_cached, att.rotary_emb.sin_cached
    args = (raw, raw_tables, beacon, beacon_tables, new_k, new_v, t['window_start'], t['raw_count'],
            t['raw_positions'])
    ok_k, ok_v = kernels.paged_step_rows(*args, cos, sin, g.max_raw, SINK)
    torch.cuda.synchronize()
    with pytest.raises(IndexError):             # request 1 needs sink + 20 + 1 = 22 rows
        kernels.paged_step_rows(*args, cos, sin, g.max_raw - 1, SINK)
    torch.cuda.synchronize()
    with pytest.raises(ValueError):
        kernels.paged_step_rows(raw, raw_tables, beacon, beacon_tables, new_k, new_v, t['window_start'][:1],
                                t['raw_count'], t['raw_positions'], cos, sin, g.max_raw, SINK)
    assert ok_k.shape == (2, g.max_raw, HKV, D) and ok_v.shape == ok_k.shape


@pytest.mark.parametrize('cfg', [(32, 8, 0), (64, 16, 1)])
def test_paged_step_other_configurations(device, cfg):
    """No sink (every raw row of the memory is a window row) and a longer
    window at a higher ratio: the same checks over one step of a mixed batch."""
    window, ratio, sink = cfg
    processed = [1, 7, 15, 16, 31, 33, 47, 63, 64, 95, 150, 255]
    att, gen = _attention(device, False, seed=31 + window)
    layout, raw, beacon, raw_tables, beacon_tables = _pool(device, processed, gen, seed=6, cfg=cfg)
    _step(att, gen, device, layout, raw, beacon, raw_tables, beacon_tables, processed, cfg=cfg)
