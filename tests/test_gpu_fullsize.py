"""Parity at the full benchmark sizes, on the inputs the benchmarks build.

C1  latent beacon decode, Llama-3.1-8B layer, B16 x 8192 beacons + 133 raw
    rows, one seeded layer per latent rank 16 / 32 / 48 built exactly as
    bench.py builds its sweep (bench.make_layer / bench.run_layer), against
    the oracle's restatement of the reference decode (fa2_decode.py:143-164).
C2  reconstruction decode, Qwen2.5-14B layer (B8, 40/8 heads, 8192 beacons,
    beacon K-RoPE) as bench_workloads.recon_layer builds it; sampled batch
    rows against the float64 attention over the rebuilt cache and the
    reference's eager formulation (modeling_llama.py:1405-1483).
C3  the window prefill chain, B4, 8 windows of 1024 raw + 256 beacons, 32/8
    heads: every window through prefill_forward (the join-prefill branch of
    LlamaFlashAttention2.forward, modeling_llama.py:1632-1750) with the
    previous windows' latents as history; windows 0, 3 and 7 against the
    oracle on sampled heads, every window's latents within one bf16 ulp.
C4  the paged workload's own seeded draw (64 sequences, 400K-page pool):
    the gathered beacon rows bit for bit at the oracle's indices
    (paged_cache.py:60-67), the paged decode bit-identical to gather + decode,
    and sampled sequences against the oracle.
    The benchmark's own call (raw rows through their raw pages too, the
    automatic compact schedule) on every sequence against the oracle.
Qwen2.5-14B latent beacon decode (bench.py --workload qwen): B16 x 8192
    beacons, 40/8 heads, up-projection biases, one layer per rank.
Bar: max abs 2e-2, mean abs 2e-3 and relative l2 1e-2 on bf16 outputs; LSE
within 2e-3.  C1 also runs with queries twice the benchmark's (a peaked
softmax).
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import paged as opaged
from oracle import rope as orope
from oracle.bf16 import round_bf16
from tests.helpers import assert_close, assert_lse_close, bits, to_np

pytestmark = pytest.mark.gpu


def _rot_at(x_bhsd, cos, sin, pos):
    """Oracle RoPE of bf16 rows [B, H, L, D] at one position (float32 arrays)."""
    c = to_np(cos[pos]).astype(np.float32)[None, None, None]
    s = to_np(sin[pos]).astype(np.float32)[None, None, None]
    return orope.rotate_bf16(to_np(x_bhsd).astype(np.float32), c, s).astype(np.float64)


# ----------------------------------------------------------------------------- C1

@pytest.mark.parametrize('rank,q_scale', [(16, 1), (32, 1), (48, 1), (32, 2)])
def test_c1_latent_decode_full_size(device, rank, q_scale):
    """q_scale 2: queries twice the benchmark's (an exact bf16 scaling), a
    peaked softmax whose outputs are dominated by few rows."""
    import bench
    from slimkv_amd import kernels
    from slimkv_amd.workloads import rope_tables
    print(f'C1: B{bench.B} beacons {bench.BEACONS} rank {rank} q x{q_scale}', flush=True)
    cos, sin = rope_tables(bench.CONTEXT + 1, bench.D, 500000.0, device)
    layer = bench.make_layer(torch, device, rank, 9000 + rank, cos, sin)
    layer['q'].mul_(q_scale)
    pos = torch.full((bench.B, 1), bench.CONTEXT, dtype=torch.int64, device=device)
    rows = kernels.query_rope_rows(cos, sin, pos)
    scale = 1.0 / math.sqrt(bench.D)
    bench.run_layer(kernels, layer, rows, scale, None)
    torch.cuda.synchronize()
    q_rot = _rot_at(layer['q'].transpose(1, 2), cos, sin, bench.CONTEXT)
    want, want_lse = oa.latent_layer(q_rot, to_np(layer['raw_k'].transpose(1, 2)),
                                     to_np(layer['raw_v'].transpose(1, 2)), to_np(layer['lat_k'])[:, None],
                                     to_np(layer['lat_v'])[:, None], to_np(layer['up_k']), to_np(layer['up_v']),
                                     scale, bench.HKV)
    assert_close(to_np(layer['out'].transpose(1, 2)), want, what=f'C1 rank {rank} q x{q_scale}')
    assert_lse_close(to_np(layer['lse']), want_lse, what=f'C1 rank {rank} q x{q_scale}')


@pytest.mark.parametrize('rank', [16, 32, 48])
def test_qwen_latent_decode_full_size(device, rank):
    """The sweep's Qwen2.5-14B layer (bench.py --workload qwen): B16 x 8192
    beacons, 40/8 heads, biases on both up-projections."""
    import bench
    from slimkv_amd import kernels
    from slimkv_amd.workloads import rope_tables
    print(f'Qwen2.5-14B: B{bench.B} beacons {bench.BEACONS} rank {rank}', flush=True)
    cos, sin = rope_tables(bench.CONTEXT + 1, bench.D, 500000.0, device)
    layer = bench.make_layer(torch, device, rank, 9100 + rank, cos, sin, hq=40, bias=True)
    pos = torch.full((bench.B, 1), bench.CONTEXT, dtype=torch.int64, device=device)
    rows = kernels.query_rope_rows(cos, sin, pos)
    scale = 1.0 / math.sqrt(bench.D)
    bench.run_layer(kernels, layer, rows, scale, None)
    torch.cuda.synchronize()
    q_rot = _rot_at(layer['q'].transpose(1, 2), cos, sin, bench.CONTEXT)
    want, want_lse = oa.latent_layer(q_rot, to_np(layer['raw_k'].transpose(1, 2)),
                                     to_np(layer['raw_v'].transpose(1, 2)), to_np(layer['lat_k'])[:, None],
                                     to_np(layer['lat_v'])[:, None], to_np(layer['up_k']), to_np(layer['up_v']),
                                     scale, bench.HKV, to_np(layer['bk']), to_np(layer['bv']))
    assert_close(to_np(layer['out'].transpose(1, 2)), want, what=f'Qwen rank {rank}')
    assert_lse_close(to_np(layer['lse']), want_lse, what=f'Qwen rank {rank}')


# ----------------------------------------------------------------------------- C2

def test_c2_recon_decode_full_size_sampled_rows(device):
    from bench_workloads import RECON_SHAPE, recon_layer, recon_positions
    from slimkv_amd import kernels
    from slimkv_amd.workloads import rope_tables
    c = RECON_SHAPE
    HKV, D, CTX = c['HKV'], c['D'], c['CTX']
    print(f"C2: B{c['B']} beacons {c['NB']} {c['HQ']}/{HKV} heads", flush=True)
    cos, sin = rope_tables(CTX + 1, D, 500000.0, device)
    layer = recon_layer(torch, device, 4242)
    qpos, bpos = recon_positions(torch, device)
    scale = D ** -0.5
    out, lse = kernels.recon_decode(layer['q'], layer['raw_k'], layer['raw_v'], layer['lat_k'], layer['lat_v'],
                                    layer['up_k'], layer['up_v'], scale, beacon_positions=bpos, block_diagonal=True,
                                    q_positions=qpos, cos=cos, sin=sin)
    torch.cuda.synchronize()
    cn, sn = to_np(cos).astype(np.float32), to_np(sin).astype(np.float32)
    bp = bpos[0].cpu().numpy()
    for b in (0, 5):
        sl = slice(b, b + 1)
        q_rot = _rot_at(layer['q'][sl].transpose(1, 2), cos, sin, CTX)             # [1, H, 1, D]
        # the reference's keys (bf16 up-projection, bf16 RoPE steps) and the
        # fused route's fp32 rotation (float64 model, one rounding)
        rk = oa.reconstruct(to_np(layer['lat_k'][sl])[:, None], to_np(layer['up_k']), None, HKV, D)
        rk = orope.rotate_bf16(rk[0].astype(np.float32), cn[bp][None], sn[bp][None]).astype(np.float64)[None]
        xk = oa.reconstruct(to_np(layer['lat_k'][sl])[:, None], to_np(layer['up_k']), None, HKV, D,
                            bf16_boundaries=False)[0]
        c64, s64 = round_bf16(cn[bp][None]).astype(np.float64), round_bf16(sn[bp][None]).astype(np.float64)
        fk = round_bf16(xk * c64 + orope.rotate_half(xk) * s64).astype(np.float64)[None]
        rv = oa.reconstruct(to_np(layer['lat_v'][sl])[:, None], to_np(layer['up_v']), None, HKV, D)
        got = to_np(out[sl])                                                          # [1, 1, H, D]
        for name, keys in (('reference keys', rk), ('fp32-rotated keys', fk)):
            k = np.concatenate([keys, to_np(layer['raw_k'][sl].transpose(1, 2))], axis=2)
            v = np.concatenate([rv, to_np(layer['raw_v'][sl].transpose(1, 2))], axis=2)
            exact, exact_lse = oa.eager_forward(q_rot.transpose(0, 2, 1, 3), k.transpose(0, 2, 1, 3),
                                                v.transpose(0, 2, 1, 3), scale)
            eager, _ = oa.eager_recon_layer(q_rot, k, v, scale)
            assert_close(got, exact, what=f'C2 row {b} vs float64, {name}')
            assert_close(got, eager.transpose(0, 2, 1, 3), what=f'C2 row {b} vs eager bf16, {name}')
            assert_lse_close(to_np(lse[sl]), exact_lse, what=f'C2 row {b}, {name}')


# ----------------------------------------------------------------------------- C3

class RotaryEmbedding:          # the type name the prefill RoPE fusion recognises
    def __init__(self, rows, device):
        from slimkv_amd.workloads import rope_tables
        self.cos_cached, self.sin_cached = rope_tables(rows, 128, 500000.0, device)
        self.max_seq_len_cached = rows


def _llama8b_module(device, seed):
    """A Llama-3.1-8B attention layer as prefill_forward uses it: hidden 4096,
    32/8 heads, head_dim 128, beacon K/V latents of rank 32 per KV head
    (down Linear 4096 -> 256, orthonormal per-head up-projections)."""
    from types import SimpleNamespace
    from slimkv_amd.workloads import block_diagonal, orthonormal_columns
    H, Hk, D, hidden, r = 32, 8, 128, 4096, 32
    gen = torch.Generator(device=device).manual_seed(seed)

    def linear(i, o, weight=None):
        lin = torch.nn.Linear(i, o, bias=False, device=device, dtype=torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_(weight if weight is not None else torch.randn(o, i, generator=gen, device=device) / i ** 0.5)
        return lin
    up = [block_diagonal([orthonormal_columns(D, r, torch.Generator().manual_seed(seed + 10 * j + i))
                          for i in range(Hk)]).to(device, torch.bfloat16) for j in range(2)]
    config = SimpleNamespace(beacon_param=['q', 'k', 'v'], beacon_decode_backend='latent', beacon_sink_size=4,
                             _attn_implementation='flash_attention_2')
    att = SimpleNamespace(
        config=config, num_heads=H, num_key_value_heads=Hk, head_dim=D, hidden_size=hidden,
        q_proj=linear(hidden, H * D), k_proj=linear(hidden, Hk * D), v_proj=linear(hidden, Hk * D),
        beacon_q_proj=linear(hidden, H * D),
        beacon_k_down_proj=linear(hidden, Hk * r), beacon_v_down_proj=linear(hidden, Hk * r),
        beacon_k_up_proj=linear(Hk * r, Hk * D, up[0]), beacon_v_up_proj=linear(Hk * r, Hk * D, up[1]),
        rotary_emb=RotaryEmbedding(8192, device))
    att._use_shared_kv_down_proj = lambda: False
    att.o_proj_with_beacon = lambda output, size, indices: output
    return att, gen


def test_c3_prefill_window_chain(device):
    """The chain through prefill_forward with the append-only PrefillHistory
    (each window rebuilds only its new beacons) against the oracle; every
    window's output and latents also bit-identical to the same window run
    through ReconstructionCache.materialize (the whole history rebuilt)."""
    from slimkv_amd.memory import ReconstructionCache
    from slimkv_amd.prefill import PrefillHistory, prefill_forward
    from slimkv_amd.prefill_ops import PrefillMetadata
    B, L, H, Hk, D, R, S, NB, WINDOWS = 4, 1280, 32, 8, 128, 256, 4, 256, 8
    heads = (5, 30)                                           # sampled query heads (KV heads 1 and 7)
    check = (0, 3, 7)
    att, gen = _llama8b_module(device, 77)
    store = PrefillHistory(B, Hk, D, S + NB * WINDOWS + L, device)
    roles = torch.zeros(L, dtype=torch.long, device=device)
    roles[4::5] = 1                                           # a beacon after every 4 raw tokens
    brows = (roles != 0).nonzero().flatten().cpu().numpy()
    sink = hist_k = hist_v = None
    for w in range(WINDOWS):
        print(f'C3: window {w}', flush=True)
        hidden = (0.5 * torch.randn(B, L, 4096, generator=gen, device=device)).to(torch.bfloat16)
        n_hist = 0 if hist_k is None else hist_k.shape[2]
        N = (S if w else 0) + n_hist + L
        pk = ReconstructionCache(None if sink is None else sink[0], hist_k, None, None, None, Hk, D, 'k')
        pv = ReconstructionCache(None if sink is None else sink[1], hist_v, None, None, None, Hk, D, 'v')
        positions = torch.arange(N, device=device)[None].expand(B, -1)
        att._prefill_metadata = PrefillMetadata((roles == 0).nonzero().flatten(), (roles != 0).nonzero().flatten(),
                                                roles, positions, False)
        with torch.no_grad():
            out, _, update = prefill_forward(att, hidden, positions, (pk, pv, NB, roles), history=store)
            full, _, full_update = prefill_forward(att, hidden, positions, (pk, pv, NB, roles))
            torch.cuda.synchronize()
            assert torch.equal(out, full), f'window {w}: append-only history output differs from the full rebuild'
            assert torch.equal(update.key_latents, full_update.key_latents)
            assert torch.equal(update.value_latents, full_update.value_latents)
            assert (store.sink, store.history) == (S, NB * (w + 1))
            if w in check:
                q_mod = torch.where((roles == 0)[:, None], att.q_proj(hidden), att.beacon_q_proj(hidden))
                kf, vf = att.k_proj(hidden), att.v_proj(hidden)
        h = to_np(hidden)
        for kind, got in (('k', update.key_latents), ('v', update.value_latents)):
            down = to_np(getattr(att, f'beacon_{kind}_down_proj').weight)
            exact = oa.down_project(h, down, brows, bf16_boundaries=False)
            mag = np.maximum(np.abs(exact), 1e-30)
            ulp = 2.0 ** (np.floor(np.log2(mag)) - 7)
            terms = oa.down_project(np.abs(h), np.abs(down), brows, bf16_boundaries=False) * 2.0 ** -20
            assert (np.abs(to_np(got[:, 0]) - exact) < ulp * 1.0001 + terms).all(), f'window {w} {kind} latents'
        if w in check:
            cur = {}
            for kind, full in (('k', kf), ('v', vf)):
                up = getattr(att, f'beacon_{kind}_up_proj').weight
                lat = oa.down_project(h, to_np(getattr(att, f'beacon_{kind}_down_proj').weight), brows)
                rec = oa.reconstruct(lat[:, None], to_np(up), None, Hk, D)
                cf = to_np(full).reshape(B, L, Hk, D).transpose(0, 2, 1, 3).copy()
                cf[:, :, brows] = rec
                cur[kind] = cf
            K = oa.materialize(None if sink is None else to_np(sink[0]), None if hist_k is None else to_np(hist_k),
                               None, None, None, to_np(att.beacon_k_up_proj.weight), None, Hk, D, cur['k'])
            V = oa.materialize(None if sink is None else to_np(sink[1]), None if hist_v is None else to_np(hist_v),
                               None, None, None, to_np(att.beacon_v_up_proj.weight), None, Hk, D, cur['v'])
            kv = [hh // (H // Hk) for hh in heads]
            c = to_np(att.rotary_emb.cos_cached).astype(np.float32)
            s = to_np(att.rotary_emb.sin_cached).astype(np.float32)
            qn = to_np(q_mod).reshape(B, L, H, D).transpose(0, 2, 1, 3)[:, list(heads)].astype(np.float32)
            q_rot, k_rot = orope.prefill_rope(qn, K[:, kv].astype(np.float32), c, s, positions.cpu().numpy(),
                                              roles.cpu().numpy(), S if w else 0)
            want, _ = oa.eager_forward(q_rot.transpose(0, 2, 1, 3), k_rot.transpose(0, 2, 1, 3),
                                       V[:, kv].transpose(0, 2, 1, 3), D ** -0.5, causal=True)
            got = to_np(out).reshape(B, L, H, D)[:, :, list(heads)]
            assert_close(got, want, what=f'C3 window {w}')
        # the cache update as the memory keeps it: sinks from window 0, latents appended
        if w == 0:
            sink = (update[0][:, :, :S].contiguous(), update[1][:, :, :S].contiguous())
        hist_k = update.key_latents if hist_k is None else torch.cat([hist_k, update.key_latents], dim=2)
        hist_v = update.value_latents if hist_v is None else torch.cat([hist_v, update.value_latents], dim=2)
    assert hist_k.shape == (B, 1, NB * WINDOWS, R)


# ----------------------------------------------------------------------------- C4

def test_c4_paged_full_size_indices_and_parity(device):
    from bench_workloads import PAGED_SHAPE, paged_case
    from slimkv_amd import kernels
    from slimkv_amd.paged_cache import BeaconPages, RawPages
    c = PAGED_SHAPE
    HKV, D, HQ = c['HKV'], c['D'], c['HQ']
    pc = paged_case(torch, device, 0)
    nb, raw_count, layout = pc['nb'], pc['raw_count'], pc['layout']
    print(f"C4: {len(nb)} sequences, {sum(nb)} beacons, pool {pc['pool'].shape[0]} pages", flush=True)
    olayout = opaged.Layout(layout.raw_block_size, layout.token_ratio, layout.key_rank, layout.value_rank,
                            layout.raw_width)
    # 1. every beacon row of every sequence, gathered by the page kernel, at
    #    the oracle's (page, column) indices, bit for bit
    lat_k, lat_v = BeaconPages(pc['pool'], layout).read_batch(pc['tables'], pc['lat_len'])
    flat = pc['pool'].view(-1)
    stride = pc['pool'].stride(0)
    width = torch.arange(layout.width, device=device)
    tables = pc['tables_cpu'].numpy()
    for b, n in enumerate(nb):
        page, first = opaged.beacon_indices(olayout, tables[b], 0, n)
        idx = torch.from_numpy(page * stride + first).to(device)[:, None] + width[None]
        rows = flat[idx]
        assert torch.equal(lat_k[b, :n], rows[:, :layout.key_rank]), f'sequence {b} K rows'
        assert torch.equal(lat_v[b, :n], rows[:, layout.key_rank:]), f'sequence {b} V rows'
        assert not lat_k[b, n:].any()
    # raw rows (sinks + tail + current token) at the oracle's raw indices
    max_raw = max(raw_count)
    raw_k = torch.zeros(len(nb), HKV, max_raw, D, dtype=torch.bfloat16, device=device)
    raw_v = torch.zeros_like(raw_k)
    kernels.raw_pages(pc['raw_pool'], pc['raw_tables'], raw_k, raw_v, start=0, count=max_raw, to_pages=False,
                      lengths=pc['raw_len'])
    rt = pc['raw_tables'].cpu().numpy()
    for b, n in enumerate(raw_count):
        blk, off = opaged.raw_indices(16, rt[b], 0, n)
        want = pc['raw_pool'][torch.from_numpy(blk).to(device), torch.from_numpy(off).to(device)]   # [n, 2, Hkv, D]
        assert torch.equal(raw_k[b, :, :n], want[:, 0].transpose(0, 1))
        assert torch.equal(raw_v[b, :, :n], want[:, 1].transpose(0, 1))
    # 2. the paged decode reads the same rows: bit-identical to gather + decode
    scale = D ** -0.5
    common = dict(block_diagonal=True, raw_lengths=pc['raw_len'], raw_splits=4)   # one split plan on both sides
    dense = kernels.latent_decode(pc['q'], raw_k.transpose(1, 2), raw_v.transpose(1, 2), lat_k, lat_v, pc['up_k'],
                                  pc['up_v'], scale, lat_lengths=pc['lat_len'], lat_splits=48, **common)
    paged = kernels.paged_latent_decode(pc['q'], raw_k.transpose(1, 2), raw_v.transpose(1, 2), pc['pool'],
                                        pc['tables'], pc['lat_len'], max(nb), layout, pc['up_k'], pc['up_v'], scale,
                                        lat_splits=48, **common)
    torch.cuda.synchronize()
    assert torch.equal(paged[0], dense[0]) and torch.equal(paged[1], dense[1])
    # 3. the benchmark's call (automatic compact schedule) on sampled sequences
    #    against the oracle
    out, lse = kernels.paged_latent_decode(pc['q'], raw_k.transpose(1, 2), raw_v.transpose(1, 2), pc['pool'],
                                           pc['tables'], pc['lat_len'], max(nb), layout, pc['up_k'], pc['up_v'],
                                           scale, rows_total=sum(nb), **common)
    torch.cuda.synchronize()
    order = np.argsort(nb)
    for b in (int(order[0]), int(order[len(nb) // 2]), int(order[-1])):
        n, m = nb[b], raw_count[b]
        want, want_lse = oa.latent_layer(to_np(pc['q'][b:b + 1].transpose(1, 2)), to_np(raw_k[b:b + 1, :, :m]),
                                         to_np(raw_v[b:b + 1, :, :m]), to_np(lat_k[b:b + 1, :n])[:, None],
                                         to_np(lat_v[b:b + 1, :n])[:, None], to_np(pc['up_k']), to_np(pc['up_v']),
                                         scale, HKV)
        assert_close(to_np(out[b:b + 1].transpose(1, 2)), want, what=f'C4 sequence {b} ({n} beacons)')
        assert_lse_close(to_np(lse[b:b + 1]), want_lse, what=f'C4 sequence {b}')
    # 4. the timed configuration itself (bench_workloads.paged): raw rows read
    #    through the raw pages and their block table as well, the automatic
    #    compact schedule; every sequence against the oracle
    status = torch.zeros(1, dtype=torch.int32, device=device)
    out, lse = kernels.paged_latent_decode(pc['q'], None, None, pc['pool'], pc['tables'], pc['lat_len'], max(nb),
                                           layout, pc['up_k'], pc['up_v'], scale, rows_total=sum(nb),
                                           block_diagonal=True, raw_lengths=pc['raw_len'], status=status,
                                           raw_pages=pc['raw_pool'], raw_tables=pc['raw_tables'], raw_keys=max_raw)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    worst = 0.0
    for b, (n, m) in enumerate(zip(nb, raw_count)):
        want, want_lse = oa.latent_layer(to_np(pc['q'][b:b + 1].transpose(1, 2)), to_np(raw_k[b:b + 1, :, :m]),
                                         to_np(raw_v[b:b + 1, :, :m]), to_np(lat_k[b:b + 1, :n])[:, None],
                                         to_np(lat_v[b:b + 1, :n])[:, None], to_np(pc['up_k']), to_np(pc['up_v']),
                                         scale, HKV)
        got = to_np(out[b:b + 1].transpose(1, 2))
        worst = max(worst, float(np.abs(got - want).max()))
        assert_close(got, want, what=f'C4 timed call, sequence {b} ({n} beacons, {m} raw rows)')
        assert_lse_close(to_np(lse[b:b + 1]), want_lse, what=f'C4 timed call, sequence {b}')
    print(f'C4 timed call: {len(nb)} sequences, worst max abs err {worst:.3e}', flush=True)
