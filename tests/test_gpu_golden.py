"""The HIP path on the golden fixtures' inputs (tests/golden/*.npz) against the
stored oracle results: RoPE'd queries/keys and page gathers bit-exact (SHA-256
of their bf16 bits), attention outputs to the bf16 bar (max abs 2e-2, mean
2e-3), LSE to 2e-3, beacon latents within one rounding of the exact GEMM.
Inputs are drawn on the host and must carry the fixture's digests first.
"""
import hashlib

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle.bf16 import round_bf16
from tests.golden import make_golden as mg
from tests.helpers import assert_close, assert_lse_close, bits, neighbour_of_exact, to_np

pytestmark = pytest.mark.gpu


def _digest(t):
    return hashlib.sha256(np.ascontiguousarray(bits(t)).tobytes()).hexdigest()


def _case(case, device):
    stored = mg.load(case)
    inp, meta = mg.BUILDERS[case][0]()
    for name, d in mg.input_digests(inp).items():
        assert stored[f'sha_{name}'] == d, f'{case}: input {name} drawn on this host differs from the fixture'
    print(f'{case}: inputs match the fixture', flush=True)

    def dev(name):
        x = torch.from_numpy(np.ascontiguousarray(inp[name])).to(device)
        return x.to(torch.bfloat16) if inp[name].dtype == np.float32 and name not in ('cos', 'sin') else x

    return stored, inp, meta, dev


@pytest.mark.parametrize('block_diagonal', [True, False])
def test_c0_latent_decode(device, block_diagonal):
    """fused_rope bit-exact, then the fused decode (query RoPE in its prologue)
    over the rotated raw rows and the beacon latents; the general-basis route
    reads the same block-diagonal weights as dense matrices."""
    from slimkv_amd import kernels
    st, inp, meta, dev = _case('c0_latent_decode', device)
    q, raw_k, raw_v = dev('q'), dev('raw_k'), dev('raw_v')
    cos, sin, qpos = dev('cos'), dev('sin'), dev('q_positions')
    oq, ok = kernels.rope_decode(q.transpose(1, 2), raw_k.transpose(1, 2), cos, sin, qpos, dev('raw_indices'),
                                 meta['sink'], meta['history'])
    out, lse = kernels.latent_decode(q, ok.transpose(1, 2), raw_v, dev('lat_k'), dev('lat_v'), dev('up_k'),
                                     dev('up_v'), meta['scale'], block_diagonal=block_diagonal, q_positions=qpos,
                                     cos=cos, sin=sin)
    torch.cuda.synchronize()
    assert _digest(oq) == st['sha_q_rot']
    assert _digest(ok) == st['sha_k_rot']
    assert_close(to_np(out.transpose(1, 2)), st['out'], what=f'C0 fixture, block_diagonal={block_diagonal}')
    assert_lse_close(to_np(lse), st['lse'], what='C0 fixture')


@pytest.mark.parametrize('reference_rounding', [True, False])
def test_c2_recon_decode(device, reference_rounding):
    """Beacon keys rebuilt and rotated inside the attention kernel: with the
    reference's bf16 RoPE steps, and with the fp32 rotation."""
    from slimkv_amd import kernels
    st, inp, meta, dev = _case('c2_recon_decode', device)
    out, lse = kernels.recon_decode(dev('q'), dev('raw_k'), dev('raw_v'), dev('lat_k'), dev('lat_v'), dev('up_k'),
                                    dev('up_v'), meta['scale'], beacon_positions=dev('beacon_positions'),
                                    block_diagonal=True, q_positions=dev('q_positions'), cos=dev('cos'),
                                    sin=dev('sin'), reference_rounding=reference_rounding)
    torch.cuda.synchronize()
    name = 'reference' if reference_rounding else 'fp32'
    assert_close(to_np(out), st[f'out_{name}'], what=f'C2 fixture, {name} keys')
    assert_lse_close(to_np(lse), st[f'lse_{name}'], what=f'C2 fixture, {name} keys')


def test_c3_prefill_window(device):
    """fused_prefill_rope bit-exact (beacon keys left unrotated), the causal
    window attention, and the beacon rows' K latents."""
    from slimkv_amd import kernels
    st, inp, meta, dev = _case('c3_prefill_window', device)
    q, k, v = dev('q'), dev('k'), dev('v')
    oq, ok = kernels.prefill_rope(q.transpose(1, 2), k.transpose(1, 2), dev('cos'), dev('sin'), dev('positions'),
                                  dev('roles'), meta['sink'])
    out, lse = kernels.prefill_attention(oq.transpose(1, 2), ok.transpose(1, 2), v, meta['scale'], True)
    lat = kernels.down_project(dev('hidden'), dev('down'), dev('beacon_rows'))
    torch.cuda.synchronize()
    assert _digest(oq) == st['sha_q_rot']
    assert _digest(ok) == st['sha_k_rot']
    assert_close(to_np(out), st['out'], what='C3 fixture')
    assert_lse_close(to_np(lse), st['lse'], what='C3 fixture')
    terms = oa.down_project(np.abs(inp['hidden']).astype(np.float64), np.abs(inp['down']).astype(np.float64),
                            inp['beacon_rows'], bf16_boundaries=False)
    neighbour_of_exact(to_np(lat), st['latents'], round_bf16(st['latents']), terms)


def test_c4_paged_decode(device):
    """Page gathers of the beacon and raw rows bit-exact at the fixture's
    indices (a sequence with no beacons included), then the decode that reads
    the beacon rows straight from the pages."""
    from slimkv_amd import kernels
    from slimkv_amd.paged_cache import BeaconPageLayout, BeaconPages
    st, inp, meta, dev = _case('c4_paged_decode', device)
    layout = BeaconPageLayout(*mg.C4_LAYOUT)
    pool, tables, raw_pool, raw_tables = dev('pool'), dev('tables'), dev('raw_pool'), dev('raw_tables')
    lat_len = dev('lat_len').to(torch.int32)
    raw_len = dev('raw_len').to(torch.int32)
    nb, nr = inp['lat_len'], inp['raw_len']
    lat_k, lat_v = BeaconPages(pool, layout).read_batch(tables, lat_len)
    B, HKV, D = len(nb), raw_pool.shape[3], raw_pool.shape[4]
    raw_k = torch.zeros(B, HKV, int(nr.max()), D, dtype=torch.bfloat16, device=device)
    raw_v = torch.zeros_like(raw_k)
    kernels.raw_pages(raw_pool, raw_tables, raw_k, raw_v, start=0, count=int(nr.max()), to_pages=False,
                      lengths=raw_len)
    out, lse = kernels.paged_latent_decode(dev('q'), raw_k.transpose(1, 2), raw_v.transpose(1, 2), pool, tables,
                                           lat_len, int(nb.max()), layout, dev('up_k'), dev('up_v'), meta['scale'],
                                           block_diagonal=True, raw_lengths=raw_len, rows_total=int(nb.sum()))
    torch.cuda.synchronize()
    assert _digest(torch.cat([lat_k, lat_v], -1)) == st['sha_beacon_rows']
    assert _digest(torch.stack([raw_k, raw_v], 2).transpose(1, 3)) == st['sha_raw_rows']
    assert_close(to_np(out.transpose(1, 2)), st['out'], what='C4 fixture')
    assert_lse_close(to_np(lse), st['lse'], what='C4 fixture')
