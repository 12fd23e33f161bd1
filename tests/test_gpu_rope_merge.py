"""Decode RoPE, prefill RoPE and the LSE merge kernels against the oracle.

RoPE must be bit-exact (slimkv/llama3/decode_kernels.py:44-51,
prefill_kernels.py:40-53; the reference's own GPU gate is bitwise,
tools/validation/validate_decode_ops.py:49).  The merge is compared to the
float64 closed form within the reference gate atol 1e-3 / rtol 8e-3
(validate_decode_ops.py:61) and our bf16 bar.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import rope as orope
from oracle.bf16 import to_bits
from slimkv_amd.workloads import rope_tables
from tests.helpers import assert_close, bits, to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('B,Hq,Hk,L,N,sink,history', [(2, 32, 8, 1, 133, 4, 9000), (1, 32, 8, 2, 40, 1, 17),
                                                       (3, 40, 8, 1, 1, 0, 0), (2, 4, 2, 2, 9, 0, 5)])
def test_decode_rope_bit_exact(device, B, Hq, Hk, L, N, sink, history):
    from slimkv_amd import kernels
    gen = torch.Generator(device=device).manual_seed(N + L)
    q = (3 * torch.randn(B, L, Hq, 128, generator=gen, device=device)).to(torch.bfloat16).transpose(1, 2)
    k = (3 * torch.randn(B, N, Hk, 128, generator=gen, device=device)).to(torch.bfloat16).transpose(1, 2)
    middle = max(0, N - 1 - sink)
    raw_idx = torch.sort(torch.randperm(middle + 5, generator=torch.Generator().manual_seed(1))[:middle])[0].to(device)
    rows = sink + history + 64 + 8
    cos, sin = rope_tables(max(rows, 12000), 128, 500000.0, device)
    qpos = torch.randint(0, 11000, (B, L), generator=gen, device=device)
    oq, ok = kernels.rope_decode(q, k, cos, sin, qpos, raw_idx, sink, history)
    torch.cuda.synchronize()
    eq, ek = orope.rope_decode(to_np(q).astype(np.float32), to_np(k).astype(np.float32), to_np(cos).astype(np.float32),
                               to_np(sin).astype(np.float32), qpos.cpu().numpy(), raw_idx.cpu().numpy(), sink, history)
    assert oq.is_contiguous() and ok.is_contiguous()
    assert (bits(oq) == to_bits(eq)).all()
    assert (bits(ok) == to_bits(ek)).all()


def test_prefill_rope_leaves_beacon_keys_bit_exact(device):
    from slimkv_amd import kernels
    B, Hq, Hk, Lq, sink = 2, 8, 2, 10, 1
    roles = torch.tensor([0, 0, 1, 0, 0, 1, 0, 2, 0, 0, 0, 0], device=device)
    N = 20                                   # prefix of 8 = 1 sink + 7 history beacons
    gen = torch.Generator(device=device).manual_seed(2)
    q = torch.randn(B, Lq, Hq, 128, generator=gen, device=device).to(torch.bfloat16).transpose(1, 2)
    k = torch.randn(B, Hk, N, 128, generator=gen, device=device).to(torch.bfloat16)
    positions = torch.arange(N, device=device)[None].expand(B, -1)
    cos, sin = rope_tables(64, 128, 10000.0, device)
    oq, ok = kernels.prefill_rope(q, k, cos, sin, positions, roles, sink)
    torch.cuda.synchronize()
    eq, ek = orope.prefill_rope(to_np(q).astype(np.float32), to_np(k).astype(np.float32), to_np(cos).astype(np.float32),
                                to_np(sin).astype(np.float32), positions.cpu().numpy(), roles.cpu().numpy(), sink)
    assert (bits(oq) == to_bits(eq)).all()
    assert (bits(ok) == to_bits(ek)).all()
    mask = orope.prefill_beacon_mask(N, roles.numel(), roles.cpu().numpy(), sink)
    assert (bits(ok)[:, :, mask] == bits(k)[:, :, mask]).all()


def test_merge_matches_closed_form(device):
    from slimkv_amd import kernels
    gen = torch.Generator(device=device).manual_seed(3)
    raw = torch.randn(2, 32, 2, 128, generator=gen, device=device).to(torch.bfloat16)
    lat = torch.randn(2, 32, 2, 128, generator=gen, device=device).to(torch.bfloat16)
    rl = 5 * torch.randn(2, 32, 2, generator=gen, device=device)
    ll = 5 * torch.randn(2, 32, 2, generator=gen, device=device)
    ll[0, 0, 0] = -float('inf')             # a zero-mass branch (fa2_decode.py:34-37)
    out = kernels.merge(raw, rl, lat, ll)
    torch.cuda.synchronize()
    expected = oa.merge_attention(to_np(raw), to_np(rl), to_np(lat), to_np(ll))
    assert_close(to_np(out), expected, max_abs=1e-2, mean_abs=1e-3)
    assert (bits(out[0, 0, 0]) == bits(raw[0, 0, 0])).all()
