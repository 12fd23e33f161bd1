"""Latent rows in two tensors (history and current window, read where they lie)
give the same bits as the same rows joined into one tensor
(slimkv/llama3/fa2_decode.py:133-135 joins them every step), for block-diagonal
and global bases, the two-query causal insertion step, splits at the first,
a middle and the last row, and views of [B, 1, N, R] cache tensors.
"""
import pytest
import torch

from slimkv_amd.workloads import block_diagonal, orthonormal_columns

pytestmark = pytest.mark.gpu


def _case(device, B, Lq, nl, rank, bd, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    Hq, Hkv, D = 32, 8, 128
    R = Hkv * rank if bd else rank
    rnd = lambda *s: torch.randn(*s, generator=gen, device=device).to(torch.bfloat16)
    q = rnd(B, Lq, Hq, D)
    raw_k, raw_v = rnd(B, 133, Hkv, D), rnd(B, 133, Hkv, D)
    lat_k, lat_v = rnd(B, 1, nl, R), rnd(B, 1, nl, R)          # cache layout [B, 1, N, R]
    if bd:
        cpu = torch.Generator().manual_seed(seed)
        up_k = block_diagonal([orthonormal_columns(D, rank, cpu) for _ in range(Hkv)]).to(device, torch.bfloat16)
        up_v = block_diagonal([orthonormal_columns(D, rank, cpu) for _ in range(Hkv)]).to(device, torch.bfloat16)
    else:
        up_k = (torch.randn(Hkv * D, R, generator=gen, device=device) / R ** 0.5).to(torch.bfloat16)
        up_v = (torch.randn(Hkv * D, R, generator=gen, device=device) / R ** 0.5).to(torch.bfloat16)
    return q, raw_k, raw_v, lat_k, lat_v, up_k, up_v


@pytest.mark.parametrize('bd,rank,Lq,split', [(True, 32, 1, 1), (True, 32, 2, 700), (True, 48, 1, 1023),
                                              (True, 16, 2, 512), (False, 256, 1, 300)])
def test_two_segments_equal_joined_rows(device, bd, rank, Lq, split):
    from slimkv_amd import kernels
    B, nl = 3, 1024
    q, raw_k, raw_v, lat_k, lat_v, up_k, up_v = _case(device, B, Lq, nl, rank, bd, rank + split)
    common = dict(block_diagonal=bd, lat_causal=Lq == 2, raw_splits=2, lat_splits=8)
    print(f'bd={bd} rank={rank} Lq={Lq} split={split}', flush=True)
    joined = kernels.latent_decode(q, raw_k, raw_v, lat_k[:, 0], lat_v[:, 0], up_k, up_v, 0.088, **common)
    hist_k, win_k = lat_k[:, :, :split], lat_k[:, :, split:]
    hist_v, win_v = lat_v[:, :, :split], lat_v[:, :, split:]
    two = kernels.latent_decode(q, raw_k, raw_v, hist_k[:, 0], hist_v[:, 0], up_k, up_v, 0.088,
                                lat_k2=win_k.contiguous()[:, 0], lat_v2=win_v.contiguous()[:, 0], **common)
    torch.cuda.synchronize()
    assert torch.equal(joined[0], two[0]) and torch.equal(joined[1], two[1])


def test_empty_segments_fall_back_to_one(device):
    from slimkv_amd import kernels
    q, raw_k, raw_v, lat_k, lat_v, up_k, up_v = _case(device, 2, 1, 256, 32, True, 5)
    common = dict(block_diagonal=True, raw_splits=2, lat_splits=4)
    joined = kernels.latent_decode(q, raw_k, raw_v, lat_k[:, 0], lat_v[:, 0], up_k, up_v, 0.088, **common)
    only_second = kernels.latent_decode(q, raw_k, raw_v, lat_k[:, 0, :0], lat_v[:, 0, :0], up_k, up_v, 0.088,
                                        lat_k2=lat_k[:, 0], lat_v2=lat_v[:, 0], **common)
    only_first = kernels.latent_decode(q, raw_k, raw_v, lat_k[:, 0], lat_v[:, 0], up_k, up_v, 0.088,
                                       lat_k2=lat_k[:, 0, :0], lat_v2=lat_v[:, 0, :0], **common)
    torch.cuda.synchronize()
    assert torch.equal(joined[0], only_second[0]) and torch.equal(joined[0], only_first[0])
