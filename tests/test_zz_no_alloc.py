"""slimkv_latent_decode_noalloc (the allocation-free latent decode) against
slimkv_latent_decode, through the C ABI: two calls in a row on the shared
device scratch, the second smaller, each bit-identical to the workspace entry
point on the same inputs; a call too large for the scratch is refused before
anything is launched."""
import ctypes

import pytest
import torch

from slimkv_amd.workloads import latent_case

pytestmark = pytest.mark.gpu


def _noalloc(case, raw_k):
    from slimkv_amd import _lib, kernels
    a, out, lse, keep = kernels._latent_args(
        case.q, raw_k, case.raw_v, case.lat_k, case.lat_v, case.up_k, case.up_v, case.scale, None, None, True,
        False, case.q_positions, case.cos, case.sin, None, None, 0, 0, None, None)
    rc = _lib.lib().slimkv_latent_decode_noalloc(ctypes.byref(a), _lib.stream_handle(case.q.device))
    _lib.check(rc)
    torch.cuda.synchronize()
    del keep
    return out, lse


def _with_workspace(case, raw_k):
    from slimkv_amd import kernels
    out, lse = kernels.latent_decode(case.q, raw_k, case.raw_v, case.lat_k, case.lat_v, case.up_k, case.up_v,
                                     case.scale, block_diagonal=True, q_positions=case.q_positions, cos=case.cos,
                                     sin=case.sin)
    torch.cuda.synchronize()
    return out, lse


@pytest.fixture(scope='module')
def cases(device):
    big = latent_case(batch=4, context=4096, tail=124, rank_k=32, rank_v=32, seed=71, device=device)
    small = latent_case(batch=2, context=1000, tail=60, rank_k=16, rank_v=16, seed=72, device=device)
    return big, small


def test_two_calls_in_a_row_match_the_workspace_entry_point(device, cases):
    # raw K stands in already rotated: both entry points take the same bits
    for case in cases:
        print(f'noalloc: B{case.q.shape[0]} beacons {case.lat_k.shape[1]} rank {case.lat_k.shape[2] // 8}', flush=True)
        got = _noalloc(case, case.raw_k)
        want = _with_workspace(case, case.raw_k)
        assert torch.equal(got[0], want[0]), 'output differs from slimkv_latent_decode'
        assert torch.equal(got[1], want[1]), 'LSE differs from slimkv_latent_decode'
        assert torch.isfinite(got[0].float()).all()


def test_call_larger_than_the_scratch_is_refused(device):
    """64 sequences with 1024 raw rows read in 64 raw splits (asked for) need
    512 fp32 partial bytes per split and query head: about 68 MB of workspace,
    over the 32 MiB scratch."""
    from slimkv_amd import _lib, kernels
    case = latent_case(batch=2, context=600, tail=20, seed=73, device=device)
    B, Nr = 64, 1024
    gen = torch.Generator(device=device).manual_seed(74)
    q = torch.randn(B, 1, 32, 128, generator=gen, device=device).to(torch.bfloat16)
    raw = torch.randn(B, Nr, 8, 128, generator=gen, device=device).to(torch.bfloat16)
    lat = torch.randn(B, 16, 256, generator=gen, device=device).to(torch.bfloat16)
    pos = torch.full((B, 1), 599, dtype=torch.int64, device=device)
    a, out, lse, keep = kernels._latent_args(q, raw, raw, lat, lat, case.up_k, case.up_v, case.scale, None, None,
                                             True, False, pos, case.cos, case.sin, None, None, 64, 0, None, None)
    need = _lib.lib().slimkv_latent_decode_workspace(ctypes.byref(a))
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    out.fill_(3.0)
    torch.cuda.synchronize()
    rc = _lib.lib().slimkv_latent_decode_noalloc(ctypes.byref(a), _lib.stream_handle(device))
    assert rc == -3
    assert b'scratch' in _lib.lib().slimkv_last_error()
    torch.cuda.synchronize()
    assert (out == 3.0).all()
    del keep
