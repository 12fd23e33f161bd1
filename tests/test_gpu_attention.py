"""Split-K attention kernel (the slimkv_fa2_decode_320.forward / flash_forward
boundary) against the oracle's eager attention, slimkv/llama3/latent_decode.py:16-41.

Bar: bf16 outputs within max abs 2e-2 / mean abs 2e-3 of the float64 eager
result; LSE within 2e-3; rows with no visible key have LSE -inf and output 0.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from tests.helpers import assert_close, assert_lse_close, to_np

pytestmark = pytest.mark.gpu


def _inputs(device, B, Lq, Hq, Hk, N, Wk, Wv, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(B, Lq, Hq, Wk, generator=gen, device=device).to(torch.bfloat16)
    k = torch.randn(B, N, Hk, Wk, generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn(B, N, Hk, Wv, generator=gen, device=device).to(torch.bfloat16)
    return q, k, v


CASES = [
    # B, Lq, Hq, Hk, N, Wk, Wv, causal   (what it covers)
    (2, 1, 32, 8, 133, 128, 128, False),     # Llama raw branch: sinks + tail + current
    (2, 2, 32, 8, 133, 128, 128, False),     # raw branch on the insertion step
    (3, 1, 40, 8, 517, 128, 128, False),     # Qwen GQA 5
    (2, 1, 32, 1, 992, 256, 256, False),     # global latent branch, R = 256
    (1, 2, 32, 1, 77, 256, 256, True),       # insertion step: bottom-right causal latent
    (2, 1, 32, 1, 300, 384, 384, False),     # R = 384 (r = 48), beyond the reference's 320 limit
    (2, 1, 32, 1, 300, 200, 200, False),     # width padded to a multiple of 8 by the reference
    (1, 1, 32, 1, 129, 320, 320, False),     # the reference's 320 instance width
    (2, 1, 32, 1, 250, 256, 128, False),     # distinct K / V ranks
    (1, 1, 8, 8, 4100, 128, 128, False),     # many splits
    (2, 2, 4, 2, 7, 64, 64, True),           # tiny, partial tiles
]


@pytest.mark.parametrize('B,Lq,Hq,Hk,N,Wk,Wv,causal', CASES)
def test_attention_matches_eager(device, B, Lq, Hq, Hk, N, Wk, Wv, causal):
    from slimkv_amd import kernels
    q, k, v = _inputs(device, B, Lq, Hq, Hk, N, Wk, Wv, seed=B * 1000 + N)
    scale = 1 / math.sqrt(128)
    out, lse = kernels.attention_forward(q, k, v, scale, causal)
    torch.cuda.synchronize()
    eo, el = oa.eager_forward(to_np(q), to_np(k), to_np(v), scale, causal)
    assert_close(to_np(out), eo, what='out')
    assert_lse_close(to_np(lse), el, what='lse')


def test_first_query_without_keys_has_zero_mass(device):
    """Q2 causal with one key: the first query sees nothing (fa2_decode.py:34-37)."""
    from slimkv_amd import kernels
    q, k, v = _inputs(device, 1, 2, 8, 1, 1, 256, 256, seed=5)
    out, lse = kernels.attention_forward(q, k, v, 0.125, True)
    torch.cuda.synchronize()
    assert torch.isneginf(lse[:, :, 0]).all()
    assert (out[:, 0] == 0).all()
    eo, el = oa.eager_forward(to_np(q), to_np(k), to_np(v), 0.125, True)
    assert_close(to_np(out), eo)
    assert_lse_close(to_np(lse), el)


def test_cache_seqlens_and_shared_kv_batch_stride(device):
    """Per-sequence device lengths and K/V batch stride 0, as paired decode uses
    (slimkv/llama3/paired_decode.py:38-42; binding.cpp:83-90)."""
    from slimkv_amd import kernels
    q, k, v = _inputs(device, 1, 2, 32, 1, 70, 256, 256, seed=9)
    qq = q.transpose(0, 1)                       # [2,1,H,W]
    kk, vv = k.expand(2, -1, -1, -1), v.expand(2, -1, -1, -1)
    lengths = torch.tensor([69, 70], dtype=torch.int32, device=device)
    out, lse = kernels.attention_forward(qq, kk, vv, 0.1, False, seqlens=lengths)
    torch.cuda.synchronize()
    eo, el = oa.eager_forward(to_np(q), to_np(k), to_np(v), 0.1, True)
    assert_close(to_np(out.transpose(0, 1)), eo)
    assert_lse_close(to_np(lse).transpose(2, 1, 0), el)


def test_explicit_split_counts_agree(device):
    from slimkv_amd import kernels
    q, k, v = _inputs(device, 2, 1, 32, 8, 1000, 128, 128, seed=3)
    ref, ref_lse = kernels.attention_forward(q, k, v, 0.088, False, splits=1)
    for splits in (2, 5, 16):
        out, lse = kernels.attention_forward(q, k, v, 0.088, False, splits=splits)
        torch.cuda.synchronize()
        assert_close(to_np(out), to_np(ref), max_abs=1e-2, mean_abs=1e-3)
        assert_lse_close(to_np(lse), to_np(ref_lse), atol=1e-4)


def test_rejects_bad_inputs(device):
    from slimkv_amd import kernels
    q, k, v = _inputs(device, 1, 1, 32, 8, 10, 128, 128, seed=1)
    with pytest.raises(ValueError):
        kernels.attention_forward(q, k, v[:, :9], 0.1)                                # K/V key counts differ
    with pytest.raises(ValueError):
        kernels.attention_forward(q, k[:, :0], v[:, :0], 0.1)                         # no keys
    with pytest.raises(ValueError):
        kernels.attention_forward(q[..., :12].contiguous(), k[..., :12].contiguous(), v, 0.1)  # width 12
