"""Prefill attention (MFMA flash attention, head_dim 128) against the oracle's
float64 attention with the reference's bottom-right causal rule
(flash_attn_func(causal=True) as called by modeling_llama.py:1752-1809;
the oracle follows latent_decode.py:16-41)."""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from tests.helpers import assert_close, assert_lse_close, to_np

pytestmark = pytest.mark.gpu


def _run(device, B, Lq, N, Hq, Hk, causal, seed, seqlens=None, strided=False):
    from slimkv_amd import kernels
    gen = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(B, Lq, Hq, 128, generator=gen, device=device).to(torch.bfloat16)
    if strided:          # K and V as views of one fused KV buffer
        kv = torch.randn(B, N, 2, Hk, 128, generator=gen, device=device).to(torch.bfloat16)
        k, v = kv[:, :, 0], kv[:, :, 1]
    else:
        k = torch.randn(B, N, Hk, 128, generator=gen, device=device).to(torch.bfloat16)
        v = torch.randn(B, N, Hk, 128, generator=gen, device=device).to(torch.bfloat16)
    scale = 128 ** -0.5
    lens = None if seqlens is None else torch.tensor(seqlens, dtype=torch.int32, device=device)
    out, lse = kernels.prefill_attention(q, k, v, scale, causal, seqlens_k=lens)
    torch.cuda.synchronize()
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    want = np.zeros((B, Lq, Hq, 128))
    want_lse = np.zeros((B, Hq, Lq))
    for b in range(B):
        n = N if seqlens is None else seqlens[b]
        if n == 0:
            want_lse[b] = -np.inf
            continue
        o, l = oa.eager_forward(qn[b:b + 1], kn[b:b + 1, :n], vn[b:b + 1, :n], scale, causal)
        want[b], want_lse[b] = o[0], l[0]
    assert_close(to_np(out), want)
    assert_lse_close(to_np(lse), want_lse)


@pytest.mark.parametrize('B,Lq,N,Hq,Hk', [
    (2, 200, 200, 8, 2),         # square causal, GQA 4
    (1, 1280, 1540, 8, 2),       # a window of 1024 raw + 256 beacons after 4 sinks + 256 history beacons
    (1, 128, 64, 4, 4),          # exact tiles, MHA
    (3, 77, 333, 6, 2),          # ragged tails, GQA 3
    (1, 300, 130, 4, 1),         # more queries than keys: leading rows see nothing
])
def test_causal_prefill_matches_oracle(device, B, Lq, N, Hq, Hk):
    _run(device, B, Lq, N, Hq, Hk, True, seed=Lq + N)


def test_non_causal_and_strided_kv(device):
    _run(device, 2, 90, 250, 8, 2, False, seed=1, strided=True)


def test_per_sequence_key_lengths(device):
    _run(device, 4, 64, 300, 8, 2, True, seed=2, seqlens=[300, 64, 1, 0])


def test_rejects_other_head_dims(device):
    from slimkv_amd import kernels
    x = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(RuntimeError):
        kernels.prefill_attention(x, x, x, 0.125)
