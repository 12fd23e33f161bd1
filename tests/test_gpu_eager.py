"""fp32 eager attention (latent_decode.eager_forward, slimkv/llama3/latent_decode.py:
16-41) and the merge for every model dtype (merge_attention, fa2_decode.py:57-66).

fp32 inputs: outputs and LSE against the oracle's float64 attention at the
reference's own eager tolerance (atol 2e-6, rtol 2e-5,
tests/test_llama_latent_eager.py:34-35).  bf16 / fp16 inputs: fp32 arithmetic
rounded once, so every output is within half an ulp of the float64 result plus
the fp32 error.  Shapes cover GQA, K/V ranks that differ, the two-query causal
insertion step, rows that see no key (LSE -inf, zero output) and a single key.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from tests.helpers import to_np

pytestmark = pytest.mark.gpu

# (B, Lq, H, Hk, N, R, Rv, causal)
SHAPES = [
    (2, 1, 8, 2, 300, 64, 48, False),
    (1, 2, 32, 8, 993, 256, 256, True),       # insertion step: the second query sees one more key
    (3, 1, 40, 8, 129, 128, 128, False),      # GQA 5
    (1, 4, 4, 1, 2, 32, 32, True),            # more queries than keys: the first two rows see nothing
    (2, 1, 4, 4, 1, 320, 96, False),          # one key
]


def _inputs(shape, dtype, device, seed):
    B, Lq, H, Hk, N, R, Rv, causal = shape
    gen = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(B, Lq, H, R, generator=gen, device=device).to(dtype)
    k = torch.randn(B, N, Hk, R, generator=gen, device=device).to(dtype)
    v = torch.randn(B, N, Hk, Rv, generator=gen, device=device).to(dtype)
    return q, k, v, R ** -0.5, causal


@pytest.mark.parametrize('shape', SHAPES)
def test_eager_forward_fp32_matches_reference_tolerance(device, shape):
    from slimkv_amd.latent_decode import eager_forward
    q, k, v, scale, causal = _inputs(shape, torch.float32, device, 3)
    out, lse = eager_forward(q, k, v, scale, causal)
    torch.cuda.synchronize()
    want, want_lse = oa.eager_forward(to_np(q), to_np(k), to_np(v), scale, causal)
    assert out.dtype == torch.float32 and lse.dtype == torch.float32
    np.testing.assert_allclose(to_np(out), want, rtol=2e-5, atol=2e-6)
    finite = np.isfinite(want_lse)
    assert (np.isfinite(to_np(lse)) == finite).all()
    np.testing.assert_allclose(to_np(lse)[finite], want_lse[finite], rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize('dtype,rel', [(torch.bfloat16, 2.0 ** -8), (torch.float16, 2.0 ** -11)])
@pytest.mark.parametrize('shape', SHAPES[:3])
def test_eager_forward_model_dtypes_round_once(device, shape, dtype, rel):
    from slimkv_amd.latent_decode import eager_forward
    q, k, v, scale, causal = _inputs(shape, dtype, device, 5)
    out, lse = eager_forward(q, k, v, scale, causal)
    torch.cuda.synchronize()
    want, want_lse = oa.eager_forward(to_np(q), to_np(k), to_np(v), scale, causal)
    assert out.dtype == dtype
    err = np.abs(to_np(out) - want)
    assert (err <= np.abs(want) * rel + 1e-5).all(), err.max()
    np.testing.assert_allclose(to_np(lse), want_lse, rtol=2e-5, atol=2e-5)


def test_eager_forward_mixed_dtypes_meet_in_fp32(device):
    from slimkv_amd.latent_decode import eager_forward
    q, k, v, scale, causal = _inputs(SHAPES[0], torch.float32, device, 7)
    out, lse = eager_forward(q.to(torch.bfloat16), k, v, scale, causal)
    torch.cuda.synchronize()
    want, _ = oa.eager_forward(to_np(q.to(torch.bfloat16)), to_np(k), to_np(v), scale, causal)
    assert out.dtype == torch.bfloat16
    assert (np.abs(to_np(out) - want) <= np.abs(want) * 2.0 ** -8 + 1e-5).all()


@pytest.mark.parametrize('dtype,tol', [(torch.float32, 1e-6), (torch.float16, 2.0 ** -11),
                                       (torch.bfloat16, 2.0 ** -8)])
def test_merge_every_dtype_matches_closed_form(device, dtype, tol):
    """merge_attention for fp32 (the reference's torch branch), fp16 and an
    odd width (the generic kernel) against logaddexp in float64."""
    from slimkv_amd.fa2_decode import merge_attention
    gen = torch.Generator(device=device).manual_seed(11)
    B, H, L, D = 2, 8, 2, 72
    raw = torch.randn(B, H, L, D, generator=gen, device=device).to(dtype)
    lat = torch.randn(B, H, L, D, generator=gen, device=device).to(dtype)
    rl = 3 * torch.randn(B, H, L, generator=gen, device=device)
    ll = 3 * torch.randn(B, H, L, generator=gen, device=device)
    out = merge_attention(raw, rl, lat, ll)
    torch.cuda.synchronize()
    r, l = to_np(rl), to_np(ll)
    t = np.logaddexp(r, l)
    want = np.exp(r - t)[..., None] * to_np(raw) + np.exp(l - t)[..., None] * to_np(lat)
    assert out.dtype == dtype and out.shape == raw.shape
    assert (np.abs(to_np(out) - want) <= np.abs(want) * tol + 1e-6).all()
