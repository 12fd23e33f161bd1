"""The torch.library operators (slimkv_amd.torch_ops) on the CPU: every
operator is registered, its fake implementation gives the HIP path's output
shapes and dtypes for tracing, and there is no CPU implementation to fall back
on (the reference's custom operators are CUDA-only as well,
tools/benchmark/context_decode_runtime.py:50-80)."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import slimkv_amd.torch_ops  # noqa: F401  (registers the operators)

OPS = ('attention', 'paired_attention', 'latent_decode', 'recon_decode', 'rope_decode', 'merge')
BF16 = torch.bfloat16


def test_every_operator_is_registered():
    for name in OPS:
        assert hasattr(torch.ops.slimkv, name), name


def _decode_inputs(B=2, Lq=2, Hq=32, Hkv=8, D=128, Nr=40, Nl=300, R=256):
    q = torch.empty(B, Lq, Hq, D, dtype=BF16, device='cuda')
    raw = torch.empty(B, Nr, Hkv, D, dtype=BF16, device='cuda')
    lat = torch.empty(B, Nl, R, dtype=BF16, device='cuda')
    up = torch.empty(Hkv * D, R, dtype=BF16, device='cuda')
    return q, raw, lat, up


def test_fake_shapes_of_the_decode_operators():
    with FakeTensorMode():
        q, raw, lat, up = _decode_inputs()
        out, lse = torch.ops.slimkv.latent_decode(q, raw, raw, lat, lat, up, up, 0.1, None, None, True, True, None,
                                                  None, None, None, None)
        assert out.shape == (2, 2, 32, 128) and out.dtype == BF16
        assert lse.shape == (2, 32, 2) and lse.dtype == torch.float32
        bpos = torch.empty(2, 300, dtype=torch.int64, device='cuda')
        out, lse = torch.ops.slimkv.recon_decode(q, raw, raw, lat, lat, up, up, 0.1, bpos, None, None, True, False,
                                                 None, None, None, None, None, False)
        assert out.shape == (2, 2, 32, 128) and lse.shape == (2, 32, 2)
        v = torch.empty(2, 40, 8, 64, dtype=BF16, device='cuda')
        out, lse = torch.ops.slimkv.attention(q, raw, v, 0.1, True, 0, None)
        assert out.shape == (2, 2, 32, 64) and lse.shape == (2, 32, 2) and lse.dtype == torch.float32
        lengths = torch.empty(2, dtype=torch.int32, device='cuda')
        out, lse = torch.ops.slimkv.paired_attention(q, raw, v, lengths, 0.1, 0)
        assert out.shape == (2, 2, 32, 64)


def test_fake_shapes_of_rope_and_merge():
    with FakeTensorMode():
        q = torch.empty(2, 32, 1, 128, dtype=BF16, device='cuda')
        k = torch.empty(2, 8, 45, 128, dtype=BF16, device='cuda')
        cos = torch.empty(4096, 128, device='cuda')
        pos = torch.empty(2, 1, dtype=torch.int64, device='cuda')
        oq, ok = torch.ops.slimkv.rope_decode(q, k, cos, cos, pos, None, 4, 100)
        assert oq.shape == q.shape and ok.shape == k.shape and ok.dtype == BF16
        lse = torch.empty(2, 32, 1, device='cuda')
        assert torch.ops.slimkv.merge(q, lse, q, lse).shape == q.shape


def test_no_cpu_implementation():
    q = torch.zeros(1, 1, 8, 128, dtype=BF16)
    k = torch.zeros(1, 4, 8, 128, dtype=BF16)
    with pytest.raises(NotImplementedError):
        torch.ops.slimkv.attention(q, k, k, 0.1, False, 0, None)
