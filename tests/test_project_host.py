"""Host-side argument checks of the decode-step projection wrapper (no GPU):
every shape slimkv_decode_qkv would index without bounds is refused with
ValueError before anything reaches the device."""
import pytest
import torch

BF16 = torch.bfloat16


def _args(B=2, K=256, heads=4, kv_heads=2):
    n = (heads + 2 * kv_heads) * 128
    return dict(x=torch.zeros(B, K, dtype=BF16), weight=torch.zeros(n, K, dtype=BF16),
                bias=torch.zeros(n, dtype=BF16), heads=heads, kv_heads=kv_heads,
                cos=torch.zeros(8, 128), sin=torch.zeros(8, 128), positions=torch.zeros(B, dtype=torch.long),
                raw_k=torch.zeros(B, 4, kv_heads, 128, dtype=BF16), raw_v=torch.zeros(B, 4, kv_heads, 128, dtype=BF16),
                slot_index=torch.zeros(1, dtype=torch.long))


def _call(**over):
    from slimkv_amd import kernels
    a = _args()
    a.update(over)
    return kernels.decode_qkv(a.pop('x'), a.pop('weight'), a.pop('bias'), a.pop('heads'), a.pop('kv_heads'),
                              a.pop('cos'), a.pop('sin'), a.pop('positions'), a.pop('raw_k'), a.pop('raw_v'),
                              a.pop('slot_index'), **a)


@pytest.mark.parametrize('over,match', [
    (dict(weight=torch.zeros(8 * 128, 200, dtype=BF16)), 'weight must be'),              # K mismatch
    (dict(weight=torch.zeros(7 * 128, 256, dtype=BF16)), 'weight must be'),              # rows mismatch
    (dict(weight=torch.zeros(256, 8 * 128, dtype=BF16).t()), 'weight must be'),          # not contiguous
    (dict(bias=torch.zeros(8 * 128 - 1, dtype=BF16)), 'bias must be'),
    (dict(bias=torch.zeros(8 * 128, dtype=torch.float32)), 'bias must be'),
    (dict(positions=torch.zeros(1, dtype=torch.long)), 'positions must be'),             # fewer than B
    (dict(positions=torch.zeros(2, 1, dtype=torch.long)), 'positions must be'),          # not 1-D
    (dict(q_out=torch.zeros(2, 3 * 128, dtype=BF16)), 'q_out must be'),
    (dict(q_out=torch.zeros(3, 4 * 128, dtype=BF16)), 'q_out must be'),
    (dict(q_out=torch.zeros(4 * 128, 2, dtype=BF16).t()), 'q_out must be'),
    (dict(x=torch.zeros(5, 256, dtype=BF16)), 'x must be'),
    (dict(x=torch.zeros(256, dtype=BF16)), 'x must be'),
    (dict(heads=3), 'heads must be'),
])
def test_decode_qkv_rejects_shapes(over, match):
    with pytest.raises(ValueError, match=match):
        _call(**over)


def test_decode_qkv_refuses_cpu_tensors():
    with pytest.raises(ValueError, match='device tensors'):
        _call()
