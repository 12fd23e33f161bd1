"""Decode-step projections (slimkv_linear_rows, slimkv_decode_qkv) against the
float64 oracle GEMM: every bf16 output is one of the two bf16 neighbours of
the exact product up to the fp32 accumulation error, almost all its correct
rounding (as any fp32-accumulating GEMM, hipBLASLt's included).  The fused
key RoPE is bit-exact given the kernel's own bf16 key: it equals the
oracle's bf16 RoPE steps (decode_kernels.py:44-51) and slimkv_rope_decode on
that key; only the step's cache slot is written."""
import numpy as np
import pytest
import torch

from oracle import rope as orope
from oracle.bf16 import round_bf16
from slimkv_amd.workloads import rope_tables
from tests.helpers import neighbour_of_exact, to_np

pytestmark = pytest.mark.gpu


def _gemm_oracle(x, w, b):
    """(exact, rounded, sum |x||w|) of x W^T (+ b) in float64."""
    xn, wn = to_np(x), to_np(w)
    exact = xn @ wn.T + (0.0 if b is None else to_np(b))
    return exact, round_bf16(exact).astype(np.float64), np.abs(xn) @ np.abs(wn).T


@pytest.mark.parametrize('m,n,k,bias', [(1, 4096, 4096, False), (2, 4096, 4096, True), (4, 384, 1000, True),
                                        (3, 1024, 13696, False)])
def test_linear_rows_matches_oracle(device, m, n, k, bias):
    """o_proj shapes (4096 x 4096) and odd ones: K not a multiple of 512
    (a partial last pass), a long K (several passes), 1-4 rows."""
    from slimkv_amd import kernels
    gen = torch.Generator(device=device).manual_seed(m * 7 + k)
    x = torch.randn(m, k, generator=gen, device=device).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=gen, device=device) * k ** -0.5).to(torch.bfloat16)
    b = torch.randn(n, generator=gen, device=device).to(torch.bfloat16) if bias else None
    out = kernels.linear_rows(x, w, b)
    torch.cuda.synchronize()
    neighbour_of_exact(to_np(out), *_gemm_oracle(x, w, b))


def test_linear_rows_strided_rows(device):
    """Rows taken from a wider activation and written into a wider output."""
    from slimkv_amd import kernels
    gen = torch.Generator(device=device).manual_seed(3)
    big = torch.randn(2, 3, 512, generator=gen, device=device).to(torch.bfloat16)
    x = big[:, 1, :256]                                  # rows 1536 apart
    w = (torch.randn(256, 256, generator=gen, device=device) / 16).to(torch.bfloat16)
    out_big = torch.zeros(2, 384, dtype=torch.bfloat16, device=device)
    kernels.linear_rows(x, w, out=out_big[:, :256])
    torch.cuda.synchronize()
    neighbour_of_exact(to_np(out_big[:, :256]), *_gemm_oracle(x, w, None))
    assert (to_np(out_big[:, 256:]) == 0).all()


@pytest.mark.parametrize('B,bias,hq,hkv', [(1, False, 32, 8), (3, True, 40, 8), (2, True, 28, 4)])
def test_decode_qkv_matches_oracle(device, B, bias, hq, hkv):
    """Llama-3.1-8B (32/8 heads), Qwen2.5-14B (40/8, q/k/v biases) and a 28/4
    layout: q, the plain and rotated keys and v at the step's cache slot."""
    from slimkv_amd import kernels
    gen = torch.Generator(device=device).manual_seed(B * 100 + hq)
    K, D, cap = 4096 if hq != 40 else 5120, 128, 37
    x = torch.randn(B, K, generator=gen, device=device).to(torch.bfloat16)
    n = (hq + 2 * hkv) * D
    w = (torch.randn(n, K, generator=gen, device=device) * K ** -0.5).to(torch.bfloat16)
    b = torch.randn(n, generator=gen, device=device).to(torch.bfloat16) if bias else None
    cos, sin = rope_tables(70000, D, 500000.0, device)
    pos = torch.tensor([5, 69999, 1234, 77][:B], device=device)
    pos[-1] = 99999 if B == 3 else pos[-1]                 # past the table: clamped to its last row
    fill = lambda: torch.full((B, cap, hkv, D), 7.0, dtype=torch.bfloat16, device=device)
    raw_k, raw_v, plain_k = fill(), fill(), fill()
    slot = torch.tensor([cap - 2], device=device)
    q = kernels.decode_qkv(x, w, b, hq, hkv, cos, sin, pos, raw_k, raw_v, slot, plain_k=plain_k)
    torch.cuda.synchronize()
    exact, rounded, abs_terms = _gemm_oracle(x, w, b)
    nq, nkv = hq * D, hkv * D
    got_k = to_np(plain_k[:, cap - 2]).reshape(B, nkv)
    neighbour_of_exact(np.concatenate([to_np(q), got_k, to_np(raw_v[:, cap - 2]).reshape(B, nkv)], 1),
                       exact, rounded, abs_terms)
    # RoPE: the oracle's bf16 steps on the kernel's own key, and slimkv_rope_decode
    p = pos.clamp(max=cos.shape[0] - 1).cpu().numpy()
    c, s = to_np(cos).astype(np.float32), to_np(sin).astype(np.float32)
    want = np.stack([orope.rotate_bf16(got_k[i].reshape(hkv, D).astype(np.float32), c[p[i]][None], s[p[i]][None])
                     for i in range(B)])
    np.testing.assert_array_equal(to_np(raw_k[:, cap - 2]), want)
    qz = torch.zeros(B, 1, 1, D, dtype=torch.bfloat16, device=device)
    _, k_rot = kernels.rope_decode(qz, plain_k[:, cap - 2:cap - 1].transpose(1, 2), cos, sin, pos[:, None], None, 0, 0)
    assert torch.equal(k_rot.transpose(1, 2)[:, 0], raw_k[:, cap - 2])
    # every other slot untouched
    for cache in (raw_k, raw_v, plain_k):
        others = torch.cat([cache[:, :cap - 2], cache[:, cap - 1:]], 1)
        assert (others == 7.0).all()


def test_decode_qkv_without_plain_key(device):
    from slimkv_amd import kernels
    gen = torch.Generator(device=device).manual_seed(9)
    x = torch.randn(1, 4096, generator=gen, device=device).to(torch.bfloat16)
    w = (torch.randn(6144, 4096, generator=gen, device=device) / 64).to(torch.bfloat16)
    cos, sin = rope_tables(100, 128, 500000.0, device)
    raw_k = torch.zeros(1, 4, 8, 128, dtype=torch.bfloat16, device=device)
    raw_v = torch.zeros_like(raw_k)
    with_plain = torch.zeros_like(raw_k)
    slot, pos = torch.tensor([1], device=device), torch.tensor([42], device=device)
    q1 = kernels.decode_qkv(x, w, None, 32, 8, cos, sin, pos, raw_k, raw_v, slot)
    rk2, rv2 = torch.zeros_like(raw_k), torch.zeros_like(raw_k)
    q2 = kernels.decode_qkv(x, w, None, 32, 8, cos, sin, pos, rk2, rv2, slot, plain_k=with_plain)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(raw_k, rk2) and torch.equal(raw_v, rv2)


def test_projection_shape_errors(device):
    from slimkv_amd import kernels
    x = torch.zeros(5, 256, dtype=torch.bfloat16, device=device)
    w = torch.zeros(128, 256, dtype=torch.bfloat16, device=device)
    with pytest.raises(Exception, match='1 to 4 rows'):
        kernels.linear_rows(x, w)
    with pytest.raises(Exception, match='multiple of 128'):
        kernels.linear_rows(x[:2], torch.zeros(100, 256, dtype=torch.bfloat16, device=device))


@pytest.mark.parametrize('bad_slot', [-1, 4, 1 << 40])
def test_decode_qkv_slot_outside_capacity(device, bad_slot):
    """A slot outside [0, capacity) writes no cache row: IndexError without a
    status word (the reference's index_copy_ raises), SLIMKV_STATUS_BAD_SLOT in
    a caller's word; q is written either way and equals an in-range call's."""
    from slimkv_amd import _lib, kernels
    gen = torch.Generator(device=device).manual_seed(11)
    x = torch.randn(2, 512, generator=gen, device=device).to(torch.bfloat16)
    w = (torch.randn(6 * 128, 512, generator=gen, device=device) / 16).to(torch.bfloat16)
    cos, sin = rope_tables(100, 128, 500000.0, device)
    pos = torch.tensor([3, 9], device=device)
    fill = lambda: torch.full((2, 4, 2, 128), 7.0, dtype=torch.bfloat16, device=device)
    raw_k, raw_v, plain_k = fill(), fill(), fill()
    slot = torch.tensor([bad_slot], device=device)
    with pytest.raises(IndexError, match='slot'):
        kernels.decode_qkv(x, w, None, 2, 2, cos, sin, pos, raw_k, raw_v, slot, plain_k=plain_k)
    for cache in (raw_k, raw_v, plain_k):
        assert (cache == 7.0).all()
    status = torch.zeros(1, dtype=torch.int32, device=device)
    q = kernels.decode_qkv(x, w, None, 2, 2, cos, sin, pos, raw_k, raw_v, slot, plain_k=plain_k, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == _lib.STATUS_BAD_SLOT
    for cache in (raw_k, raw_v, plain_k):
        assert (cache == 7.0).all()
    good = kernels.decode_qkv(x, w, None, 2, 2, cos, sin, pos, fill(), fill(), torch.tensor([0], device=device))
    assert torch.equal(q, good)
