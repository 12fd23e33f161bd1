"""Pins the oracle's attention algebra (oracle/attention.py) on the CPU.

eager_forward is checked against pure-Python loops (oracle/brute.py) and
against the reference test suite's own K/V-repetition formulation
(tests/test_llama_fa2_decode.py:14-23 in the reference, restated in
oracle.attention.repeat_kv_forward); the merge against one joint softmax
(reference tests/test_llama_fa2_decode.py:126-150); the latent layer against
the closed-form identity that makes it a drop-in for reconstruction:
q.(U l + b) = (U^T q).l + q.b and sum p (W l + b) = W sum p l + b sum p.
"""
import math

import numpy as np
import pytest

from oracle import attention as oa
from oracle import brute

RNG = np.random.default_rng(1234)


def rand(*shape):
    return RNG.standard_normal(shape)


@pytest.mark.parametrize('B,Q,H,Hk,N,R,Rv,causal', [
    (1, 1, 4, 2, 7, 13, 9, False), (2, 2, 4, 2, 7, 13, 17, True), (1, 2, 4, 1, 1, 6, 5, True),
    (2, 1, 8, 8, 5, 4, 4, False), (1, 2, 6, 3, 3, 8, 8, True)])
def test_eager_matches_brute_force(B, Q, H, Hk, N, R, Rv, causal):
    q, k, v = rand(B, Q, H, R), rand(B, N, Hk, R), rand(B, N, Hk, Rv)
    out, lse = oa.eager_forward(q, k, v, 0.3, causal)
    bo, bl = brute.attention(q.tolist(), k.tolist(), v.tolist(), 0.3, causal)
    np.testing.assert_allclose(out, np.array(bo), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse, np.array(bl), rtol=1e-12, atol=1e-12)


def test_eager_matches_repeat_kv_formulation_and_reference_tolerance():
    # Shapes of the reference's grouped-attention test (test_llama_latent_eager.py:25-36).
    for queries, keys, rk, rv in [(1, 7, 13, 9), (2, 7, 13, 17), (2, 1, 384, 392)]:
        q, k, v = rand(2, queries, 4, rk), rand(2, keys, 2, rk), rand(2, keys, 2, rv)
        for causal in (False, True):
            a, al = oa.eager_forward(q, k, v, 0.125, causal)
            b, bl = oa.repeat_kv_forward(q, k, v, 0.125, causal)
            np.testing.assert_allclose(a, b, atol=2e-6, rtol=2e-5)
            np.testing.assert_allclose(al, bl, atol=2e-6, rtol=2e-5)
            assert not np.isnan(a).any()


def test_masked_first_query_has_zero_output_and_neg_inf_lse():
    q, k, v = rand(1, 2, 4, 8), rand(1, 1, 1, 8), rand(1, 1, 1, 8)
    out, lse = oa.eager_forward(q, k, v, 0.5, True)
    assert np.isneginf(lse[:, :, 0]).all() and (out[:, 0] == 0).all()
    assert np.isfinite(lse[:, :, 1]).all()


def test_merge_of_two_key_halves_equals_joint_softmax():
    q, k, v = rand(2, 3, 4, 8), rand(2, 11, 2, 8), rand(2, 11, 2, 8)
    s = 1 / math.sqrt(8)
    x, xl = oa.eager_forward(q, k[:, :5], v[:, :5], s)
    y, yl = oa.eager_forward(q, k[:, 5:], v[:, 5:], s)
    joint, jl = oa.eager_forward(q, k, v, s)
    merged = oa.merge_attention(x.transpose(0, 2, 1, 3), xl, y.transpose(0, 2, 1, 3), yl).transpose(0, 2, 1, 3)
    np.testing.assert_allclose(merged, joint, rtol=1e-12, atol=1e-12)
    fused = oa.merge_fused_form(x.transpose(0, 2, 1, 3), xl, y.transpose(0, 2, 1, 3), yl).transpose(0, 2, 1, 3)
    np.testing.assert_allclose(fused, joint, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(np.logaddexp(xl, yl), jl, rtol=1e-12)


def test_zero_mass_branch_contributes_nothing():
    raw = rand(1, 4, 2, 8)
    lat = rand(1, 4, 2, 8)
    ll = np.zeros((1, 4, 2))
    ll[..., 0] = -np.inf
    out = oa.merge_attention(raw, np.zeros((1, 4, 2)), lat, ll)
    np.testing.assert_array_equal(out[:, :, 0], raw[:, :, 0])


def _layer(B=2, H=8, Hkv=2, D=16, Nr=5, Nl=9, rk=4, rv=6, L=1, blockdiag=True, bias=False):
    q = rand(B, H, L, D)
    raw_k, raw_v = rand(B, Hkv, Nr, D), rand(B, Hkv, Nr, D)
    lat_k, lat_v = rand(B, 1, Nl, Hkv * rk), rand(B, 1, Nl, Hkv * rv)
    if blockdiag:
        uk = np.zeros((Hkv * D, Hkv * rk))
        uv = np.zeros((Hkv * D, Hkv * rv))
        for h in range(Hkv):
            uk[h * D:(h + 1) * D, h * rk:(h + 1) * rk] = rand(D, rk)
            uv[h * D:(h + 1) * D, h * rv:(h + 1) * rv] = rand(D, rv)
    else:
        uk, uv = rand(Hkv * D, Hkv * rk), rand(Hkv * D, Hkv * rv)
    bk = rand(Hkv * D) if bias else None
    bv = rand(Hkv * D) if bias else None
    return q, raw_k, raw_v, lat_k, lat_v, uk, uv, bk, bv


@pytest.mark.parametrize('blockdiag', [True, False])
@pytest.mark.parametrize('bias', [False, True])
@pytest.mark.parametrize('L,causal', [(1, False), (2, True)])
def test_latent_layer_equals_attention_over_reconstructed_cache(blockdiag, bias, L, causal):
    """Closed form: reconstruct beacon K = U_k l + b_k and V = U_v l + b_v (no
    RoPE on beacon K), attend over [raw ; beacons] jointly; with the insertion
    step the raw query excludes the newest beacon."""
    q, raw_k, raw_v, lat_k, lat_v, uk, uv, bk, bv = _layer(L=L, blockdiag=blockdiag, bias=bias)
    Hkv, D = raw_k.shape[1], raw_k.shape[3]
    out, lse = oa.latent_layer(q, raw_k, raw_v, lat_k, lat_v, uk, uv, 0.25, Hkv, bk, bv, causal,
                               bf16_boundaries=False)
    rec_k = oa.reconstruct(lat_k, uk, bk, Hkv, D, bf16_boundaries=False)
    rec_v = oa.reconstruct(lat_v, uv, bv, Hkv, D, bf16_boundaries=False)
    B, H = q.shape[:2]
    expected = np.empty_like(out)
    Nl = lat_k.shape[2]
    for i in range(L):
        visible = Nl - L + i + 1 if causal else Nl
        k = np.concatenate([raw_k, rec_k[:, :, :visible]], axis=2)
        v = np.concatenate([raw_v, rec_v[:, :, :visible]], axis=2)
        o, _ = oa.eager_forward(q[:, :, i:i + 1].transpose(0, 2, 1, 3), k.transpose(0, 2, 1, 3),
                                v.transpose(0, 2, 1, 3), 0.25)
        expected[:, :, i] = o[:, 0]
    np.testing.assert_allclose(out, expected, rtol=1e-9, atol=1e-9)


def test_project_query_and_value_are_per_group_contractions():
    q = rand(2, 8, 1, 16)
    w = rand(2 * 16, 12)
    lq = oa.project_query(q, w, 2)
    for j in range(8):
        np.testing.assert_allclose(lq[:, j, 0], q[:, j, 0] @ w[(j // 4) * 16:(j // 4 + 1) * 16], rtol=1e-12)
    o = rand(2, 8, 1, 12)
    lv = oa.project_value(o, w, 2)
    for j in range(8):
        np.testing.assert_allclose(lv[:, j, 0], o[:, j, 0] @ w[(j // 4) * 16:(j // 4 + 1) * 16].T, rtol=1e-12)


@pytest.mark.parametrize('bias', [False, True])
def test_torch_restatement_agrees_with_numpy_oracle(bias):
    """Also with GQA groups of five (the Qwen2.5 layout) and both biases."""
    import torch
    from oracle import eager_torch
    q, raw_k, raw_v, lat_k, lat_v, uk, uv, bk, bv = _layer(B=2, H=10 if bias else 8, Hkv=2, D=16, Nr=6, Nl=11,
                                                           bias=bias)
    t = lambda x: None if x is None else torch.tensor(x, dtype=torch.float32)
    out = eager_torch.latent_layer(t(q), t(raw_k.transpose(0, 2, 1, 3)), t(raw_v.transpose(0, 2, 1, 3)),
                                   t(lat_k.transpose(0, 2, 1, 3)), t(lat_v.transpose(0, 2, 1, 3)), t(uk), t(uv),
                                   0.25, 2, t(bk), t(bv))
    expected, _ = oa.latent_layer(q, raw_k, raw_v, lat_k, lat_v, uk, uv, 0.25, 2, bk, bv, bf16_boundaries=False)
    np.testing.assert_allclose(out.numpy(), expected, rtol=1e-4, atol=1e-5)


def test_materialize_interleaves_window_beacons_by_role():
    B, Hkv, D, R = 1, 2, 4, 3
    sink = rand(B, Hkv, 1, D)
    hist = rand(B, 1, 2, Hkv * R)
    raw = rand(B, Hkv, 3, D)
    win = rand(B, 1, 1, Hkv * R)
    roles = np.array([0, 0, 1, 0], bool)
    up = rand(Hkv * D, Hkv * R)
    full = oa.materialize(sink, hist, raw, win, roles, up, None, Hkv, D, bf16_boundaries=False)
    assert full.shape == (B, Hkv, 1 + 2 + 4, D)
    np.testing.assert_array_equal(full[:, :, 0:1], sink)
    np.testing.assert_allclose(full[:, :, 1:3], oa.reconstruct(hist, up, None, Hkv, D, False))
    np.testing.assert_array_equal(full[:, :, [3, 4, 6]], raw)
    np.testing.assert_allclose(full[:, :, 5:6], oa.reconstruct(win, up, None, Hkv, D, False))


def test_down_project_matches_loops_and_selects_rows():
    """The down-projection oracle against explicit sums over the selected rows
    (rounding switched off), and its bf16 rounding against the bf16 module."""
    from oracle.bf16 import round_bf16
    x, w = rand(2, 7, 5), rand(3, 5)
    rows = [4, 0, 6, -1, 7]
    got = oa.down_project(x, w, rows, bf16_boundaries=False)
    for b in range(2):
        for i, r in enumerate(rows):
            for n in range(3):
                want = sum(x[b, r, k] * w[n, k] for k in range(5)) if 0 <= r < 7 else 0.0
                assert abs(got[b, i, n] - want) < 1e-12
    np.testing.assert_array_equal(oa.down_project(x, w, rows), round_bf16(got))
    np.testing.assert_array_equal(oa.down_project(x, w), oa.down_project(x, w, list(range(7))))


def _recon_loops(q, k, v, scale, mask, bf16):
    """LlamaAttention.forward's attention (modeling_llama.py:1450-1483) as
    per-element loops: query head h reads KV head h // (H / Hkv) (repeat_kv),
    bf16(q.k), bf16(* scale), + mask, fp32 softmax cast to bf16, bf16(p.v)."""
    from oracle.bf16 import round_bf16

    def rnd(x):
        return float(round_bf16(np.float64(x))) if bf16 else x
    B, H, L, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    rep = H // Hkv
    out = np.zeros((B, H, L, D))
    lse = np.zeros((B, H, L))
    for b in range(B):
        for h in range(H):
            kv = h // rep
            for i in range(L):
                s = []
                for n in range(N):
                    dot = rnd(sum(q[b, h, i, d] * k[b, kv, n, d] for d in range(D)))
                    x = rnd(dot * scale)
                    s.append(x + (mask[b, 0, i, n] if mask is not None else 0.0))
                m = max(s)
                z = sum(math.exp(x - m) for x in s)
                lse[b, h, i] = m + math.log(z)
                p = [rnd(math.exp(x - m) / z) for x in s]
                for d in range(D):
                    out[b, h, i, d] = rnd(sum(p[n] * v[b, kv, n, d] for n in range(N)))
    return out, lse


@pytest.mark.parametrize('bf16', [False, True])
def test_eager_recon_layer_matches_per_element_loops(bf16):
    """The reconstruction-route oracle against explicit loops on a tiny GQA
    case (3 query heads per KV head, a causal additive mask with one fully
    visible and one partly visible query)."""
    from oracle.bf16 import round_bf16
    B, H, Hkv, L, N, D = 2, 6, 2, 2, 5, 4
    q, k, v = (np.asarray(round_bf16(rand(*s) * 2), np.float64) for s in ((B, H, L, D), (B, Hkv, N, D), (B, Hkv, N, D)))
    mask = np.zeros((B, 1, L, N))
    mask[:, :, 0, N - 1] = -1e30                      # bottom-right causal for L = 2
    scale = 1 / math.sqrt(D)
    got, lse = oa.eager_recon_layer(q, k, v, scale, mask, bf16_boundaries=bf16)
    want, want_lse = _recon_loops(q, k, v, scale, mask, bf16)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse, want_lse, rtol=1e-12, atol=1e-12)


def test_eager_recon_layer_without_rounding_equals_grouped_eager_forward():
    """With the bf16 boundaries off the reconstruction route is plain GQA
    attention: eager_forward over the same K/V (BSHD) to 1e-12, causal mask
    included."""
    B, H, Hkv, L, N, D = 2, 8, 2, 2, 9, 16
    q, k, v = rand(B, H, L, D), rand(B, Hkv, N, D), rand(B, Hkv, N, D)
    mask = np.zeros((B, 1, L, N))
    mask[:, :, 0, N - 1] = -np.inf
    got, lse = oa.eager_recon_layer(q, k, v, 0.37, mask, bf16_boundaries=False)
    want, want_lse = oa.eager_forward(q.transpose(0, 2, 1, 3), k.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3),
                                      0.37, causal=True)
    np.testing.assert_allclose(got, want.transpose(0, 2, 1, 3), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse, want_lse, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize('rotate', [False, True])
def test_torch_recon_restatement_agrees_with_numpy_oracle(rotate):
    """The fp32 reconstruction route of the CPU baseline against the numpy
    oracle: reconstruct (no bf16 boundaries), optional rotation at beacon
    positions, float64 attention over [beacons ; raw rows]."""
    import torch
    from oracle import eager_torch
    from oracle import rope as orope
    B, H, Hkv, D, Nr, Nl, r = 2, 8, 2, 16, 5, 9, 4
    q, raw_k, raw_v = rand(B, H, 1, D), rand(B, Nr, Hkv, D), rand(B, Nr, Hkv, D)
    lat_k, lat_v = rand(B, Nl, Hkv * r), rand(B, Nl, Hkv * r)
    uk, uv = rand(Hkv * D, Hkv * r), rand(Hkv * D, Hkv * r)
    cos, sin = orope.tables(64, orope.inv_freq(D, 10000.0))
    pos = np.arange(3, 3 + Nl)
    t = lambda x: torch.tensor(np.asarray(x), dtype=torch.float32)
    got = eager_torch.recon_layer(t(q), t(raw_k), t(raw_v), t(lat_k), t(lat_v), t(uk), t(uv), 0.3, Hkv,
                                  t(cos[pos]) if rotate else None, t(sin[pos]) if rotate else None)
    rk = oa.reconstruct(lat_k[:, None], uk, None, Hkv, D, bf16_boundaries=False)     # [B, Hkv, Nl, D]
    if rotate:
        half = D // 2
        c, s = cos[pos].astype(np.float64), sin[pos].astype(np.float64)
        rk = rk * c + np.concatenate([-rk[..., half:], rk[..., :half]], axis=-1) * s
    rv = oa.reconstruct(lat_v[:, None], uv, None, Hkv, D, bf16_boundaries=False)
    k = np.concatenate([rk.transpose(0, 2, 1, 3), raw_k], axis=1)
    v = np.concatenate([rv.transpose(0, 2, 1, 3), raw_v], axis=1)
    want, _ = oa.eager_forward(q.transpose(0, 2, 1, 3), k, v, 0.3)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-4, atol=1e-5)
