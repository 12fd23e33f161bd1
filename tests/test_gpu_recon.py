"""Reconstruction path: the MFMA up-projection (ReconstructionCache.materialize,
slimkv/llama3/memory.py:26-48) and the reconstruction decode (LlamaAttention
.forward after materialize, slimkv/llama3/modeling_llama.py:1405-1483).

Up-projection: bf16 output of an fp32-accumulated GEMM, compared with the
oracle's float64 GEMM rounded once to bf16 -- every element within one bf16
ulp (the summation order differs), almost all identical.  Decode: within the
bf16 bar (max abs 2e-2, mean 2e-3) of both the oracle's float64 attention and
its restatement of the reference eager path with bf16 score/probability
roundings.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import rope as orope
from oracle.bf16 import round_bf16
from slimkv_amd.workloads import block_diagonal, latent_case, orthonormal_columns, rope_tables
from tests.helpers import assert_close, assert_lse_close, neighbour_of_exact, to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('bd,rank,bias,B,n', [(True, 32, False, 2, 203), (True, 48, True, 2, 203),
                                              (False, 256, True, 2, 203), (True, 16, False, 2, 203),
                                              (True, 32, True, 4, 4099), (True, 64, False, 3, 1111)])
def test_reconstruct_matches_oracle_gemm(device, bd, rank, bias, B, n):
    """Per-head widths up to 64 take the streaming kernel (several 16-row tiles per
    wavefront once B * Hkv * rows / 64 exceeds its workgroup budget, ragged last
    tile); wider contractions the per-tile kernel."""
    from slimkv_amd import kernels
    gen = torch.Generator(device=device).manual_seed(rank + n)
    Hkv, D = 8, 128
    R = Hkv * rank if bd else rank
    lat = torch.randn(B, n, R, generator=gen, device=device).to(torch.bfloat16)
    if bd:
        w = block_diagonal([orthonormal_columns(D, rank, torch.Generator().manual_seed(i)) for i in range(Hkv)])
        w = w.to(device, torch.bfloat16)
    else:
        w = (torch.randn(Hkv * D, R, generator=gen, device=device) / R ** 0.5).to(torch.bfloat16)
    b = torch.randn(Hkv * D, generator=gen, device=device).to(torch.bfloat16) if bias else None
    out = kernels.reconstruct(lat, w, b, kv_heads=Hkv, block_diagonal=bd)
    torch.cuda.synchronize()
    bias_np = None if b is None else to_np(b)
    exact = oa.reconstruct(to_np(lat)[:, None], to_np(w), bias_np, Hkv, D, bf16_boundaries=False)
    rounded = oa.reconstruct(to_np(lat)[:, None], to_np(w), bias_np, Hkv, D)
    abs_terms = oa.reconstruct(np.abs(to_np(lat))[:, None], np.abs(to_np(w)), None, Hkv, D, bf16_boundaries=False)
    neighbour_of_exact(to_np(out).transpose(0, 2, 1, 3), exact, rounded, abs_terms)


@pytest.mark.parametrize('n', [37, 4099])
def test_reconstruct_scatter_and_rope_epilogue(device, n):
    from slimkv_amd import kernels
    gen = torch.Generator(device=device).manual_seed(7)
    B, Hkv, D, r = 2, 8, 128, 32
    lat = torch.randn(B, n, Hkv * r, generator=gen, device=device).to(torch.bfloat16)
    w = block_diagonal([orthonormal_columns(D, r, torch.Generator().manual_seed(10 + i)) for i in range(Hkv)])
    w = w.to(device, torch.bfloat16)
    cos, sin = rope_tables(5000, D, 500000.0, device)
    pos = torch.randint(0, 5000, (B, n), generator=gen, device=device)
    dst = torch.randperm(n + 5, generator=torch.Generator().manual_seed(3))[:n].to(device)
    out = torch.zeros(B, n + 5, Hkv, D, dtype=torch.bfloat16, device=device)
    kernels.reconstruct(lat, w, kv_heads=Hkv, out=out, dst_rows=dst, positions=pos, cos=cos, sin=sin,
                        block_diagonal=True)
    plain = kernels.reconstruct(lat, w, kv_heads=Hkv, block_diagonal=True)
    torch.cuda.synchronize()
    # RoPE epilogue is bit-exact given the bf16 reconstruction the kernel itself produced
    x = to_np(plain).astype(np.float32)                              # [B, n, Hkv, D]
    c, s = to_np(cos).astype(np.float32), to_np(sin).astype(np.float32)
    p = pos.cpu().numpy()
    rot = np.stack([orope.rotate_bf16(x[bb], c[p[bb]][:, None], s[p[bb]][:, None]) for bb in range(B)])
    got = to_np(out)[:, dst.cpu().numpy()]
    np.testing.assert_array_equal(got, rot)
    untouched = np.setdiff1d(np.arange(n + 5), dst.cpu().numpy())
    assert (to_np(out)[:, untouched] == 0).all()


def _rotate_fp32_model(x, cos_rows, sin_rows):
    """The fused route's fp32 rotation in float64: the rebuilt key before any
    rounding, the tables' bf16 (cos, sin), x*c + rotate_half(x)*s, one bf16
    rounding at the end."""
    c = round_bf16(cos_rows).astype(np.float64)
    s = round_bf16(sin_rows).astype(np.float64)
    return round_bf16(x * c + orope.rotate_half(x) * s).astype(np.float64)


def _recon_oracles(case, q_rot, k_rot, beacon_pos, lat_causal, bk=None, bv=None, rounding='reference'):
    """Float64 attention over [rebuilt beacons ; raw rows] and the reference
    eager formulation with bf16 scores/probabilities.  Rotated beacon keys are
    rebuilt as the reference does (bf16 up-projection, then its bf16 RoPE
    steps) or, rounding='fp32', as the fused route's fp32 rotation (float64
    rebuild with bias, rotated, rounded once)."""
    Hkv, D = case.kv_heads, 128
    bk_np = None if bk is None else to_np(bk)
    exact_k = rounding == 'fp32' and beacon_pos is not None
    rk = oa.reconstruct(to_np(case.lat_k)[:, None], to_np(case.up_k), bk_np, Hkv, D, bf16_boundaries=not exact_k)
    rv = oa.reconstruct(to_np(case.lat_v)[:, None], to_np(case.up_v), None if bv is None else to_np(bv), Hkv, D)
    if beacon_pos is not None:
        c, s = to_np(case.cos).astype(np.float32), to_np(case.sin).astype(np.float32)
        bp = beacon_pos.cpu().numpy()
        if exact_k:
            rk = np.stack([_rotate_fp32_model(rk[b], c[bp[b]][None], s[bp[b]][None]) for b in range(rk.shape[0])])
        else:
            rk = np.stack([orope.rotate_bf16(rk[b].astype(np.float32), c[bp[b]][None], s[bp[b]][None])
                           for b in range(rk.shape[0])]).astype(np.float64)
    raw_k, raw_v = to_np(k_rot), to_np(case.raw_v.transpose(1, 2))
    q = to_np(q_rot)                                                  # [B, H, L, D]
    B, H, L, _ = q.shape
    nl = rk.shape[2]
    exact = np.empty((B, H, L, D))
    eager = np.empty((B, H, L, D))
    lse = np.empty((B, H, L))
    for i in range(L):
        vis = nl - L + i + 1 if lat_causal else nl
        k = np.concatenate([rk[:, :, :vis], raw_k], axis=2)
        v = np.concatenate([rv[:, :, :vis], raw_v], axis=2)
        o, l = oa.eager_forward(q[:, :, i:i + 1].transpose(0, 2, 1, 3), k.transpose(0, 2, 1, 3),
                                v.transpose(0, 2, 1, 3), case.scale)
        exact[:, :, i], lse[:, :, i] = o[:, 0], l[:, :, 0]
        e, _ = oa.eager_recon_layer(q[:, :, i:i + 1], k, v, case.scale)
        eager[:, :, i] = e[:, :, 0]
    return exact, eager, lse


def _rotate(case):
    from slimkv_amd import kernels
    from slimkv_amd.workloads import decode_rope_layout
    raw_idx, history = decode_rope_layout(case)
    return kernels.rope_decode(case.q.transpose(1, 2), case.raw_k.transpose(1, 2), case.cos, case.sin,
                               case.q_positions, raw_idx, case.sinks, history)


@pytest.mark.parametrize('beacon_rope,reference_rounding', [(True, False), (True, True), (False, False)])
def test_recon_decode_qwen14b_layer_shape(device, beacon_rope, reference_rounding):
    """Qwen2.5-14B attention layer shape: 40 query / 8 KV heads (GQA 5), r 32,
    4 sinks + 128 tail, K-RoPE on the rebuilt beacons at their slot positions
    (fp32 rotation, or the reference's bf16 steps)."""
    from slimkv_amd import kernels
    case = latent_case(batch=4, heads=40, context=4096 + 132, tail=128, seed=31, device=device)
    q_rot, k_rot = _rotate(case)
    nl = case.lat_k.shape[1]
    bpos = (torch.arange(nl, device=device) * 4 + 4)[None].expand(4, -1).contiguous() if beacon_rope else None
    out, lse = kernels.recon_decode(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k,
                                    case.up_v, case.scale, beacon_positions=bpos, block_diagonal=True,
                                    q_positions=case.q_positions, cos=case.cos, sin=case.sin,
                                    reference_rounding=reference_rounding)
    torch.cuda.synchronize()
    exact, eager, lse_e = _recon_oracles(case, q_rot, k_rot, bpos, False,
                                         rounding='reference' if reference_rounding else 'fp32')
    got = to_np(out.transpose(1, 2))
    assert_close(got, exact, what='vs float64')
    assert_close(got, eager, what='vs bf16 eager')
    assert_lse_close(to_np(lse), lse_e)


# (query heads, KV heads, rank, two queries, bias): Qwen2.5-7B's 28 on 4,
# multi-query attention (one KV head: three of a workgroup's four waves have
# no head), 16 on 2 and groups of three on 4 KV heads
RECON_KV_HEAD_CASES = [(28, 4, 32, False, True), (28, 4, 48, True, False), (8, 1, 32, False, False),
                       (8, 1, 16, True, True), (16, 2, 32, True, True), (12, 4, 32, False, False)]


@pytest.mark.parametrize('reference_rounding', [False, True])
@pytest.mark.parametrize('H,Hkv,rank,insertion,bias', RECON_KV_HEAD_CASES)
def test_recon_decode_fused_kv_head_counts(device, H, Hkv, rank, insertion, bias, reference_rounding):
    """The fused route (a wave per KV head, K rebuilt and rotated per tile)
    over other KV head counts and GQA groups, with beacon K-RoPE, against
    the float64 and bf16-eager oracles."""
    from slimkv_amd import kernels
    B = 3
    case = latent_case(batch=B, heads=H, kv_heads=Hkv, context=1536 + 132, tail=128, rank_k=rank, rank_v=32,
                       seed=H + 10 * Hkv + rank, device=device)
    gen = torch.Generator(device=device).manual_seed(H + rank)
    bk = bv = None
    if bias:
        bk = (0.3 * torch.randn(case.up_k.shape[0], generator=gen, device=device)).to(torch.bfloat16)
        bv = (0.3 * torch.randn(case.up_v.shape[0], generator=gen, device=device)).to(torch.bfloat16)
    if insertion:
        case.q = torch.cat([case.q, torch.randn(case.q.shape, generator=gen, device=device).to(torch.bfloat16)], 1)
        case.q_positions = torch.cat([case.q_positions, case.q_positions + 1], 1)
        case.cos, case.sin = rope_tables(int(case.q_positions.max()) + 1, 128, 500000.0, device)
    q_rot, k_rot = _rotate(case)
    nl = case.lat_k.shape[1]
    bpos = (torch.arange(nl, device=device) * 4 + 4)[None].expand(B, -1).contiguous()
    out, lse = kernels.recon_decode(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k,
                                    case.up_v, case.scale, beacon_positions=bpos, up_k_bias=bk, up_v_bias=bv,
                                    block_diagonal=True, lat_causal=insertion, q_positions=case.q_positions,
                                    cos=case.cos, sin=case.sin, reference_rounding=reference_rounding)
    torch.cuda.synchronize()
    exact, eager, lse_e = _recon_oracles(case, q_rot, k_rot, bpos, insertion, bk, bv,
                                         rounding='reference' if reference_rounding else 'fp32')
    got = to_np(out.transpose(1, 2))
    assert_close(got, exact, what='vs float64')
    assert_close(got, eager, what='vs bf16 eager')
    assert_lse_close(to_np(lse), lse_e)


@pytest.mark.parametrize('rank', [256, 64])
def test_recon_decode_insertion_step_with_biases_general_weights(device, rank):
    """General (not block-diagonal) bases: rank 256 rebuilds V, rank 64 keeps V
    latent (shared by every head) and lifts it in the combine."""
    from slimkv_amd import kernels
    case = latent_case(batch=2, context=900, tail=40, seed=5, device=device)
    gen = torch.Generator(device=device).manual_seed(6)
    if rank != case.lat_k.shape[-1]:
        shape = case.lat_k.shape[:-1] + (rank,)
        case.lat_k = torch.randn(shape, generator=gen, device=device).to(torch.bfloat16)
        case.lat_v = torch.randn(shape, generator=gen, device=device).to(torch.bfloat16)
    case.up_k = (torch.randn(1024, rank, generator=gen, device=device) / rank ** 0.5).to(torch.bfloat16)
    case.up_v = (torch.randn(1024, rank, generator=gen, device=device) / rank ** 0.5).to(torch.bfloat16)
    bk = (0.3 * torch.randn(1024, generator=gen, device=device)).to(torch.bfloat16)
    bv = (0.3 * torch.randn(1024, generator=gen, device=device)).to(torch.bfloat16)
    case.q = torch.randn(2, 2, 32, 128, generator=gen, device=device).to(torch.bfloat16)
    case.q_positions = torch.tensor([[900, 901]] * 2, device=device)
    case.cos, case.sin = rope_tables(902, 128, 500000.0, device)
    q_rot, k_rot = _rotate(case)
    out, lse = kernels.recon_decode(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k,
                                    case.up_v, case.scale, up_k_bias=bk, up_v_bias=bv, lat_causal=True,
                                    q_positions=case.q_positions, cos=case.cos, sin=case.sin)
    torch.cuda.synchronize()
    exact, eager, lse_e = _recon_oracles(case, q_rot, k_rot, None, True, bk, bv)
    got = to_np(out.transpose(1, 2))
    assert_close(got, exact)
    assert_close(got, eager)
    assert_lse_close(to_np(lse), lse_e)


@pytest.mark.parametrize('reference_rounding', [False, True])
@pytest.mark.parametrize('rk,rv,bias,insertion', [(32, 32, True, True), (16, 64, False, False), (48, 32, True, False),
                                                  (32, 64, False, True)])
def test_recon_decode_fused_block_diagonal_variants(device, rk, rv, bias, insertion, reference_rounding):
    """Block-diagonal bases take the fused route (K rebuilt and rotated per tile
    inside the attention kernel, V lifted after the sum): K ranks 16/32/48, V
    ranks 32/64, K/V biases, the two-query insertion step with a causal beacon
    segment, beacon K-RoPE at slot positions."""
    from slimkv_amd import kernels
    case = latent_case(batch=3, heads=32, context=2048 + 132, tail=128, rank_k=rk, rank_v=rv, seed=rk + rv,
                       device=device)
    gen = torch.Generator(device=device).manual_seed(rk)
    bk = bv = None
    if bias:
        bk = (0.3 * torch.randn(case.up_k.shape[0], generator=gen, device=device)).to(torch.bfloat16)
        bv = (0.3 * torch.randn(case.up_v.shape[0], generator=gen, device=device)).to(torch.bfloat16)
    if insertion:
        case.q = torch.cat([case.q, torch.randn(case.q.shape, generator=gen, device=device).to(torch.bfloat16)], 1)
        case.q_positions = torch.cat([case.q_positions, case.q_positions + 1], 1)
        case.cos, case.sin = rope_tables(int(case.q_positions.max()) + 1, 128, 500000.0, device)
    q_rot, k_rot = _rotate(case)
    nl = case.lat_k.shape[1]
    bpos = (torch.arange(nl, device=device) * 4 + 4)[None].expand(3, -1).contiguous()
    out, lse = kernels.recon_decode(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k,
                                    case.up_v, case.scale, beacon_positions=bpos, up_k_bias=bk, up_v_bias=bv,
                                    block_diagonal=True, lat_causal=insertion, q_positions=case.q_positions,
                                    cos=case.cos, sin=case.sin, reference_rounding=reference_rounding)
    torch.cuda.synchronize()
    exact, eager, lse_e = _recon_oracles(case, q_rot, k_rot, bpos, insertion, bk, bv,
                                         rounding='reference' if reference_rounding else 'fp32')
    got = to_np(out.transpose(1, 2))
    assert_close(got, exact, what='vs float64')
    assert_close(got, eager, what='vs bf16 eager')
    assert_lse_close(to_np(lse), lse_e)


def test_recon_decode_fused_ragged_lengths(device):
    """Per-sequence beacon and raw lengths on the fused route."""
    from slimkv_amd import kernels
    case = latent_case(batch=4, heads=32, context=3000, tail=100, seed=77, device=device)
    q_rot, k_rot = _rotate(case)
    nl, nr = case.lat_k.shape[1], case.raw_k.shape[1]
    lat_len = torch.tensor([nl, 0, 1, nl // 3], dtype=torch.int32, device=device)
    raw_len = torch.tensor([nr, 7, nr - 3, 1], dtype=torch.int32, device=device)
    bpos = (torch.arange(nl, device=device) * 4 + 4)[None].expand(4, -1).contiguous()
    out, lse = kernels.recon_decode(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k,
                                    case.up_v, case.scale, beacon_positions=bpos, block_diagonal=True,
                                    q_positions=case.q_positions, cos=case.cos, sin=case.sin,
                                    lat_lengths=lat_len, raw_lengths=raw_len)
    torch.cuda.synchronize()
    from types import SimpleNamespace
    for b in range(4):
        nb, rb = int(lat_len[b]), int(raw_len[b])
        sub = SimpleNamespace(kv_heads=case.kv_heads, scale=case.scale, cos=case.cos, sin=case.sin,
                              lat_k=case.lat_k[b:b + 1, :nb], lat_v=case.lat_v[b:b + 1, :nb],
                              up_k=case.up_k, up_v=case.up_v, raw_v=case.raw_v[b:b + 1, :rb])
        exact, _, lse_e = _recon_oracles(sub, q_rot[b:b + 1], k_rot[b:b + 1, :, :rb], bpos[b:b + 1, :nb], False,
                                         rounding='fp32')
        assert_close(to_np(out.transpose(1, 2))[b:b + 1], exact, what=f'sequence {b}')
        assert_lse_close(to_np(lse)[b:b + 1], lse_e)


def test_recon_decode_general_rope_tables_take_the_materialising_route(device):
    """RoPE tables whose rows do not repeat their first half cannot use the
    fused route's half-row pairs; the call rebuilds rotated K into the
    workspace instead and still matches the oracle."""
    from slimkv_amd import kernels
    case = latent_case(batch=2, heads=32, context=1500, tail=64, seed=91, device=device)
    gen = torch.Generator(device=device).manual_seed(92)
    rows = case.cos.shape[0]
    ang = torch.rand(rows, 128, generator=gen, device=device) * 6.28
    case.cos, case.sin = torch.cos(ang), torch.sin(ang)          # no repeated halves
    _, repeats = kernels.prepare_rope_pairs(case.cos, case.sin)
    assert not repeats
    q_rot, k_rot = _rotate(case)
    nl = case.lat_k.shape[1]
    bpos = (torch.arange(nl, device=device) * 4 + 4)[None].expand(2, -1).contiguous()
    out, lse = kernels.recon_decode(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k,
                                    case.up_v, case.scale, beacon_positions=bpos, block_diagonal=True,
                                    q_positions=case.q_positions, cos=case.cos, sin=case.sin)
    torch.cuda.synchronize()
    exact, eager, lse_e = _recon_oracles(case, q_rot, k_rot, bpos, False)
    got = to_np(out.transpose(1, 2))
    assert_close(got, exact, what='vs float64')
    assert_close(got, eager, what='vs bf16 eager')
    assert_lse_close(to_np(lse), lse_e)


def test_recon_decode_fused_query_rotation_and_stages(device):
    """The fused route rotates its queries inside the split kernel (its
    prologue stage does nothing): a call given the query and its positions
    equals, bit for bit, a call given the query already rotated by
    kernels.rope_decode (bit-exact against the oracle) without tables; and
    the three stages run as separate calls over one workspace equal one call."""
    from slimkv_amd import _lib, kernels
    case = latent_case(batch=4, heads=40, context=2048 + 132, tail=128, seed=91, device=device)
    q_rot, k_rot = _rotate(case)
    args = (k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k, case.up_v, case.scale)
    rope = dict(q_positions=case.q_positions, cos=case.cos, sin=case.sin)
    full = kernels.recon_decode(case.q, *args, block_diagonal=True, **rope)
    pre = kernels.recon_decode(q_rot.transpose(1, 2).contiguous(), *args, block_diagonal=True)
    torch.cuda.synchronize()
    assert torch.equal(full[0], pre[0]) and torch.equal(full[1], pre[1])
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=device)
    out = torch.full_like(full[0], 7.0)
    lse = torch.full_like(full[1], 7.0)
    for stage in (_lib.STAGE_PROLOGUE, _lib.STAGE_ATTEND, _lib.STAGE_COMBINE):
        kernels.recon_decode(case.q, *args, block_diagonal=True, out=out, lse=lse, workspace=ws, stages=stage, **rope)
    torch.cuda.synchronize()
    assert torch.equal(out, full[0]) and torch.equal(lse, full[1])
