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


@pytest.mark.parametrize('B,Lq,N,Hq,Hk,seqlens', [
    (4, 1280, 1540, 32, 8, None),           # the window-prefill benchmark shape
    (8, 300, 700, 64, 8, [700, 1, 0, 333, 700, 64, 650, 2]),   # ragged keys, partial last block
])
def test_wide_query_tiles_on_sampled_heads(device, B, Lq, N, Hq, Hk, seqlens):
    """Full-size grids (hundreds of workgroups, ragged key lengths, a partial
    last query block); the oracle checks a sample of (batch, head) slices."""
    from slimkv_amd import kernels
    gen = torch.Generator(device=device).manual_seed(Lq)
    q = torch.randn(B, Lq, Hq, 128, generator=gen, device=device).to(torch.bfloat16)
    k = torch.randn(B, N, Hk, 128, generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn(B, N, Hk, 128, generator=gen, device=device).to(torch.bfloat16)
    scale = 128 ** -0.5
    lens = None if seqlens is None else torch.tensor(seqlens, dtype=torch.int32, device=device)
    out, lse = kernels.prefill_attention(q, k, v, scale, True, seqlens_k=lens)
    torch.cuda.synchronize()
    g = Hq // Hk
    for b, h in [(0, 0), (B - 1, Hq - 1), (1, g), (B // 2, Hq // 2 + 1), (3, 5)]:
        n = N if seqlens is None else seqlens[b]
        got = to_np(out[b:b + 1, :, h:h + 1])
        if n == 0:
            assert not got.any() and np.isneginf(to_np(lse[b, h])).all()
            continue
        qn = to_np(q[b:b + 1, :, h:h + 1])
        kn, vn = to_np(k[b:b + 1, :n, h // g:h // g + 1]), to_np(v[b:b + 1, :n, h // g:h // g + 1])
        o, l = oa.eager_forward(qn, kn, vn, scale, True)
        assert_close(got, o, what=f'batch {b} head {h}')
        assert_lse_close(to_np(lse[b:b + 1, h:h + 1]), l)


def test_reference_maximum_moves_mid_sequence(device):
    """Keys with large norms late in the sequence (rows 100-109 six times, rows
    600-619 twelve times the others) lift the scores of the queries that see
    them by far more than 2^8 (log2 units) after many tiles of ordinary keys:
    the kernel's reference maximum moves mid-sequence and the accumulated
    output is rescaled; against the oracle."""
    from slimkv_amd import kernels
    B, Lq, N, Hq, Hk = 2, 300, 900, 8, 2
    gen = torch.Generator(device=device).manual_seed(77)
    q = torch.randn(B, Lq, Hq, 128, generator=gen, device=device)
    k = torch.randn(B, N, Hk, 128, generator=gen, device=device)
    v = torch.randn(B, N, Hk, 128, generator=gen, device=device)
    k[:, 100:110] *= 6.0
    k[:, 600:620] *= 12.0
    q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    scale = 128 ** -0.5
    out, lse = kernels.prefill_attention(q, k, v, scale, True)
    torch.cuda.synchronize()
    want, want_lse = oa.eager_forward(to_np(q), to_np(k), to_np(v), scale, True)
    assert_close(to_np(out), want)
    assert_lse_close(to_np(lse), want_lse)


def test_non_causal_and_strided_kv(device):
    _run(device, 2, 90, 250, 8, 2, False, seed=1, strided=True)


def test_per_sequence_key_lengths(device):
    _run(device, 4, 64, 300, 8, 2, True, seed=2, seqlens=[300, 64, 1, 0])


@pytest.mark.parametrize('B,Lq,N,Hq,Hk,sink', [(2, 200, 330, 8, 2, 4), (1, 64, 64, 4, 1, 0)])
def test_query_rope_inside_attention_is_bit_identical(device, B, Lq, N, Hq, Hk, sink):
    """Queries rotated as the attention kernel loads them (q_positions, cos,
    sin) give the bits of prefill_rope's rotated queries fed to the same
    kernel; rope_keys gives prefill_rope's keys; the queries' positions are
    the last Lq of [B, N] (here shuffled per batch entry, so each row reads
    its own position), beacon roles in the window."""
    from slimkv_amd import kernels
    from slimkv_amd.workloads import rope_tables
    gen = torch.Generator(device=device).manual_seed(7)
    q = torch.randn(B, Lq, Hq, 128, generator=gen, device=device).to(torch.bfloat16)
    k = torch.randn(B, N, Hk, 128, generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn(B, N, Hk, 128, generator=gen, device=device).to(torch.bfloat16)
    cos, sin = rope_tables(4096, 128, 500000.0, device)
    positions = torch.stack([torch.randperm(4000, generator=torch.Generator().manual_seed(b))[:N]
                             for b in range(B)]).to(device)
    roles = torch.zeros(Lq, dtype=torch.long, device=device)
    roles[4::5] = 1
    q_rot, k_rot = kernels.prefill_rope(q.transpose(1, 2), k.transpose(1, 2), cos, sin, positions, roles, sink)
    k_only = kernels.rope_keys(k.transpose(1, 2), cos, sin, positions, roles, sink)
    want, want_lse = kernels.prefill_attention(q_rot.transpose(1, 2), k_rot.transpose(1, 2), v, 0.0883883)
    got, got_lse = kernels.prefill_attention(q, k_only.transpose(1, 2), v, 0.0883883, q_positions=positions[:, -Lq:],
                                             cos=cos, sin=sin)
    torch.cuda.synchronize()
    assert torch.equal(k_only.view(torch.int16), k_rot.view(torch.int16))
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(got_lse, want_lse)


def test_rejects_other_head_dims(device):
    from slimkv_amd import kernels
    x = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(RuntimeError):
        kernels.prefill_attention(x, x, x, 0.125)


def _neighbour_of_exact(actual, exact, abs_terms):
    """bf16 outputs of an fp32-accumulated GEMM: each within one bf16 ulp of the
    float64 result plus the fp32 accumulation bound, almost all correctly rounded."""
    from oracle.bf16 import round_bf16
    a, x = np.asarray(actual, np.float64), np.asarray(exact, np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(x), 1e-30))) - 7)
    bad = np.abs(a - x) >= ulp * 1.0001 + np.asarray(abs_terms) * 2.0 ** -20
    assert not bad.any(), list(zip(a[bad][:4], x[bad][:4]))
    assert (a == round_bf16(x)).mean() > 0.98


@pytest.mark.parametrize('K,N,blocks,rows', [
    (4096, 256, 1, 'beacons'),      # hidden -> global rank (split contraction)
    (1024, 256, 8, 'beacons'),      # per-head K_full[128] -> r 32, block-diagonal
    (512, 128, 1, 'all'),
    (1024, 384, 8, 'bad'),          # rank 48 per head; an out-of-range row gives zeros
])
def test_down_projection_matches_oracle(device, K, N, blocks, rows):
    from slimkv_amd import kernels
    from slimkv_amd.workloads import orthonormal_columns
    gen = torch.Generator(device=device).manual_seed(K + N)
    B, L = 3, 320
    x = torch.randn(B, L, K, generator=gen, device=device).to(torch.bfloat16)
    if blocks > 1:
        w = torch.zeros(N, K)
        nb, kb = N // blocks, K // blocks
        for h in range(blocks):
            w[h * nb:(h + 1) * nb, h * kb:(h + 1) * kb] = orthonormal_columns(kb, nb, torch.Generator().manual_seed(h)).t()
        w = w.to(device, torch.bfloat16)
    else:
        w = (torch.randn(N, K, generator=gen, device=device) / K ** 0.5).to(torch.bfloat16)
    if rows == 'all':
        idx = None
    else:
        idx = torch.arange(4, L, 5, device=device)           # one beacon after every 4 raw tokens
        if rows == 'bad':
            idx[3] = L + 7
    out = kernels.down_project(x, w, idx, blocks=blocks)
    torch.cuda.synchronize()
    ridx = None if idx is None else idx.cpu().numpy()
    exact = oa.down_project(to_np(x), to_np(w), ridx, bf16_boundaries=False)
    terms = oa.down_project(np.abs(to_np(x)), np.abs(to_np(w)), ridx, bf16_boundaries=False)
    _neighbour_of_exact(to_np(out), exact, terms)
    if rows == 'bad':
        assert not to_np(out)[:, 3].any()


class RotaryEmbedding:          # the type name the RoPE fusion recognises
    def __init__(self, rows, device):
        from slimkv_amd.workloads import rope_tables
        self.cos_cached, self.sin_cached = rope_tables(rows, 128, 500000.0, device)
        self.max_seq_len_cached = rows


def _prefill_module(device, per_head_down, bias, seed):
    """An attention layer as the prefill forward uses it: 8 query / 2 KV heads,
    head_dim 128, hidden 256, beacon rank 32 per KV head (global 64)."""
    from types import SimpleNamespace
    from slimkv_amd.workloads import block_diagonal, orthonormal_columns
    H, Hk, D, hidden, r = 8, 2, 128, 256, 32
    gen = torch.Generator(device=device).manual_seed(seed)

    def linear(i, o, b=False, weight=None):
        lin = torch.nn.Linear(i, o, bias=b, device=device, dtype=torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_(weight if weight is not None else torch.randn(o, i, generator=gen, device=device) / i ** 0.5)
            if b:
                lin.bias.copy_(0.3 * torch.randn(o, generator=gen, device=device))
        return lin

    up = [block_diagonal([orthonormal_columns(D, r, torch.Generator().manual_seed(seed + 10 * j + i))
                          for i in range(Hk)]).to(device, torch.bfloat16) for j in range(2)]
    if per_head_down:        # down weight [Hk*r, hidden] with hidden split per KV head
        down = [block_diagonal([orthonormal_columns(hidden // Hk, r, torch.Generator().manual_seed(seed + 50 + 10 * j + i))
                                for i in range(Hk)]).t().contiguous().to(device, torch.bfloat16) for j in range(2)]
    else:
        down = [None, None]
    config = SimpleNamespace(beacon_param=['q', 'k', 'v'], beacon_decode_backend='latent', beacon_sink_size=1,
                             _attn_implementation='flash_attention_2')
    att = SimpleNamespace(
        config=config, num_heads=H, num_key_value_heads=Hk, head_dim=D, hidden_size=hidden,
        q_proj=linear(hidden, H * D), k_proj=linear(hidden, Hk * D, bias), v_proj=linear(hidden, Hk * D, bias),
        beacon_q_proj=linear(hidden, H * D),
        beacon_k_down_proj=linear(hidden, Hk * r, weight=down[0]), beacon_v_down_proj=linear(hidden, Hk * r, weight=down[1]),
        beacon_k_up_proj=linear(Hk * r, Hk * D, bias, up[0]), beacon_v_up_proj=linear(Hk * r, Hk * D, bias, up[1]),
        rotary_emb=RotaryEmbedding(4096, device))
    att._use_shared_kv_down_proj = lambda: False
    att.o_proj_with_beacon = lambda output, size, indices: output
    return att, gen


@pytest.mark.parametrize('per_head_down,bias,n_hist', [(False, False, 24), (True, True, 40), (False, True, 0)])
def test_prefill_window_matches_oracle(device, per_head_down, bias, n_hist):
    """One prefill window: [sink | up(history latents) | 1024/4-style window of
    32 raw + 8 beacons], latents of the new beacons, output after attention."""
    from oracle import rope as orope
    from slimkv_amd.memory import ReconstructionCache
    from slimkv_amd.prefill import prefill_forward
    from slimkv_amd.prefill_ops import PrefillMetadata
    att, gen = _prefill_module(device, per_head_down, bias, seed=7 + n_hist)
    B, L, Hk, D, R = 2, 40, 2, 128, 64
    rnd = lambda *s: torch.randn(*s, generator=gen, device=device).to(torch.bfloat16)
    sink_k, sink_v = rnd(B, Hk, 1, D), rnd(B, Hk, 1, D)
    hist_k = rnd(B, 1, n_hist, R) if n_hist else None
    hist_v = rnd(B, 1, n_hist, R) if n_hist else None
    pk = ReconstructionCache(sink_k, hist_k, None, None, None, Hk, D, 'k')
    pv = ReconstructionCache(sink_v, hist_v, None, None, None, Hk, D, 'v')
    roles = torch.zeros(L, dtype=torch.long, device=device)
    roles[4::5] = 1
    N = 1 + n_hist + L
    positions = torch.arange(N, device=device)[None].expand(B, -1)
    att._prefill_metadata = PrefillMetadata((roles == 0).nonzero().flatten(), (roles != 0).nonzero().flatten(),
                                            roles, positions, False)
    hidden = (0.5 * torch.randn(B, L, 256, generator=gen, device=device)).to(torch.bfloat16)
    with torch.no_grad():
        out, none, update = prefill_forward(att, hidden, positions, (pk, pv, 8, roles))
        torch.cuda.synchronize()
        # oracle: the module's own projections, then the restated low-rank path
        q = torch.where((roles == 0)[:, None], att.q_proj(hidden), att.beacon_q_proj(hidden))
        kf, vf = att.k_proj(hidden), att.v_proj(hidden)
    brows = (roles != 0).nonzero().flatten().cpu().numpy()
    h = to_np(hidden)
    lat = {}
    cur = {}
    for kind, full in (('k', kf), ('v', vf)):
        down = getattr(att, f'beacon_{kind}_down_proj').weight
        up = getattr(att, f'beacon_{kind}_up_proj')
        lat[kind] = oa.down_project(h, to_np(down), brows)
        rec = oa.reconstruct(lat[kind][:, None], to_np(up.weight), None if up.bias is None else to_np(up.bias), Hk, D)
        c = to_np(full).reshape(B, L, Hk, D).transpose(0, 2, 1, 3).copy()
        c[:, :, brows] = rec
        cur[kind] = c
    # latents: bit-level check against the oracle GEMM (one bf16 ulp at most)
    for kind, got in (('k', update.key_latents), ('v', update.value_latents)):
        down = getattr(att, f'beacon_{kind}_down_proj').weight
        exact = oa.down_project(h, to_np(down), brows, bf16_boundaries=False)
        terms = oa.down_project(np.abs(h), np.abs(to_np(down)), brows, bf16_boundaries=False)
        assert got.shape == (B, 1, len(brows), R)
        _neighbour_of_exact(to_np(got[:, 0]), exact, terms)
    up_k, up_v = att.beacon_k_up_proj, att.beacon_v_up_proj
    bk = None if up_k.bias is None else to_np(up_k.bias)
    bv = None if up_v.bias is None else to_np(up_v.bias)
    K = oa.materialize(to_np(sink_k), None if hist_k is None else to_np(hist_k), None, None, None,
                       to_np(up_k.weight), bk, Hk, D, cur['k'])
    V = oa.materialize(to_np(sink_v), None if hist_v is None else to_np(hist_v), None, None, None,
                       to_np(up_v.weight), bv, Hk, D, cur['v'])
    c = to_np(att.rotary_emb.cos_cached).astype(np.float32)
    s = to_np(att.rotary_emb.sin_cached).astype(np.float32)
    qn = to_np(q).reshape(B, L, 8, D).transpose(0, 2, 1, 3).astype(np.float32)
    q_rot, k_rot = orope.prefill_rope(qn, K.astype(np.float32), c, s, positions.cpu().numpy(),
                                      roles.cpu().numpy(), 1)
    want, _ = oa.eager_forward(q_rot.transpose(0, 2, 1, 3), k_rot.transpose(0, 2, 1, 3), V.transpose(0, 2, 1, 3),
                               D ** -0.5, causal=True)
    assert none is None
    assert_close(to_np(out), want.reshape(B, L, 8 * D))
    assert update[2] == 8 and update.raw_indices.tolist() == (roles == 0).nonzero().flatten().tolist()


@pytest.mark.parametrize('rk,rv,rows_v', [(32, 32, 256), (16, 16, 100), (32, 16, 256), (64, 64, 0)])
def test_reconstruct_pair_equals_single_launches(device, rk, rv, rows_v):
    """slimkv_reconstruct_pair (the K and V rebuild of a window's beacon rows
    in one launch; widths that differ, or an empty second problem, take two
    launches): the bits of two slimkv_reconstruct calls, scatter and bias
    included."""
    from slimkv_amd import kernels
    from slimkv_amd.workloads import block_diagonal, orthonormal_columns
    gen = torch.Generator(device=device).manual_seed(rk + rv + rows_v)
    cpu = torch.Generator().manual_seed(5)
    B, Hk, D, L = 3, 8, 128, 300
    lat_k = torch.randn(B, 256, Hk * rk, generator=gen, device=device).to(torch.bfloat16)
    lat_v = torch.randn(B, rows_v, Hk * rv, generator=gen, device=device).to(torch.bfloat16)
    up_k = block_diagonal([orthonormal_columns(D, rk, cpu) for _ in range(Hk)]).to(device, torch.bfloat16)
    up_v = block_diagonal([orthonormal_columns(D, rv, cpu) for _ in range(Hk)]).to(device, torch.bfloat16)
    bias = torch.randn(Hk * D, generator=gen, device=device).to(torch.bfloat16)
    rows_k = torch.randperm(L, generator=torch.Generator().manual_seed(6))[:256].sort().values.to(device)
    outs = [torch.zeros(B, L, Hk, D, dtype=torch.bfloat16, device=device) for _ in range(4)]
    first = dict(latent=lat_k, weight=up_k, bias=bias, kv_heads=Hk, dst_rows=rows_k, block_diagonal=True)
    second = dict(latent=lat_v, weight=up_v, kv_heads=Hk, block_diagonal=True)
    kernels.reconstruct_pair(dict(first, out=outs[0]), dict(second, out=outs[1]))
    kernels.reconstruct(**dict(first, out=outs[2]))
    kernels.reconstruct(**dict(second, out=outs[3]))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[2]) and torch.equal(outs[1], outs[3])
    assert outs[0].abs().sum() > 0 and (rows_v == 0 or outs[1].abs().sum() > 0)


@pytest.mark.parametrize('K,N,blocks,n', [(1024, 256, 8, 256), (4096, 256, 1, 64), (512, 128, 1, 1000)])
def test_down_project_pair_equals_single_launches(device, K, N, blocks, n):
    """slimkv_down_project_pair: one launch for two projections without split
    partials, one after the other with them (the long contraction of the
    second case); the bits of two slimkv_down_project calls."""
    from slimkv_amd import kernels
    gen = torch.Generator(device=device).manual_seed(K + N + n)
    B, L = 2, max(n, 300)
    x = [torch.randn(B, L, K, generator=gen, device=device).to(torch.bfloat16) for _ in range(2)]
    w = []
    for _ in range(2):
        m = torch.randn(N, K, generator=gen, device=device)
        if blocks > 1:
            mask = torch.block_diag(*[torch.ones(N // blocks, K // blocks, device=device)] * blocks)
            m = m * mask
        w.append(m.to(torch.bfloat16))
    rows = torch.randperm(L, generator=torch.Generator().manual_seed(7))[:n].to(device)
    pair = kernels.down_project_pair(*({'x': x[j], 'weight': w[j], 'rows': rows, 'blocks': blocks} for j in (0, 1)))
    single = [kernels.down_project(x[j], w[j], rows, blocks=blocks) for j in (0, 1)]
    torch.cuda.synchronize()
    assert torch.equal(pair[0], single[0]) and torch.equal(pair[1], single[1])


def test_rope_keys_copies_values_in_the_same_launch(device):
    """rope_keys with v / out_v: the rotated keys are rope_keys' alone and the
    value rows land unchanged, strided views on both sides."""
    from slimkv_amd import kernels
    from slimkv_amd.workloads import rope_tables
    gen = torch.Generator(device=device).manual_seed(8)
    B, Hk, L, D, cap = 2, 8, 333, 128, 500
    k = torch.randn(B, L, Hk, D, generator=gen, device=device).to(torch.bfloat16).transpose(1, 2)
    v = torch.randn(B, L, Hk, D, generator=gen, device=device).to(torch.bfloat16).transpose(1, 2)
    cos, sin = rope_tables(cap, D, 500000.0, device)
    positions = torch.arange(cap, device=device)[None].expand(B, -1)[:, 100:100 + L]
    roles = torch.zeros(L, dtype=torch.long, device=device)
    roles[4::5] = 1
    store_k = torch.zeros(B, Hk, cap, D, dtype=torch.bfloat16, device=device)
    store_v = torch.zeros_like(store_k)
    kernels.rope_keys(k, cos, sin, positions, roles, 0, out_k=store_k[:, :, 100:100 + L], v=v,
                      out_v=store_v[:, :, 100:100 + L])
    alone = kernels.rope_keys(k, cos, sin, positions, roles, 0)
    torch.cuda.synchronize()
    assert torch.equal(store_k[:, :, 100:100 + L], alone)
    assert torch.equal(store_v[:, :, 100:100 + L], v)
    assert not store_v[:, :, :100].any() and not store_v[:, :, 100 + L:].any()
    with pytest.raises(ValueError):
        kernels.rope_keys(k, cos, sin, positions, roles, 0, v=v)
