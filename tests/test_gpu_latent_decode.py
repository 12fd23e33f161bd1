"""Fused latent beacon decode (one layer) against the oracle's restatement of
the reference bf16 decode path, slimkv/llama3/fa2_decode.py:143-164.

Inputs are the seeded synthetic Llama-3.1-8B decode layer: sinks and a raw
tail with RoPE'd full-dim K, beacon latents without RoPE, per-KV-head
orthonormal bases assembled into block-diagonal global weights.  Bar: max abs
2e-2, mean abs 2e-3 on the bf16 output; decode RoPE of q and raw K bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import rope as orope
from slimkv_amd.workloads import decode_rope_layout, latent_case, rope_tables
from tests.helpers import assert_close, assert_lse_close, bits, to_np

pytestmark = pytest.mark.gpu


def _rotated(case):
    """Rotate q and raw K with the HIP decode RoPE (BHSD views) and check the
    bits against the oracle rotation."""
    from slimkv_amd import kernels
    raw_idx, history = decode_rope_layout(case)
    q_bhsd = case.q.transpose(1, 2)
    k_bhsd = case.raw_k.transpose(1, 2)
    oq, ok = kernels.rope_decode(q_bhsd, k_bhsd, case.cos, case.sin, case.q_positions, raw_idx,
                                 case.sinks, history)
    torch.cuda.synchronize()
    eq, ek = orope.rope_decode(to_np(q_bhsd).astype(np.float32), to_np(k_bhsd).astype(np.float32),
                               to_np(case.cos).astype(np.float32), to_np(case.sin).astype(np.float32),
                               case.q_positions.cpu().numpy(), raw_idx.cpu().numpy(), case.sinks, history)
    from oracle.bf16 import to_bits
    assert (bits(oq) == to_bits(eq)).all(), 'decode RoPE of q is not bit-exact'
    assert (bits(ok) == to_bits(ek)).all(), 'decode RoPE of raw K is not bit-exact'
    return oq, ok      # BHSD contiguous


def _oracle(case, q_rot_bhsd, k_rot_bhsd, lat_causal=False, up_k_bias=None, up_v_bias=None,
            lat_k=None, lat_v=None):
    lat_k = case.lat_k if lat_k is None else lat_k
    lat_v = case.lat_v if lat_v is None else lat_v
    return oa.latent_layer(
        to_np(q_rot_bhsd), to_np(k_rot_bhsd), to_np(case.raw_v.transpose(1, 2)),
        to_np(lat_k)[:, None], to_np(lat_v)[:, None], to_np(case.up_k), to_np(case.up_v),
        case.scale, case.kv_heads, None if up_k_bias is None else to_np(up_k_bias),
        None if up_v_bias is None else to_np(up_v_bias), lat_causal)


def _run(case, k_rot_bhsd, block_diagonal=True, rope_in_kernel=True, q_rot=None, **kw):
    from slimkv_amd import kernels
    raw_k = k_rot_bhsd.transpose(1, 2)
    if rope_in_kernel:
        q, extra = case.q, dict(q_positions=case.q_positions, cos=case.cos, sin=case.sin)
    else:
        q, extra = q_rot, {}
    out, lse = kernels.latent_decode(q, raw_k, case.raw_v, kw.pop('lat_k', case.lat_k),
                                     kw.pop('lat_v', case.lat_v), case.up_k, case.up_v, case.scale,
                                     block_diagonal=block_diagonal, **extra, **kw)
    torch.cuda.synchronize()
    return out, lse


# (block_diagonal, prepared_bases): block-diagonal bases with the MFMA
# absorption from prepared per-head bases, the same with the generic prologue,
# and general (dense) bases.
VARIANTS = [(True, True), (True, False), (False, True)]


@pytest.mark.parametrize('block_diagonal,prepared', VARIANTS)
def test_config0_shape(device, block_diagonal, prepared):
    """B1, 32/8 heads, d 128, context 4096, t4, 4 sinks + 124 tail, r 32."""
    case = latent_case(batch=1, context=4096, tail=124, seed=0, device=device)
    q_rot, k_rot = _rotated(case)
    out, lse = _run(case, k_rot, block_diagonal, prepared_bases=prepared)
    eo, el = _oracle(case, q_rot, k_rot)
    assert_close(to_np(out.transpose(1, 2)), eo, what='out')
    assert_lse_close(to_np(lse), el, what='lse')


@pytest.mark.parametrize('rk,rv', [(16, 16), (32, 32), (48, 48), (16, 48), (48, 32)])
def test_layer_adaptive_ranks(device, rk, rv):
    case = latent_case(batch=3, context=2048, tail=128, rank_k=rk, rank_v=rv, seed=rk * 100 + rv,
                       device=device)
    q_rot, k_rot = _rotated(case)
    eo, el = _oracle(case, q_rot, k_rot)
    for bd, prep in VARIANTS:
        out, lse = _run(case, k_rot, bd, prepared_bases=prep)
        assert_close(to_np(out.transpose(1, 2)), eo, what=f'out bd={bd} prepared={prep}')
        assert_lse_close(to_np(lse), el, what=f'lse bd={bd} prepared={prep}')


def test_prerotated_query_and_biases(device):
    """q given already rotated; U_K / U_V biases fold into the LSE and output
    (fa2_decode.py:157-163)."""
    case = latent_case(batch=2, context=1500, tail=100, seed=11, device=device)
    q_rot, k_rot = _rotated(case)
    gen = torch.Generator(device=device).manual_seed(4)
    bk = (0.5 * torch.randn(case.up_k.shape[0], generator=gen, device=device)).to(torch.bfloat16)
    bv = (0.5 * torch.randn(case.up_v.shape[0], generator=gen, device=device)).to(torch.bfloat16)
    eo, el = _oracle(case, q_rot, k_rot, up_k_bias=bk, up_v_bias=bv)
    for bd, prep in VARIANTS:
        out, lse = _run(case, k_rot, bd, rope_in_kernel=False, q_rot=q_rot.transpose(1, 2),
                        up_k_bias=bk, up_v_bias=bv, prepared_bases=prep)
        assert_close(to_np(out.transpose(1, 2)), eo, what=f'out bd={bd} prepared={prep}')
        assert_lse_close(to_np(lse), el, what=f'lse bd={bd} prepared={prep}')
    for prep in (True, False):          # biases with the query rotated in the prologue
        out, lse = _run(case, k_rot, True, up_k_bias=bk, up_v_bias=bv, prepared_bases=prep)
        assert_close(to_np(out.transpose(1, 2)), eo, what=f'out rope prepared={prep}')
        assert_lse_close(to_np(lse), el, what=f'lse rope prepared={prep}')


def test_insertion_step_two_queries(device):
    """Raw token + its new beacon (Q2): the raw query sees N-1 latents, the
    beacon query sees N (fa2_decode.py:153-154; paired_decode.py:30-43)."""
    case = latent_case(batch=2, context=1000, tail=60, seed=21, device=device)
    gen = torch.Generator(device=device).manual_seed(22)
    q2 = torch.randn(2, 2, 32, 128, generator=gen, device=device).to(torch.bfloat16)
    case.q = q2
    case.q_positions = torch.tensor([[1000, 1001]] * 2, device=device)
    case.cos, case.sin = rope_tables(1002, 128, 500000.0, device)
    q_rot, k_rot = _rotated(case)
    eo, el = _oracle(case, q_rot, k_rot, lat_causal=True)
    for bd, prep in VARIANTS:
        out, lse = _run(case, k_rot, bd, lat_causal=True, prepared_bases=prep)
        assert_close(to_np(out.transpose(1, 2)), eo, what=f'out bd={bd} prepared={prep}')
        assert_lse_close(to_np(lse), el, what=f'lse bd={bd} prepared={prep}')


def test_empty_latent_branch(device):
    """No history yet: the output is the raw branch alone (fa2_decode.py:149-150)."""
    from slimkv_amd import kernels
    case = latent_case(batch=2, context=200, tail=120, seed=3, device=device)
    q_rot, k_rot = _rotated(case)
    out, lse = kernels.latent_decode(case.q, k_rot.transpose(1, 2), case.raw_v, None, None, case.up_k,
                                     case.up_v, case.scale, block_diagonal=True,
                                     q_positions=case.q_positions, cos=case.cos, sin=case.sin)
    torch.cuda.synchronize()
    eo, el = oa.eager_forward(to_np(q_rot.transpose(1, 2)), to_np(k_rot.transpose(1, 2)),
                              to_np(case.raw_v), case.scale)
    assert_close(to_np(out), eo)
    assert_lse_close(to_np(lse), el)


def test_batch16_config1_shape_reduced_context(device):
    """The batch-16 t4f4 geometry (32/8 heads, 4 sinks, 128 tail, r 32) at an
    8K context so the oracle finishes in seconds."""
    case = latent_case(batch=16, context=8192 + 132, tail=128, seed=7, device=device)
    q_rot, k_rot = _rotated(case)
    out, lse = _run(case, k_rot, True)
    eo, el = _oracle(case, q_rot, k_rot)
    assert_close(to_np(out.transpose(1, 2)), eo)
    assert_lse_close(to_np(lse), el)


def test_prepared_bases_are_the_per_head_transpose(device):
    from slimkv_amd import kernels
    case = latent_case(batch=1, context=300, tail=20, rank_k=48, seed=5, device=device)
    bases = kernels.prepare_latent_bases(case.up_k, 8)
    torch.cuda.synchronize()
    w = case.up_k.view(8, 128, 8, 48)
    want = torch.stack([w[h, :, h, :].t() for h in range(8)])
    assert torch.equal(bases, want)
    assert kernels.prepare_latent_bases(case.up_k, 8) is bases          # cached per weight version


@pytest.mark.parametrize('block_diagonal,prepared', VARIANTS)
def test_rope_rows_gathered_once_per_step_equal_positions(device, block_diagonal, prepared):
    """cos/sin rows taken at the query positions once (query_rope_rows) and
    passed without positions give the same bits as the positions and full
    tables, for per-sequence positions, two queries per step and a position
    past the table (clamped by both routes)."""
    from slimkv_amd import kernels
    case = latent_case(batch=4, context=1500, tail=70, seed=41, device=device)
    _, k_rot = _rotated(case)
    gen = torch.Generator(device=device).manual_seed(42)
    case.q = torch.randn(4, 2, 32, 128, generator=gen, device=device).to(torch.bfloat16)
    pos = torch.tensor([[1500, 1501], [9, 10], [70000, 3], [0, 1]], device=device)
    rows = kernels.query_rope_rows(case.cos, case.sin, pos)
    common = dict(block_diagonal=block_diagonal, lat_causal=True, prepared_bases=prepared)
    want = kernels.latent_decode(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k,
                                 case.up_v, case.scale, q_positions=pos, cos=case.cos, sin=case.sin, **common)
    got = kernels.latent_decode(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k,
                                case.up_v, case.scale, cos=rows[0], sin=rows[1], **common)
    torch.cuda.synchronize()
    assert torch.equal(got[0], want[0])
    assert torch.equal(got[1], want[1])


def test_rope_rows_without_positions_must_cover_every_query(device):
    from slimkv_amd import kernels
    case = latent_case(batch=3, context=300, tail=20, seed=43, device=device)
    _, k_rot = _rotated(case)
    with pytest.raises(ValueError, match='query positions'):
        kernels.latent_decode(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k,
                              case.up_v, case.scale, block_diagonal=True, cos=case.cos[:2], sin=case.sin[:2])


@pytest.mark.parametrize('block_diagonal', [True, False])
def test_stages_in_separate_calls_equal_one_call(device, block_diagonal):
    """slimkv_latent_decode_stages: the prologue, attend and combine stages run
    as three calls over one workspace write exactly what one full call writes;
    a call without the combine stage leaves the output untouched."""
    from slimkv_amd import _lib, kernels
    case = latent_case(batch=2, context=900, tail=40, seed=51, device=device)
    _, k_rot = _rotated(case)
    nbytes = kernels.latent_decode_workspace_bytes(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v,
                                                   case.up_k, case.up_v, case.scale, block_diagonal=block_diagonal,
                                                   q_positions=case.q_positions, cos=case.cos, sin=case.sin)
    want = _run(case, k_rot, block_diagonal)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
    out = torch.full_like(want[0], 7.0)
    lse = torch.full_like(want[1], 7.0)
    _run(case, k_rot, block_diagonal, workspace=ws, out=out, lse=lse,
         stages=_lib.STAGE_PROLOGUE | _lib.STAGE_ATTEND)
    torch.cuda.synchronize()
    assert (out == 7.0).all() and (lse == 7.0).all()
    _run(case, k_rot, block_diagonal, workspace=ws, out=out, lse=lse, stages=_lib.STAGE_COMBINE)
    assert torch.equal(out, want[0]) and torch.equal(lse, want[1])
    ws.zero_()
    for stage in (_lib.STAGE_PROLOGUE, _lib.STAGE_ATTEND, _lib.STAGE_COMBINE):
        _run(case, k_rot, block_diagonal, workspace=ws, out=out, lse=lse, stages=stage)
    assert torch.equal(out, want[0]) and torch.equal(lse, want[1])
    with pytest.raises(ValueError, match='stages'):
        _run(case, k_rot, block_diagonal, workspace=ws, stages=0)
    with pytest.raises(ValueError, match='workspace'):
        _run(case, k_rot, block_diagonal, stages=_lib.STAGE_ATTEND)


@pytest.mark.parametrize('rank,queries', [(32, 1), (48, 1), (32, 2)])
def test_batch1_long_context_many_splits(device, rank, queries):
    """Batch 1 at 8192 beacons: the planner fills the GPU with over 128 latent
    splits, which the 256-thread fast combine merges (the reference's B1
    decode shape, fa2_decode.py:143-164), also for the two-query insertion
    step with its causal latent branch."""
    case = latent_case(batch=1, context=8192 * 4 + 132, tail=128, rank_k=rank, rank_v=rank, seed=61 + rank,
                       device=device)
    if queries == 2:
        gen = torch.Generator(device=device).manual_seed(62)
        case.q = torch.randn(1, 2, 32, 128, generator=gen, device=device).to(torch.bfloat16)
        ctx = 8192 * 4 + 132
        case.q_positions = torch.tensor([[ctx, ctx + 1]], device=device)
        case.cos, case.sin = rope_tables(ctx + 2, 128, 500000.0, device)
    q_rot, k_rot = _rotated(case)
    out, lse = _run(case, k_rot, True, lat_causal=queries == 2)
    eo, el = _oracle(case, q_rot, k_rot, lat_causal=queries == 2)
    assert_close(to_np(out.transpose(1, 2)), eo)
    assert_lse_close(to_np(lse), el)


@pytest.mark.parametrize('rank,raw_splits,lat_splits', [(32, 5, 16), (16, 8, 56), (48, 3, 16)])
def test_one_wave_combine_matches_workgroup_combine(device, rank, raw_splits, lat_splits):
    """The one-wave merge of the split partials and the workgroup merge, on the
    same partials (one split plan; an output row stride of 129 elements is one
    the one-wave merge does not take): every output within one bf16 ulp of the
    other, the LSE within fp32 rounding, and both against the oracle."""
    case = latent_case(batch=4, context=4096 + 132, tail=128, rank_k=rank, rank_v=rank, seed=71 + rank,
                       device=device)
    q_rot, k_rot = _rotated(case)
    plan = dict(raw_splits=raw_splits, lat_splits=lat_splits)
    wave = _run(case, k_rot, True, **plan)
    wide = torch.zeros(4, 1, 32, 129, dtype=torch.bfloat16, device=device)
    group = _run(case, k_rot, True, out=wide[..., :128], **plan)
    a, b = wave[0].float(), group[0].float()
    mag = torch.maximum(a.abs(), b.abs()).clamp_min(1e-30)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    assert ((a - b).abs() <= ulp).all(), float((a - b).abs().max())
    assert torch.allclose(wave[1], group[1], rtol=1e-6, atol=1e-6)
    eo, el = _oracle(case, q_rot, k_rot)
    for name, (out, lse) in (('one-wave', wave), ('workgroup', group)):
        assert_close(to_np(out.transpose(1, 2)), eo, what=f'{name} merge, rank {rank}')
        assert_lse_close(to_np(lse), el, what=f'{name} merge, rank {rank}')


def _fused_and_staged(call, nbytes, device):
    """(one call: the split kernel makes the query operands, the prologue
    stage and the attend + combine stages as two calls over one workspace:
    the prologue kernel writes them)."""
    from slimkv_amd import _lib
    one = call(stages=_lib.STAGE_ALL, workspace=None)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
    call(stages=_lib.STAGE_PROLOGUE, workspace=ws)
    two = call(stages=_lib.STAGE_ATTEND | _lib.STAGE_COMBINE, workspace=ws)
    torch.cuda.synchronize()
    return one, two


@pytest.mark.parametrize('rank,queries,segments', [(32, 1, 1), (16, 1, 1), (48, 1, 1), (32, 2, 1), (32, 1, 2),
                                                   (48, 2, 2), (16, 2, 1)])
def test_operands_made_in_the_split_kernel_equal_the_prologue(device, rank, queries, segments):
    """With per-head bases and no K bias a full call makes the query operands
    inside the split kernel (no prologue launch): bit-identical to the
    prologue's operands consumed by the attend stage, over ragged lengths that
    leave splits of 0 to 6 tiles, the two-query insertion step and latent rows
    in two segments; and against the oracle."""
    from slimkv_amd import kernels
    case = latent_case(batch=6, context=1600 + 132, tail=128, rank_k=rank, rank_v=rank, seed=91 + rank + queries,
                       device=device)
    if queries == 2:
        gen = torch.Generator(device=device).manual_seed(92)
        case.q = torch.randn(6, 2, 32, 128, generator=gen, device=device).to(torch.bfloat16)
        case.q_positions = torch.tensor([[1732, 1733]] * 6, device=device)
        case.cos, case.sin = rope_tables(1734, 128, 500000.0, device)
    q_rot, k_rot = _rotated(case)
    n = case.lat_k.shape[1]
    lat_len = torch.tensor([n, 1, 17, 40, 100, n - 3], dtype=torch.int32, device=device)
    lat = dict(lat_k=case.lat_k, lat_v=case.lat_v)
    if segments == 2:
        cut = n - 37
        lat = dict(lat_k=case.lat_k[:, :cut], lat_v=case.lat_v[:, :cut], lat_k2=case.lat_k[:, cut:],
                   lat_v2=case.lat_v[:, cut:])
    common = dict(block_diagonal=True, lat_causal=queries == 2, q_positions=case.q_positions, cos=case.cos,
                  sin=case.sin, lat_lengths=lat_len, lat_splits=24)

    def call(stages, workspace):
        return kernels.latent_decode(case.q, k_rot.transpose(1, 2), case.raw_v, lat['lat_k'], lat['lat_v'],
                                     case.up_k, case.up_v, case.scale, lat_k2=lat.get('lat_k2'),
                                     lat_v2=lat.get('lat_v2'), stages=stages, workspace=workspace, **common)
    nbytes = kernels.latent_decode_workspace_bytes(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v,
                                                   case.up_k, case.up_v, case.scale, **common)
    one, two = _fused_and_staged(call, nbytes, device)
    assert torch.equal(one[0], two[0]) and torch.equal(one[1], two[1])
    for b in range(6):
        m = int(lat_len[b])
        eo, el = oa.latent_layer(to_np(q_rot[b:b + 1]), to_np(k_rot[b:b + 1]),
                                 to_np(case.raw_v[b:b + 1].transpose(1, 2)), to_np(case.lat_k[b:b + 1, :m])[:, None],
                                 to_np(case.lat_v[b:b + 1, :m])[:, None], to_np(case.up_k), to_np(case.up_v),
                                 case.scale, case.kv_heads, lat_causal=queries == 2)
        assert_close(to_np(one[0][b:b + 1].transpose(1, 2)), eo, what=f'sequence {b} ({m} beacons)')
        assert_lse_close(to_np(one[1][b:b + 1]), el)


QWEN_CASES = [(40, 32, 1, True), (40, 16, 1, True), (40, 48, 1, True), (40, 32, 2, True), (40, 16, 2, False),
              (40, 48, 2, False), (40, 32, 1, False)]
# GQA groups of eight (64 query heads, the Llama-70B layout) and of two, one
# and two queries: every wave takes whole KV heads, two or four of them
GROUP_CASES = [(64, 32, 1, False), (64, 48, 1, True), (64, 16, 2, False), (16, 16, 1, False), (16, 32, 2, True),
               (16, 48, 1, False), (32, 48, 2, True), (32, 32, 2, False)]


@pytest.mark.parametrize('H,rank,queries,bias', QWEN_CASES + GROUP_CASES)
def test_qwen_gqa5_shape(device, H, rank, queries, bias):
    """Qwen2.5-14B's head layout: 40 query heads on 8 KV heads (five a KV
    head, which does not pack into the eight- or sixteen-row tiles of a GQA
    group of four: every wave takes whole KV heads) with biases on both
    up-projections (attention_bias); and groups of eight and two.  One call
    -- the split kernel makes the query operands and, from its raw waves, the
    K bias's LSE shift -- is bit-identical to the prologue stage's operands
    and shift consumed by the attend and combine stages, over ragged latent
    lengths; and against the oracle (fa2_decode.py:143-164, the biases at
    :157-163)."""
    _gqa_layer(device, H, 8, rank, queries, bias)


# (query heads, KV heads, rank, queries, bias): Qwen2.5-7B's 28 on 4 (seven a
# KV head: one or two KV heads a wave, 14 query rows with two queries),
# multi-query attention (one KV head: one wave column set of 8 or 16 rows),
# and groups of three on 4 KV heads.
KV_HEAD_CASES = [(28, 4, 32, 1, True), (28, 4, 16, 2, False), (28, 4, 48, 1, False), (8, 1, 32, 1, False),
                 (8, 1, 48, 2, True), (8, 1, 16, 1, True), (12, 4, 16, 1, True), (12, 4, 32, 2, False),
                 (16, 2, 32, 1, False)]


@pytest.mark.parametrize('H,Hkv,rank,queries,bias', KV_HEAD_CASES)
def test_kv_head_counts(device, H, Hkv, rank, queries, bias):
    """Other KV head counts: the tile plan keeps whole KV heads in a wave and
    its head count divides the KV heads; same checks as the Qwen2.5-14B
    layout."""
    _gqa_layer(device, H, Hkv, rank, queries, bias)


def test_more_than_sixteen_query_rows_a_kv_head_is_refused(device):
    """128 query heads on 8 KV heads with two queries are 32 query rows a KV
    head, beyond one 16-column MFMA tile: the library refuses the call (the
    workspace query, which plans the call first, reports the planner's
    error)."""
    from slimkv_amd import kernels
    case = latent_case(batch=1, heads=128, context=400 + 132, tail=128, rank_k=32, rank_v=32, seed=5,
                       device=device)
    q = torch.zeros(1, 2, 128, 128, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match='16 query rows'):
        kernels.latent_decode(q, case.raw_k, case.raw_v, case.lat_k, case.lat_v, case.up_k, case.up_v,
                              case.scale, block_diagonal=True, lat_causal=True)


def _gqa_layer(device, H, Hkv, rank, queries, bias):
    from slimkv_amd import kernels
    B = 5
    case = latent_case(batch=B, heads=H, kv_heads=Hkv, context=1400 + 132, tail=128, rank_k=rank, rank_v=rank,
                       seed=7 * rank + queries + bias + H + 1000 * (Hkv != 8), device=device)
    if queries == 2:
        gen = torch.Generator(device=device).manual_seed(93)
        case.q = torch.randn(B, 2, H, 128, generator=gen, device=device).to(torch.bfloat16)
        case.q_positions = torch.tensor([[1532, 1533]] * B, device=device)
        case.cos, case.sin = rope_tables(1534, 128, 500000.0, device)
    q_rot, k_rot = _rotated(case)
    bk = bv = None
    if bias:
        gen = torch.Generator(device=device).manual_seed(94)
        bk = (0.5 * torch.randn(case.up_k.shape[0], generator=gen, device=device)).to(torch.bfloat16)
        bv = (0.5 * torch.randn(case.up_v.shape[0], generator=gen, device=device)).to(torch.bfloat16)
    n = case.lat_k.shape[1]
    lat_len = torch.tensor([n, 1, 30, 257, n - 5], dtype=torch.int32, device=device)
    common = dict(up_k_bias=bk, up_v_bias=bv, block_diagonal=True, lat_causal=queries == 2,
                  q_positions=case.q_positions, cos=case.cos, sin=case.sin, lat_lengths=lat_len)

    def call(stages, workspace):
        return kernels.latent_decode(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v,
                                     case.up_k, case.up_v, case.scale, stages=stages, workspace=workspace, **common)
    nbytes = kernels.latent_decode_workspace_bytes(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v,
                                                   case.up_k, case.up_v, case.scale, **common)
    one, two = _fused_and_staged(call, nbytes, device)
    assert torch.equal(one[0], two[0]) and torch.equal(one[1], two[1])
    for b in range(B):
        m = int(lat_len[b])
        eo, el = oa.latent_layer(to_np(q_rot[b:b + 1]), to_np(k_rot[b:b + 1]),
                                 to_np(case.raw_v[b:b + 1].transpose(1, 2)), to_np(case.lat_k[b:b + 1, :m])[:, None],
                                 to_np(case.lat_v[b:b + 1, :m])[:, None], to_np(case.up_k), to_np(case.up_v),
                                 case.scale, case.kv_heads, None if bk is None else to_np(bk),
                                 None if bv is None else to_np(bv), lat_causal=queries == 2)
        assert_close(to_np(one[0][b:b + 1].transpose(1, 2)), eo, what=f'sequence {b} ({m} beacons)')
        assert_lse_close(to_np(one[1][b:b + 1]), el)
