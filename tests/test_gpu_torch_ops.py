"""The torch.library operators on the GPU: torch.library.opcheck (schema,
fake-tensor agreement, AOT dispatch with dynamic shapes) for each operator,
bitwise equality with the direct slimkv_amd.kernels calls (whose parity with
the oracle the other GPU tests establish), and a torch.compile(fullgraph=True)
trace of a decode step that keeps the operators in one graph."""
import pytest
import torch

import slimkv_amd.torch_ops  # noqa: F401
from slimkv_amd import kernels
from slimkv_amd.workloads import decode_rope_layout, latent_case

pytestmark = pytest.mark.gpu
OPS = torch.ops.slimkv


def _case(device, seed=5):
    case = latent_case(batch=2, context=700, tail=40, seed=seed, device=device)
    raw_idx, history = decode_rope_layout(case)
    q_rot, k_rot = kernels.rope_decode(case.q.transpose(1, 2), case.raw_k.transpose(1, 2), case.cos, case.sin,
                                       case.q_positions, raw_idx, case.sinks, history)
    return case, raw_idx, history, q_rot, k_rot


def _latent_args(case, k_rot):
    return (case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k, case.up_v, case.scale,
            None, None, True, False, case.q_positions, case.cos, case.sin, None, None)


def test_latent_decode_operator(device):
    case, _, _, _, k_rot = _case(device)
    args = _latent_args(case, k_rot)
    torch.library.opcheck(OPS.latent_decode.default, args)
    got = OPS.latent_decode(*args)
    want = kernels.latent_decode(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k,
                                 case.up_v, case.scale, block_diagonal=True, q_positions=case.q_positions,
                                 cos=case.cos, sin=case.sin)
    torch.cuda.synchronize()
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


def test_recon_decode_operator(device):
    case, _, _, _, k_rot = _case(device, seed=6)
    nl = case.lat_k.shape[1]
    bpos = (torch.arange(nl, device=device) * 4 + 4)[None].expand(2, -1).contiguous()
    args = (case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k, case.up_v, case.scale,
            bpos, None, None, True, False, case.q_positions, case.cos, case.sin, None, None, False)
    torch.library.opcheck(OPS.recon_decode.default, args)
    got = OPS.recon_decode(*args)
    want = kernels.recon_decode(case.q, k_rot.transpose(1, 2), case.raw_v, case.lat_k, case.lat_v, case.up_k,
                                case.up_v, case.scale, beacon_positions=bpos, block_diagonal=True,
                                q_positions=case.q_positions, cos=case.cos, sin=case.sin)
    torch.cuda.synchronize()
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


def test_attention_rope_and_merge_operators(device):
    case, raw_idx, history, q_rot, k_rot = _case(device, seed=7)
    args = (case.q.transpose(1, 2), case.raw_k.transpose(1, 2), case.cos, case.sin, case.q_positions, raw_idx,
            case.sinks, history)
    torch.library.opcheck(OPS.rope_decode.default, args)
    oq, ok = OPS.rope_decode(*args)
    assert torch.equal(oq, q_rot) and torch.equal(ok, k_rot)
    q = q_rot.transpose(1, 2)
    k, v = k_rot.transpose(1, 2), case.raw_v
    lengths = torch.tensor([k.shape[1], k.shape[1] - 5], dtype=torch.int32, device=device)
    for args in ((q, k, v, case.scale, False, 0, None), (q, k, v, case.scale, False, 3, lengths)):
        torch.library.opcheck(OPS.attention.default, args)
        got = OPS.attention(*args)
        want = kernels.attention_forward(q, k, v, case.scale, False, splits=args[5], seqlens=args[6])
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
    q2 = torch.cat([q, q], 1)
    args = (q2, k, v, lengths, case.scale, 0)
    torch.library.opcheck(OPS.paired_attention.default, args)
    out, lse = OPS.attention(q, k, v, case.scale, False, 0, None)
    margs = (out.transpose(1, 2), lse, out.transpose(1, 2), lse)
    torch.library.opcheck(OPS.merge.default, margs)
    assert torch.equal(OPS.merge(*margs), kernels.merge(*margs))


def test_compiled_decode_step_is_one_graph(device):
    """A decode step (query/key RoPE, then the fused latent decode) compiled
    with fullgraph=True: tracing must not break at the operators, and the
    compiled step gives the eager step's bits."""
    case, raw_idx, history, _, _ = _case(device, seed=8)

    def step(q, raw_k, raw_v, lat_k, lat_v, up_k, up_v, cos, sin, pos, raw_idx):
        _, k_rot = OPS.rope_decode(q.transpose(1, 2), raw_k.transpose(1, 2), cos, sin, pos, raw_idx, case.sinks,
                                   history)
        return OPS.latent_decode(q, k_rot.transpose(1, 2), raw_v, lat_k, lat_v, up_k, up_v, case.scale, None, None,
                                 True, False, pos, cos, sin, None, None)

    args = (case.q, case.raw_k, case.raw_v, case.lat_k, case.lat_v, case.up_k, case.up_v, case.cos, case.sin,
            case.q_positions, raw_idx)
    compiled = torch.compile(step, backend='aot_eager', fullgraph=True)
    got = compiled(*args)
    want = step(*args)
    torch.cuda.synchronize()
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
