"""The append-only decode cache on the GPU, stepped by the schedule, against
the oracle: at every step the fused decode over the cache equals the oracle's
latent layer (slimkv/llama3/fa2_decode.py:143-164 semantics) over the cache
contents the reference's update_memory would hold (slimkv/llama3/memory.py:233-278),
through beacon insertions (two queries, causal latent branch), window
rollovers and the first-window sink refresh.  Raw K is rotated with the
bf16-exact rule at the key position each row had when it was appended."""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import rope as orope
from oracle import schedule as osched
from slimkv_amd.workloads import block_diagonal, orthonormal_columns, rope_tables
from tests.helpers import assert_close, to_np

pytestmark = pytest.mark.gpu

B, HQ, HKV, D, R = 2, 8, 2, 128, 64


def _rot(x, pos, c, s):
    """bf16-exact rotation of x [B, Hkv, D] (float32 of bf16) at integer pos."""
    return orope.rotate_bf16(x, c[pos][None, None], s[pos][None, None])


@pytest.mark.parametrize('window,ratio,processed', [(16, 4, 21), (8, 4, 3)])
def test_cache_steps_match_oracle(device, window, ratio, processed):
    from slimkv_amd import kernels
    from slimkv_amd.decode_state import DecodeSchedule, LatentDecodeCache
    gen = torch.Generator(device=device).manual_seed(window + processed)
    rnd = lambda *s: torch.randn(*s, generator=gen, device=device).to(torch.bfloat16)
    up_k = block_diagonal([orthonormal_columns(D, R // HKV, torch.Generator().manual_seed(i)) for i in range(HKV)])
    up_v = block_diagonal([orthonormal_columns(D, R // HKV, torch.Generator().manual_seed(9 + i)) for i in range(HKV)])
    up_k, up_v = up_k.to(device, torch.bfloat16), up_v.to(device, torch.bfloat16)
    cos, sin = rope_tables(4096, D, 500000.0, device)
    c, s = to_np(cos).astype(np.float32), to_np(sin).astype(np.float32)
    sched = DecodeSchedule.after_prefill(window, ratio, 1, processed)
    cache = LatentDecodeCache(B, HKV, D, R, R, window + 2, 64, device)
    # prefilled contents: token tensors by label
    tok = {}
    sink = rnd(B, 1, HKV, D), rnd(B, 1, HKV, D)
    n_raw, n_win = sched.window_raw, sched.window_beacons
    raw = rnd(B, n_raw, HKV, D), rnd(B, n_raw, HKV, D)
    hist = rnd(B, sched.history, R), rnd(B, sched.history, R)
    win = rnd(B, n_win, R), rnd(B, n_win, R)
    raw_pos = [i for i, r in enumerate(sched.roles) if r == 0] if not sched.is_full else []
    positions = torch.tensor([0] + [1 + sched.history + p for p in raw_pos], device=device)[None].expand(B, -1)
    cache.load(sink[0], sink[1], raw[0], raw[1], hist[0], hist[1], win[0], win[1], cos, sin, positions.contiguous())
    mem = osched.LatentMemory(sink=['s'], history=[f'h{i}' for i in range(sched.history)],
                              raw=[f'r{i}' for i in range(n_raw)], window=[f'w{i}' for i in range(n_win)])
    tok['s'] = (to_np(sink[0][:, 0]), to_np(sink[1][:, 0]), 0)
    for i in range(n_raw):
        tok[f'r{i}'] = (to_np(raw[0][:, i]), to_np(raw[1][:, i]), 1 + sched.history + raw_pos[i])
    for i in range(sched.history):
        tok[f'h{i}'] = (to_np(hist[0][:, i]), to_np(hist[1][:, i]))
    for i in range(n_win):
        tok[f'w{i}'] = (to_np(win[0][:, i]), to_np(win[1][:, i]))
    for step in range(2 * window + 3):
        plan = sched.step()
        L = 1 + plan.size
        q = rnd(B, L, HQ, D)
        k_new, v_new = rnd(B, 1, HKV, D), rnd(B, 1, HKV, D)
        lk, lv = (rnd(B, plan.size, R), rnd(B, plan.size, R)) if plan.size else (None, None)
        qpos = torch.arange(plan.position, plan.position + L, device=device)[None].expand(B, -1).contiguous()
        cache.prepare(plan)
        _, k_rot = kernels.rope_decode(q.transpose(1, 2), k_new.transpose(1, 2), cos, sin, qpos, None, 0, 0)
        cache.write(k_rot.transpose(1, 2), k_new, v_new, lk, lv)
        out, _ = cache.attend(q, up_k, up_v, D ** -0.5, q_positions=qpos, cos=cos, sin=sin, size=plan.size)
        torch.cuda.synchronize()
        # oracle contents: raw branch = sink + window raw + new token, latent = history + window + new beacon
        tok[f't{step}'] = (to_np(k_new[:, 0]), to_np(v_new[:, 0]), plan.position)
        if plan.size:
            tok[f'b{step}'] = (to_np(lk[:, 0]), to_np(lv[:, 0]))
        raw_labels = mem.sink + mem.raw + [f't{step}']
        lat_labels = mem.history + mem.window + ([f'b{step}'] if plan.size else [])
        rk = np.stack([_rot(tok[x][0].astype(np.float32), 0 if x == mem.sink[0] and i == 0 else tok[x][2], c, s)
                       for i, x in enumerate(raw_labels)], axis=2)
        rv = np.stack([tok[x][1] for x in raw_labels], axis=2)
        lkk = np.stack([tok[x][0] for x in lat_labels], axis=1)[:, None] if lat_labels else np.zeros((B, 1, 0, R))
        lvv = np.stack([tok[x][1] for x in lat_labels], axis=1)[:, None] if lat_labels else np.zeros((B, 1, 0, R))
        q_rot = np.stack([_rot(to_np(q)[:, l].transpose(0, 1, 2).astype(np.float32).swapaxes(0, 0),
                               plan.position + l, c, s) for l in range(L)], axis=2)
        want, _ = oa.latent_layer(q_rot, rk, rv, lkk, lvv, to_np(up_k), to_np(up_v), D ** -0.5, HKV,
                                  lat_causal=bool(plan.size))
        assert_close(to_np(out).transpose(0, 2, 1, 3), want, what=f'step {step}')
        refresh = not mem.history
        cache.commit(plan, refresh, cos, sin)
        mem.update(f't{step}', [f'b{step}'] * plan.size, plan.full)
        if refresh:
            tok[f't{step}'] = tok[f't{step}']          # the sink label now refers to this token at position 0
            mem.sink = [f't{step}']
        assert (cache.history, cache.window, cache.sink + cache.raw) == \
            (len(mem.history), len(mem.window), len(mem.sink) + len(mem.raw))
        sizes = cache.cache_bytes()
        assert sizes == mem.cache_bytes(2 * HKV * D * 2 * B, 2 * R * 2 * B)
