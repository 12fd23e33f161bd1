#!/usr/bin/env python3
"""Latent beacon decode attention benchmark on one MI355X.

Workload: Llama-3.1-8B attention layer shape, t4f4 -- batch 16, 32 query / 8 KV
heads, head_dim 128, context 32768 per sequence: 8192 beacon latent rows per
sequence, 4 sinks + a 128-token raw tail + the current token with full-dim
RoPE'd K/V.  One step is a sweep over 32 layers, each with its own buffers
(~4.6 GB, far beyond the 256 MB MALL) and a latent rank drawn per layer by seed
from {16, 32, 48} (K and V rank equal).  Each layer runs the fused decode:
query RoPE + absorption, split-K attention over raw and latent rows, combine +
V lift.  The step gathers the RoPE table rows at its query positions once (every
layer rotates at the same positions) and passes them to each layer.  The
32-layer sweep is captured once in a HIP graph and replayed.

`--workload qwen` runs the same sweep at the Qwen2.5-14B layer shape: 40 query
heads on 8 KV heads (five a KV head), biases on both up-projections (the
model's attention_bias), 48 layers.

value  = algorithmic bytes of the sweep / sweep time (GB/s), inputs resident in HBM.
roofline = the split-K attention kernel alone (it makes its own query operands):
           its algorithmic bytes per launch / its average duration measured with
           HIP events on the launch stream.
cpu_baseline = the reference eager fp32 path restated in torch, one full-shape
           rank-32 layer repeated for ~10-30 s on the host cores.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = 'decode attn GB/s and % HBM peak, Llama-3.1-8B t4f4 b16 ctx32K; decode tokens/s'
HBM_PEAK_GBPS = 8000.0

B, HQ, HKV, D = 16, 32, 8, 128
# Layer shapes of the latent sweep (B16, 32K context, t4, ranks by seed):
# the headline Llama-3.1-8B layer and the Qwen2.5-14B layer (GQA group 5,
# up-projection biases).
SHAPES = {
    'latent': dict(model='Llama-3.1-8B', hq=32, bias=False, layers=32, metric=METRIC),
    'qwen': dict(model='Qwen2.5-14B', hq=40, bias=True, layers=48,
                 metric='decode attn GB/s and % HBM peak, Qwen2.5-14B t4f4 b16 ctx32K; decode tokens/s'),
}
CONTEXT, RATIO, SINKS, TAIL = 32768, 4, 4, 128
BEACONS = CONTEXT // RATIO          # 8192 latent rows
RAW = SINKS + TAIL + 1              # sinks + tail + current token
RANKS = (16, 32, 48)


# HBM bytes per launch of the split kernel (query operands made in the
# kernel) of a rank-r layer, from two rocprofv3 --pmc passes (FETCH_SIZE, then
# WRITE_SIZE; KiB a dispatch) over
# `bench.py --layers 5 --steps 2 --warmup 1 --no-cpu --no-graph`, scaled by the
# same counters on the run's ceiling probe (its 4 GiB stream reads read
# FETCH_SIZE = half the bytes read; its 256 MiB fills WRITE_SIZE = the bytes
# written): (2 x fetch + write) x 1024.
SPLIT_TRAFFIC_BYTES = {32: (2 * 70_840.53 + 2_628.01) * 1024, 16: (2 * 37_944.51 + 2_628.01) * 1024,
                       48: (2 * 107_667.30 + 3_140.01) * 1024}
SPLIT_TRAFFIC_BYTES = {r: int(v) for r, v in SPLIT_TRAFFIC_BYTES.items()}
# the same for the Qwen2.5-14B layers (`bench.py --workload qwen --layers 5
# --steps 2 --warmup 1 --no-cpu --no-graph`, same scaling)
QWEN_SPLIT_TRAFFIC_BYTES = {32: (2 * 70_980.81 + 3_288.15) * 1024, 16: (2 * 38_075.66 + 3_614.12) * 1024,
                            48: (2 * 109_590.98 + 3_928.19) * 1024}
QWEN_SPLIT_TRAFFIC_BYTES = {r: int(v) for r, v in QWEN_SPLIT_TRAFFIC_BYTES.items()}
TRAFFIC_SOURCE = ('rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, split_kernel, scaled by the ceiling probe\'s '
                  '4 GiB stream reads and 256 MiB fills')


def layer_bytes(rk, rv, hq=HQ, bias=False):
    """Algorithmic bytes of one layer step: latent rows, raw rows, q in, out,
    and the two up-projection weights (and their biases) once."""
    rows = B * (BEACONS * HKV * (rk + rv) * 2 + RAW * HKV * D * 2 * 2)
    return rows + B * 2 * hq * D * 2 + HKV * D * (rk + rv) * 2 + (2 * HKV * D * 2 if bias else 0)


def split_kernel_bytes(rk, rv, hq=HQ):
    """Bytes the split-K kernel must read: latent rows, raw rows and q once."""
    return B * (BEACONS * HKV * (rk + rv) * 2 + RAW * HKV * D * 2 * 2 + hq * D * 2)


def fused_kernel_bytes(rk, rv, hq=HQ, bias=False):
    """The split kernel that makes its own query operands also reads U_K (and
    its bias) once."""
    return split_kernel_bytes(rk, rv, hq) + HKV * D * rk * 2 + (HKV * D * 2 if bias else 0)


REPLAYS = 50
PROFILE_REPLAYS = 20


def replay_median_ms(torch, step, replays):
    """Median of `replays` single steps, each bracketed by HIP events."""
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
    for a, b in pairs:
        a.record()
        step()
        b.record()
    torch.cuda.synchronize()
    times = sorted(a.elapsed_time(b) for a, b in pairs)
    return times[len(times) // 2]


def gpu_clocks():
    """Current shader and memory clocks of the first amdgpu card, read from the
    driver's DPM tables in sysfs (the level marked '*'); None if unreadable.
    Plain file reads: no process is started from a process that holds the GPU."""
    import glob
    import re
    for dev in sorted(glob.glob('/sys/class/drm/card*/device')):
        found = {}
        for key in ('sclk', 'mclk', 'fclk', 'socclk'):
            try:
                with open(os.path.join(dev, f'pp_dpm_{key}')) as f:
                    text = f.read()
            except OSError:
                continue
            m = re.search(r'^\s*\d+:\s*(\S+)\s*\*\s*$', text, re.M)
            if m:
                found[key] = m.group(1)
        if found:
            return found
    return None


def draw_ranks(layers, seed):
    import random
    rng = random.Random(seed)
    return [rng.choice(RANKS) for _ in range(layers)]


def make_layer(torch, device, rank, seed, cos, sin, hq=HQ, bias=False):
    from slimkv_amd import kernels
    from slimkv_amd.workloads import block_diagonal, orthonormal_columns
    gen = torch.Generator(device=device).manual_seed(seed)
    cpu_gen = torch.Generator().manual_seed(seed + 1)

    def randn(*shape):
        return torch.randn(*shape, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)

    lat_k = randn(B, BEACONS, HKV * rank)
    lat_v = randn(B, BEACONS, HKV * rank)
    raw_k = randn(B, RAW, HKV, D)
    raw_v = randn(B, RAW, HKV, D)
    q = randn(B, 1, hq, D)
    up_k = block_diagonal([orthonormal_columns(D, rank, cpu_gen) for _ in range(HKV)]).to(device, torch.bfloat16)
    up_v = block_diagonal([orthonormal_columns(D, rank, cpu_gen) for _ in range(HKV)]).to(device, torch.bfloat16)
    # up-projection biases of the size a trained Qwen2.5 layer's K/V biases take
    bk = (0.5 * randn(HKV * D).float()).to(torch.bfloat16) if bias else None
    bv = (0.5 * randn(HKV * D).float()).to(torch.bfloat16) if bias else None
    q_pos = torch.full((B, 1), CONTEXT, dtype=torch.int64, device=device)
    # Raw K is kept rotated in the cache (rotated once when appended): sinks at
    # 0..3, tail at CONTEXT-TAIL.., current token at CONTEXT.
    raw_idx = torch.arange(TAIL, device=device)
    history = CONTEXT - TAIL - SINKS
    _, k_rot = kernels.rope_decode(q.transpose(1, 2), raw_k.transpose(1, 2), cos, sin, q_pos, raw_idx,
                                   SINKS, history)
    raw_k = k_rot.transpose(1, 2).contiguous()
    return dict(rank=rank, q=q, q_pos=q_pos, raw_k=raw_k, raw_v=raw_v, lat_k=lat_k, lat_v=lat_v,
                up_k=up_k, up_v=up_v, bk=bk, bv=bv,
                out=torch.empty(B, 1, hq, D, dtype=torch.bfloat16, device=device),
                lse=torch.empty(B, hq, 1, dtype=torch.float32, device=device))


def run_layer(kernels, L, rows, scale, workspace, stages=7):
    """One layer's fused decode; `rows` = the step's RoPE rows at the query
    positions (kernels.query_rope_rows), shared by every layer of the step."""
    kernels.latent_decode(L['q'], L['raw_k'], L['raw_v'], L['lat_k'], L['lat_v'], L['up_k'], L['up_v'], scale,
                          up_k_bias=L.get('bk'), up_v_bias=L.get('bv'), block_diagonal=True, cos=rows[0],
                          sin=rows[1], out=L['out'], lse=L['lse'], workspace=workspace, stages=stages)


def cpu_baseline(torch, layer, cos, sin, scale, hq=HQ, bias=False):
    """The torch fp32 eager restatement of the reference decode path on the
    host: one full-shape layer, at every host thread and at one thread."""
    from bench_workloads import cpu_baseline as timed
    from oracle import eager_torch
    from slimkv_amd import kernels
    q_rot, _ = kernels.rope_decode(layer['q'].transpose(1, 2), layer['raw_k'].transpose(1, 2)[:, :, :1].contiguous(),
                                   cos, sin, layer['q_pos'], None, 0, 0)
    cpu = {k: None if layer.get(k) is None else layer[k].float().cpu()
           for k in ('raw_k', 'raw_v', 'lat_k', 'lat_v', 'up_k', 'up_v', 'bk', 'bv')}
    q_cpu = q_rot.float().cpu()
    lat_k, lat_v = cpu['lat_k'][:, :, None], cpu['lat_v'][:, :, None]

    def once():
        return eager_torch.latent_layer(q_cpu, cpu['raw_k'], cpu['raw_v'], lat_k, lat_v, cpu['up_k'], cpu['up_v'],
                                        scale, HKV, cpu['bk'], cpu['bv'])
    rk = layer['rank']
    return timed(torch, once, layer_bytes(rk, rk, hq, bias), 'GB/s', 1e9,
                 f'one full-shape rank-{rk} layer (B16, {hq}/{HKV} heads, 8192 beacons, 133 raw'
                 f'{", up-projection biases" if bias else ""}), torch fp32 eager restatement of the reference decode')


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=5)
    ap.add_argument('--layers', type=int, default=None, help='layers of the latent sweep (32; 48 for qwen)')
    ap.add_argument('--seed', type=int, default=0)
    ap.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline leg')
    ap.add_argument('--no-graph', action='store_true', help='time eager launches instead of graph replay')
    ap.add_argument('--workload', default='latent',
                    choices=('latent', 'qwen', 'prefill', 'recon', 'paged', 'paged_step', 'b1', 'ceiling'),
                    help='latent: the headline decode sweep; qwen: the same sweep at the Qwen2.5-14B layer '
                         'shape; prefill / recon / paged: the window prefill, '
                         'reconstruction decode and paged-cache decode workloads; paged_step: one attention '
                         'layer of a batched vLLM decode step over the pages; b1: batch-1 ms per token '
                         'at the contexts the reference publishes; ceiling: the HBM read rate a plain '
                         'stream reaches on this GPU')
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) > 1:
        print('bench.py measures one GPU: the decode path shards by sequence with no exchange, '
              'so multi-GPU runs are not part of this build (use --gpus 1).', file=sys.stderr)
        sys.exit(2)
    if os.environ.get('SLIMKV_HIP_LIBRARY'):
        # an A/B override of the library: the line says so ("library"."override")
        print(f"bench: SLIMKV_HIP_LIBRARY={os.environ['SLIMKV_HIP_LIBRARY']} overrides the in-tree library",
              file=sys.stderr, flush=True)
    if args.workload not in SHAPES:
        from bench_workloads import run_workload
        print(json.dumps(run_workload(args)), flush=True)
        return
    shape = SHAPES[args.workload]
    hq, bias = shape['hq'], shape['bias']
    if args.layers is None:
        args.layers = shape['layers']

    import torch
    from slimkv_amd import _lib, kernels
    from slimkv_amd.workloads import rope_tables

    device = torch.device('cuda:0')
    torch.cuda.set_device(device)
    scale = 1.0 / D ** 0.5
    cos, sin = rope_tables(CONTEXT + 1, D, 500000.0, device)
    ranks = draw_ranks(args.layers, args.seed)
    print(f'bench: building {args.layers} layers, ranks {ranks}', file=sys.stderr, flush=True)
    layers = [make_layer(torch, device, r, args.seed * 1000 + i, cos, sin, hq, bias) for i, r in enumerate(ranks)]
    ws_bytes = max(kernels.latent_decode_workspace_bytes(
        L['q'], L['raw_k'], L['raw_v'], L['lat_k'], L['lat_v'], L['up_k'], L['up_v'], up_k_bias=L['bk'],
        up_v_bias=L['bv'], block_diagonal=True, q_positions=L['q_pos'], cos=cos, sin=sin) for L in layers)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    torch.cuda.synchronize()

    # The step's query positions (the current token of every sequence): every
    # layer rotates its query at them, so the table rows are gathered once per
    # step, inside the timed step.
    step_pos = torch.full((B, 1), CONTEXT, dtype=torch.int64, device=device)

    def sweep():
        rows = kernels.query_rope_rows(cos, sin, step_pos)
        for L in layers:
            run_layer(kernels, L, rows, scale, workspace)

    sweep()
    torch.cuda.synchronize()
    if args.no_graph:
        step = sweep
    else:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            sweep()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            sweep()
        step = graph.replay
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed / args.steps * 1e3
    sweep_bytes = sum(layer_bytes(r, r, hq, bias) for r in ranks)
    gbps = sweep_bytes / (elapsed / args.steps) / 1e9
    print(f'bench: sweep {ms_per_step:.3f} ms, {gbps:.1f} GB/s', file=sys.stderr, flush=True)
    replay_ms = replay_median_ms(torch, step, REPLAYS)

    # The split kernel alone, as the sweep runs it: with per-head bases a call
    # of the prologue and attend stages is one launch of the split kernel that
    # makes its own query operands (query RoPE, absorption into U_K, the K
    # bias's LSE shift).  One rank's layers -- each with its own buffers, so the cache
    # holds none of them -- are captured back to back in one graph and timed
    # with HIP events over PROFILE_REPLAYS replays: the per-launch average
    # includes the hand-off between launches, as the kernel trace does, and no
    # per-launch event cost.  Beside it the attend stage alone over query
    # operands a prologue stage wrote beforehand (the three-launch form).
    from slimkv_amd._lib import STAGE_ATTEND, STAGE_PROLOGUE
    rows = kernels.query_rope_rows(cos, sin, step_pos)

    def timed_graph(body):
        body()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            body()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            body()
        for _ in range(3):
            g.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(PROFILE_REPLAYS):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e-3 / PROFILE_REPLAYS

    durations, staged = {}, {}
    for r in sorted(set(ranks)):
        group = [L for L in layers if L['rank'] == r]

        def fused_sweep():
            for L in group:
                run_layer(kernels, L, rows, scale, workspace, stages=STAGE_PROLOGUE | STAGE_ATTEND)
        durations[r] = [timed_graph(fused_sweep) / len(group)]
    stage_ws = [torch.empty(ws_bytes, dtype=torch.uint8, device=device) for _ in layers]
    for L, w in zip(layers, stage_ws):
        run_layer(kernels, L, rows, scale, w, stages=STAGE_PROLOGUE)
    torch.cuda.synchronize()
    for r in sorted(set(ranks)):
        group = [(L, w) for L, w in zip(layers, stage_ws) if L['rank'] == r]

        def attend_sweep():
            for L, w in group:
                run_layer(kernels, L, rows, scale, w, stages=STAGE_ATTEND)
        staged[r] = timed_graph(attend_sweep) / len(group)
    del stage_ws
    # The read rate a plain grid-stride stream reaches on this GPU (the
    # slimkv_probe_stream_read ceiling probe), to read the split kernel's rate
    # against beside the 8 TB/s peak.
    from bench_workloads import ceiling_probe, launch_floor_probe
    _, ceiling = ceiling_probe(torch, device)
    # what a launch and its hand-off cost with no work (the combine's grid)
    floor_us = launch_floor_probe(torch, device, workgroups=B * hq)
    dom = 32 if 32 in durations else max(durations, key=lambda r: len(durations[r]))
    dur = durations[dom]
    dur_avg = sum(dur) / len(dur)
    achieved = fused_kernel_bytes(dom, dom, hq, bias) / dur_avg / 1e9
    all_split = sum(sum(v) / len(v) * ranks.count(r) for r, v in durations.items())
    roofline = {'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBPS, 'unit': 'GB/s',
                'frac': round(achieved / HBM_PEAK_GBPS, 4),
                'traffic': (QWEN_SPLIT_TRAFFIC_BYTES if bias else SPLIT_TRAFFIC_BYTES).get(dom),
                'traffic_source': TRAFFIC_SOURCE,
                'kernel': f'split_kernel, query operands made in the kernel (rank-{dom} layers)',
                'avg_us': round(dur_avg * 1e6, 2),
                'split_kernel_sweep_frac': round(all_split / (elapsed / args.steps), 3),
                'ceiling': {'plain_gbps': ceiling['plain'], 'nt_gbps': ceiling['nt'],
                            'frac_of_plain': round(achieved / ceiling['plain'], 4),
                            'source': 'slimkv_probe_stream_read over 4 GiB, best configuration, same run'},
                'launch_floor_us': floor_us,
                'avg_us_by_rank': {str(r): round(sum(v) / len(v) * 1e6, 2) for r, v in sorted(durations.items())},
                'attend_stage_us_by_rank': {str(r): round(v * 1e6, 2) for r, v in sorted(staged.items())}}

    result = {
        'metric': shape['metric'], 'value': round(gbps, 1), 'unit': 'GB/s', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': round(ms_per_step, 4), 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16', 'data': 'synthetic',
        'config': {'workload': f"latent beacon decode, {len(layers)}-layer sweep, {shape['model']} layer shape t4f4"
                               + (', up-projection biases' if bias else ''),
                   'batch': B, 'context': CONTEXT, 'beacons': BEACONS, 'raw_tokens': RAW,
                   'q_heads': hq, 'kv_heads': HKV, 'head_dim': D, 'layer_ranks': ranks,
                   'graph': not args.no_graph},
        'hbm_frac': round(gbps / HBM_PEAK_GBPS, 4),
        'tokens_per_s': round(B / (elapsed / args.steps), 1),
        'us_per_layer': round(ms_per_step * 1e3 / len(layers), 2),
        'roofline': roofline,
        'replays': {'count': REPLAYS, 'median_ms': round(replay_ms, 4),
                    'median_gbps': round(sweep_bytes / (replay_ms * 1e-3) / 1e9, 1)},
        'clocks': gpu_clocks(),
        'library': _lib.library_identity(),
    }
    if not args.no_cpu:
        rank32 = next((L for L in layers if L['rank'] == 32), layers[0])
        print('bench: CPU baseline leg', file=sys.stderr, flush=True)
        result['cpu_baseline'] = cpu_baseline(torch, rank32, cos, sin, scale, hq, bias)
    print(json.dumps(result), flush=True)


if __name__ == '__main__':
    main()
