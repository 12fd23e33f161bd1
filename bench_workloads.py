"""The non-headline workloads of bench.py (`--workload prefill|recon|paged`).

prefill  Window-chunked prefill at batch 4: an 8192-token prompt in 8 windows of
         1024 raw tokens + 256 beacons (t4), 32 query / 8 KV heads, head_dim 128,
         4 sinks, per-head beacon rank 32.  A step runs every window: rebuild
         the history beacons' K/V (MFMA up-projection), compress the window's
         beacon rows (MFMA down-projection, per-head bases), causal flash
         attention over [sinks | history | window] (MFMA).  value = attention
         TFLOP/s over the whole step.
recon    Reconstruction decode, Qwen2.5-14B layer shape: batch 8, 40 query / 8 KV
         heads, 32K context at t4 (8192 beacons, rank 32 per head), 4 sinks +
         128 tail + current token, beacon K rotated at its slot position; 8
         layers with their own buffers.  value = algorithmic GB/s (latents,
         raw rows, q/out, weights once) over the step.
paged    Paged-cache decode: 64 sequences with contexts drawn in [1024, 131072],
         t8, BeaconPageLayout(16, 8, 256, 256, 1024) pages scattered over a
         400K-page pool, sinks + a tail of up to 255 raw tokens in raw pages.
         A step gathers the raw rows out of their pages and runs the fused
         latent decode reading the beacon rows straight from the pages
         (per-sequence lengths, splits over the total row count).  The
         restore path (gather every row, then decode) is timed beside it.
         value = algorithmic GB/s of the decode inputs.
"""
import os
import time

HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
_STAGE_PROLOGUE, _STAGE_ATTEND, _STAGE_ALL = 1, 2, 7      # SLIMKV_STAGE_* of include/slimkv_hip.h

# HBM bytes a launch of each workload's dominant kernel moves: two rocprofv3
# --pmc passes (FETCH_SIZE, then WRITE_SIZE, KiB a dispatch) over
# `bench.py --workload recon|paged --steps 1 --warmup 1 --no-cpu`, scaled as the
# latent decode's (FETCH_SIZE counts half the bytes read, WRITE_SIZE the bytes
# written, from the ceiling probe's transfers of known size).
RECON_TRAFFIC_BYTES = int((2 * 38_293.9 + 1_644.2) * 1024)      # recon_split_kernel<2, 1, 2>
PAGED_TRAFFIC_BYTES = int((2 * 321_411.8 + 10_669.7) * 1024)    # split_kernel<4, 8, 1, 0, 1>
TRAFFIC_SOURCE = ('rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this workload\'s kernel, scaled by the ceiling '
                  'probe\'s stream reads and fills')


def _events(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def _time_steps(torch, step, steps, warmup):
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def _timed_graph(torch, body, replays=20):
    """Seconds per run of `body` captured as one HIP graph and replayed back to
    back (HIP events around the replays): the kernels' own time at warm
    clocks, with no host launch gaps."""
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
    a, b = _events(torch)
    torch.cuda.synchronize()
    a.record()
    for _ in range(replays):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / replays


def _replays(torch, step, count=50):
    """Median of `count` single steps bracketed by HIP events, and the clocks."""
    from bench import gpu_clocks, replay_median_ms
    return {'count': count, 'median_ms': round(replay_median_ms(torch, step, count), 4)}, gpu_clocks()


def cpu_info():
    """Host CPU model and the threads this process may use."""
    model = None
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    model = line.split(':', 1)[1].strip()
                    break
    except OSError:
        pass
    return {'model': model, 'threads_available': len(os.sched_getaffinity(0))}


def _time_cpu(torch, fn, threads, budget_s):
    """Median seconds of `fn` at `threads` host threads: one warm-up, then at
    least 5 runs or until budget_s[0] seconds, at most budget_s[1]."""
    torch.set_num_threads(threads)
    fn()
    times = []
    start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        elapsed = time.perf_counter() - start
        if (elapsed >= budget_s[0] and len(times) >= 5) or elapsed >= budget_s[1]:
            break
    times.sort()
    return times[len(times) // 2], len(times), elapsed


def cpu_baseline(torch, fn, work, unit, scale, sample, budget_s=(8.0, 20.0)):
    """The reference's path restated on the host (the oracle's torch fp32
    port), timed at every available thread and at one thread (the reference
    CI's setting): value = work / median seconds / scale in `unit`."""
    threads = int(os.environ.get('OMP_NUM_THREADS', '0')) or len(os.sched_getaffinity(0))
    med, runs, elapsed = _time_cpu(torch, fn, threads, budget_s)
    med1, runs1, elapsed1 = _time_cpu(torch, fn, 1, (budget_s[0] / 2, budget_s[1] / 2))
    torch.set_num_threads(threads)
    return {'value': round(work / med / scale, 4), 'unit': unit, 'cores': threads, 'kind': 'port',
            'sample': f'{sample}; median of {runs} runs in {elapsed:.1f}s',
            'ms_per_run': round(med * 1e3, 2),
            'one_thread': {'value': round(work / med1 / scale, 4), 'cores': 1, 'ms_per_run': round(med1 * 1e3, 2),
                           'runs': runs1},
            'cpu': cpu_info()}


def staged_attend_seconds(torch, calls, stage_prologue, stage_attend, replays=20):
    """Per-launch seconds of the attend stage (the split-K kernel): every call's
    prologue stage runs once, then the attend stages of all calls -- each on
    its own buffers and workspace -- are captured back to back in one graph
    and timed with HIP events over `replays` replays."""
    for call in calls:
        call(stage_prologue)
    torch.cuda.synchronize()

    def sweep():
        for call in calls:
            call(stage_attend)
    sweep()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        sweep()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sweep()
    for _ in range(3):
        graph.replay()
    a, b = _events(torch)
    torch.cuda.synchronize()
    a.record()
    for _ in range(replays):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / (replays * len(calls))


def _result(metric, value, unit, args, seconds, dtype, config, **extra):
    out = {'metric': metric, 'value': round(value, 2), 'unit': unit, 'n_gpus': 1, 'steps': args.steps,
           'warmup': args.warmup, 'ms_per_step': round(seconds * 1e3, 4), 'higher_is_better': True,
           'scaling': 'weak', 'vs_baseline': None, 'dtype': dtype, 'data': 'synthetic', 'config': config}
    out.update(extra)
    return out


# ----------------------------------------------------------------------------- prefill

def prefill(args):
    """The window prefill step as prefill_forward runs it over a prefill
    history (slimkv_amd.prefill.PrefillHistory): per window the window's
    beacon rows are down-projected (K and V in one launch) and rebuilt as
    up(latent) in the projection's K/V rows (one launch), the prefill RoPE
    rotates the window's keys (beacon keys copied unrotated) into the store
    after the held keys and copies its values beside them (one launch), the
    causal attention rotates its queries as it loads them and runs over
    [sink | history | window], and the window's 256 new beacons are rebuilt
    onto the history (one launch).  The k/v projections of the window
    (nn.Linear layers of the model) stand as given rows, copied into the
    projections' output buffers each window."""
    import torch
    from slimkv_amd import kernels
    from slimkv_amd.workloads import block_diagonal, orthonormal_columns, rope_tables
    B, HQ, HKV, D, WIN, NB, S, r, WINDOWS = 4, 32, 8, 128, 1024, 256, 4, 32, 8
    L, R = WIN + NB, HKV * r
    dev = torch.device('cuda:0')
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    rnd = lambda *sh: torch.randn(*sh, generator=gen, device=dev).to(torch.bfloat16)
    cpu = torch.Generator().manual_seed(args.seed + 1)
    up = [block_diagonal([orthonormal_columns(D, r, cpu) for _ in range(HKV)]).to(dev, torch.bfloat16) for _ in range(2)]
    down = [block_diagonal([orthonormal_columns(D, r, cpu) for _ in range(HKV)]).t().contiguous().to(dev, torch.bfloat16)
            for _ in range(2)]                                  # per-head K_full[128] -> r bases [R, Hkv*D]
    n_max = S + NB * (WINDOWS - 1) + L
    work_k = torch.zeros(B, n_max, HKV, D, dtype=torch.bfloat16, device=dev)   # rotated keys as attended
    work_v = torch.zeros_like(work_k)
    proj_k = torch.zeros(B, L, HKV, D, dtype=torch.bfloat16, device=dev)      # the window's K projection
    proj_v = torch.zeros_like(proj_k)                                           # and its V projection
    latents = [torch.zeros(B, NB * WINDOWS, R, dtype=torch.bfloat16, device=dev) for _ in range(2)]
    qs = [rnd(B, L, HQ, D) for _ in range(WINDOWS)]
    cur = [(rnd(B, L, HKV, D), rnd(B, L, HKV, D)) for _ in range(WINDOWS)]
    roles = torch.zeros(L, dtype=torch.long, device=dev)
    roles[4::5] = 1                                             # one beacon after every 4 raw tokens
    beacon_rows = roles.nonzero().flatten()
    cos, sin = rope_tables(n_max, D, 500000.0, dev)
    positions = torch.arange(n_max, device=dev)[None].expand(B, -1)
    out = torch.empty(B, L, HQ, D, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, HQ, L, dtype=torch.float32, device=dev)
    scale = D ** -0.5

    def keys(w):
        return L if w == 0 else S + NB * w + L

    def attend(w):
        n = keys(w)
        base = 0 if w == 0 else S + NB * w
        kernels.prefill_attention(qs[w], work_k[:, :n], work_v[:, :n], scale, True, out=out, lse=lse,
                                  q_positions=positions[:, base:n], cos=cos, sin=sin)

    def window(w):
        n = keys(w)
        base = 0 if w == 0 else S + NB * w           # the window follows [sink | history]
        proj_k.copy_(cur[w][0])
        proj_v.copy_(cur[w][1])
        lats = [latents[j][:, NB * w:NB * (w + 1)] for j in (0, 1)]
        kernels.down_project_pair(*({'x': cur[w][j].view(B, L, HKV * D), 'weight': down[j], 'rows': beacon_rows,
                                     'blocks': HKV, 'out': lats[j]} for j in (0, 1)))
        kernels.reconstruct_pair(*({'latent': lats[j], 'weight': up[j], 'kv_heads': HKV, 'out': dst,
                                    'dst_rows': beacon_rows, 'block_diagonal': True}
                                   for j, dst in ((0, proj_k), (1, proj_v))))
        kernels.rope_keys(proj_k.transpose(1, 2), cos, sin, positions[:, base:n], roles, 0,
                          out_k=work_k[:, base:n].transpose(1, 2), v=proj_v.transpose(1, 2),
                          out_v=work_v[:, base:n].transpose(1, 2))
        attend(w)
        # the window's new beacons onto the history (after the sink of window 0)
        hist = S + NB * w
        kernels.reconstruct_pair(*({'latent': lats[j], 'weight': up[j], 'kv_heads': HKV,
                                    'out': dst[:, hist:hist + NB], 'block_diagonal': True}
                                   for j, dst in ((0, work_k), (1, work_v))))

    def step():
        for w in range(WINDOWS):
            window(w)

    seconds = _time_steps(torch, step, args.steps, args.warmup)
    replays, clocks = _replays(torch, step)
    pairs = [sum(min(keys(w), i + keys(w) - L + 1) for i in range(L)) for w in range(WINDOWS)]
    flops = [p * 4 * D * HQ * B for p in pairs]
    # the eight attention launches of a step alone, replayed back to back as
    # one graph (their cost does not depend on the values the buffers hold)
    attention_only = lambda: [attend(w) for w in range(WINDOWS)]
    if args.no_graph:                                 # counter runs: eager launches, events around them
        attention_only()
        a, b = _events(torch)
        torch.cuda.synchronize()
        a.record()
        attention_only()
        b.record()
        torch.cuda.synchronize()
        kernel_s = a.elapsed_time(b) * 1e-3
    else:
        kernel_s = _timed_graph(torch, attention_only)
    achieved = sum(flops) / kernel_s / 1e12
    result = _result('prefill attention TFLOP/s, 8 windows of 1024+256, b4, 32/8 heads', sum(flops) / seconds / 1e12,
                     'TFLOP/s', args, seconds, 'bf16',
                     {'workload': 'window prefill, 8192-token prompt, t4, per-head rank 32', 'batch': B,
                      'window': WIN, 'beacons_per_window': NB, 'windows': WINDOWS, 'q_heads': HQ, 'kv_heads': HKV,
                      'head_dim': D, 'sinks': S,
                      'step': 'window K/V projection outputs, beacon K/V down-projection and rebuild (one launch '
                              'each), prefill RoPE of the window keys into the kept key set with its values copied '
                              'beside them, attention (query RoPE inside), the 256 new beacons rebuilt onto an '
                              'append-only history'},
                     roofline={'bound': 'mfma', 'achieved': round(achieved, 1), 'peak': MFMA_BF16_PEAK_TFLOPS,
                               'unit': 'TFLOP/s', 'frac': round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                               'traffic': None, 'kernel': 'prefill_kernel', 'kernel_ms': round(kernel_s * 1e3, 3)},
                     attention_tflop=round(sum(flops) / 1e12, 4), replays=replays, clocks=clocks)
    # LDS reads of prefill_kernel: each of a workgroup's four waves reads the
    # whole 64-key K tile and V^T tile (2 x 64 x 128 x 2 B) per key tile it
    # attends, so a workgroup reads 128 KB a tile; tiles per workgroup follow
    # the causal visibility of its 128 query rows.
    lds = lds_probe(torch, dev)
    qblocks = (L + 127) // 128
    tiles = sum(sum(-(-min(keys(w), (i + 1) * 128 + keys(w) - L) // 64) for i in range(qblocks)) for w in range(WINDOWS))
    lds_bytes = tiles * B * HQ * 4 * 2 * 64 * D * 2
    cu = torch.cuda.get_device_properties(dev).multi_processor_count
    best_cu = max(lds['gbps_per_cu'].values())
    result['lds'] = dict(lds, kernel_bytes=lds_bytes, kernel_gbps_per_cu=round(lds_bytes / kernel_s / 1e9 / cu, 1),
                         bound_ms_at_probe_rate=round(lds_bytes / (best_cu * 1e9 * cu) * 1e3, 3))
    if not args.no_cpu:
        result['cpu_baseline'] = _prefill_cpu(torch, qs[1], work_k, work_v, keys(1), scale, pairs[1] * 4 * D * HQ * B)
    return result


def _prefill_cpu(torch, q, k, v, n, scale, flops):
    """Reference eager semantics in fp32 on the host for window 1 (torch
    restatement of the causal attention: 1280 queries over 1540 keys, b4,
    32/8 heads)."""
    qc = q.float().cpu().transpose(1, 2)                       # [B, H, L, D]
    kc = k[:, :n].float().cpu().transpose(1, 2)
    vc = v[:, :n].float().cpu().transpose(1, 2)
    g = qc.shape[1] // kc.shape[1]
    kc, vc = kc.repeat_interleave(g, 1), vc.repeat_interleave(g, 1)
    L = qc.shape[2]
    mask = torch.arange(n)[None, :] > (torch.arange(L)[:, None] + n - L)

    def run():
        s = (qc @ kc.transpose(-1, -2)) * scale
        s.masked_fill_(mask, float('-inf'))
        return torch.softmax(s, -1) @ vc
    return cpu_baseline(torch, run, flops, 'TFLOP/s', 1e12,
                        f'window 1 (1280 queries x {n} keys, b4, 32 heads), torch fp32 eager causal attention',
                        budget_s=(5.0, 15.0))


# ----------------------------------------------------------------------------- reconstruction decode

RECON_SHAPE = dict(B=8, HQ=40, HKV=8, D=128, NB=8192, S=4, T=128, r=32, CTX=32768)


def recon_layer(torch, dev, seed):
    """One reconstruction-decode layer at the Qwen2.5-14B shape (B8, 40/8
    heads, 8192 beacons of rank 32 per head, 4 sinks + 128 tail + current
    token); raw K stands in as already rotated."""
    from slimkv_amd.workloads import block_diagonal, orthonormal_columns
    c = RECON_SHAPE
    B, HQ, HKV, D, NB, r = c['B'], c['HQ'], c['HKV'], c['D'], c['NB'], c['r']
    RAW = c['S'] + c['T'] + 1
    gen = torch.Generator(device=dev).manual_seed(seed)
    rnd = lambda *sh: torch.randn(*sh, generator=gen, device=dev).to(torch.bfloat16)
    cpu = torch.Generator().manual_seed(seed + 50)
    return dict(
        q=rnd(B, 1, HQ, D), raw_k=rnd(B, RAW, HKV, D), raw_v=rnd(B, RAW, HKV, D),
        lat_k=rnd(B, NB, HKV * r), lat_v=rnd(B, NB, HKV * r),
        up_k=block_diagonal([orthonormal_columns(D, r, cpu) for _ in range(HKV)]).to(dev, torch.bfloat16),
        up_v=block_diagonal([orthonormal_columns(D, r, cpu) for _ in range(HKV)]).to(dev, torch.bfloat16),
        out=torch.empty(B, 1, HQ, D, dtype=torch.bfloat16, device=dev))


def recon_positions(torch, dev):
    """(query positions [B, 1], beacon slot positions [B, NB]) of the workload."""
    c = RECON_SHAPE
    qpos = torch.full((c['B'], 1), c['CTX'], dtype=torch.long, device=dev)
    bpos = (c['S'] + torch.arange(c['NB'], device=dev))[None].expand(c['B'], -1).contiguous()
    return qpos, bpos


def recon(args):
    import torch
    from slimkv_amd import kernels
    from slimkv_amd.workloads import rope_tables
    c = RECON_SHAPE
    B, HQ, HKV, D, NB, S, T, r, LAYERS = c['B'], c['HQ'], c['HKV'], c['D'], c['NB'], c['S'], c['T'], c['r'], 8
    R, RAW, CTX = HKV * r, S + T + 1, c['CTX']
    dev = torch.device('cuda:0')
    cos, sin = rope_tables(CTX + 1, D, 500000.0, dev)
    layers = [recon_layer(torch, dev, args.seed * 100 + i) for i in range(LAYERS)]
    qpos, bpos = recon_positions(torch, dev)
    scale = D ** -0.5

    def call(L, stages=_STAGE_ALL, workspace=None):
        kernels.recon_decode(L['q'], L['raw_k'], L['raw_v'], L['lat_k'], L['lat_v'], L['up_k'], L['up_v'],
                             scale, beacon_positions=bpos, block_diagonal=True, q_positions=qpos, cos=cos,
                             sin=sin, out=L['out'], stages=stages, workspace=workspace)

    def step():
        for L in layers:
            call(L)

    seconds = _time_steps(torch, step, args.steps, args.warmup)
    replays, clocks = _replays(torch, step)
    # The beacon K is rebuilt and rotated tile by tile inside the attention
    # kernel and V is lifted after the weighted sum, so HBM sees the latents
    # once; the reference's materialised K/V (write + read of both) would add
    # 4 * B * NB * HKV * D * 2 bytes per layer.
    per_layer = B * (NB * 2 * R * 2 + RAW * HKV * D * 2 * 2 + 2 * HQ * D * 2) + 2 * HKV * D * R * 2
    gbps = per_layer * LAYERS / seconds / 1e9
    # MFMA work of the split kernel per layer: the K rebuild (2 * 128 * r flops
    # per beacon per KV head), the scores (2 * 128 per beacon per query head)
    # and the latent P.V (2 * r per beacon per query head)
    rebuild_flop = B * NB * HKV * 2 * D * r
    attend_flop = B * NB * HQ * 2 * (D + r) + B * RAW * HQ * 4 * D
    # the split kernel reads the latents, the raw rows, q and U_K once
    split_bytes = B * (NB * 2 * R * 2 + RAW * HKV * D * 2 * 2 + HQ * D * 2) + HKV * D * R * 2
    ws = [torch.empty(64 << 20, dtype=torch.uint8, device=dev) for _ in layers]
    attend_s = staged_attend_seconds(torch, [lambda st, L=L, w=w: call(L, st, w) for L, w in zip(layers, ws)],
                                     _STAGE_PROLOGUE, _STAGE_ATTEND)
    del ws
    achieved = split_bytes / attend_s / 1e9
    mfma_tflops = (rebuild_flop + attend_flop) / attend_s / 1e12
    result = _result('reconstruction decode GB/s, Qwen2.5-14B layer shape b8 ctx32K t4', gbps, 'GB/s', args, seconds,
                     'bf16', {'workload': 'reconstruction decode, 8-layer sweep, 40/8 heads, rank 32, beacon K-RoPE, '
                                          'K rebuilt per tile in the attention kernel',
                              'batch': B, 'beacons': NB, 'raw_tokens': RAW},
                     hbm_frac=round(gbps / HBM_PEAK_GBPS, 4), us_per_layer=round(seconds / LAYERS * 1e6, 2),
                     bytes_per_layer=per_layer,
                     roofline={'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBPS, 'unit': 'GB/s',
                               'frac': round(achieved / HBM_PEAK_GBPS, 4), 'traffic': RECON_TRAFFIC_BYTES,
                               'traffic_source': TRAFFIC_SOURCE,
                               'kernel': 'recon_split_kernel (attend stage)', 'avg_us': round(attend_s * 1e6, 2),
                               'bytes_per_launch': split_bytes,
                               'mfma': {'achieved': round(mfma_tflops, 2), 'peak': MFMA_BF16_PEAK_TFLOPS,
                                        'unit': 'TFLOP/s', 'frac': round(mfma_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                                        'flop_per_launch': rebuild_flop + attend_flop}},
                     materialising_bytes_per_layer=per_layer + 4 * B * NB * HKV * D * 2, replays=replays,
                     clocks=clocks)
    if not args.no_cpu:
        result['cpu_baseline'] = _recon_cpu(torch, layers[0], cos, sin, qpos, bpos, scale, per_layer)
    return result


def _recon_cpu(torch, L, cos, sin, qpos, bpos, scale, per_layer):
    """The reference's reconstruction route (materialise K/V from the latents,
    RoPE the rebuilt K at its slot positions, fp32 softmax attention) in torch
    fp32 on the host, one full-shape layer (B8, 8192 beacons, 40/8 heads)."""
    from oracle import eager_torch
    c = RECON_SHAPE
    f = lambda x: x.float().cpu()
    p = int(qpos[0, 0])
    q = f(L['q']).transpose(1, 2)
    cq, sq = f(cos[p]), f(sin[p])
    q_rot = eager_torch.rotate(q, cq, sq)
    bp = bpos[0].cpu()
    cos_rows, sin_rows = f(cos[bp]), f(sin[bp])
    args = (q_rot, f(L['raw_k']), f(L['raw_v']), f(L['lat_k']), f(L['lat_v']), f(L['up_k']), f(L['up_v']), scale,
            c['HKV'], cos_rows, sin_rows)
    return cpu_baseline(torch, lambda: eager_torch.recon_layer(*args), per_layer, 'GB/s', 1e9,
                        'one full-shape layer (B8, 8192 beacons, 133 raw, 40/8 heads), torch fp32 reconstruction '
                        'route (rebuild, beacon K-RoPE, attention)')


# ----------------------------------------------------------------------------- paged decode

PAGED_SHAPE = dict(NSEQ=64, HQ=32, HKV=8, D=128, RATIO=8, S=4, r=32, POOL=400_000)


def paged_case(torch, dev, seed):
    """The paged workload's seeded draw: 64 sequences with contexts in
    [1024, 131072] and tails in [0, 255], t8 beacon pages
    BeaconPageLayout(16, 8, 256, 256, 1024) at a seeded random permutation of a
    400K-page pool, raw pages of 16 tokens for sinks + tail + current token."""
    import random
    from slimkv_amd.paged_cache import BeaconPageLayout
    from slimkv_amd.workloads import block_diagonal, orthonormal_columns
    c = PAGED_SHAPE
    NSEQ, HQ, HKV, D, RATIO, S, r, POOL = (c[k] for k in ('NSEQ', 'HQ', 'HKV', 'D', 'RATIO', 'S', 'r', 'POOL'))
    R = HKV * r
    rng = random.Random(seed)
    ctx = [rng.randint(1024, 131072) for _ in range(NSEQ)]
    tails = [rng.randint(0, 255) for _ in range(NSEQ)]
    nb = [x // RATIO for x in ctx]
    layout = BeaconPageLayout(16, RATIO, R, R, HKV * D)
    pool = torch.empty(POOL, layout.page_elements, dtype=torch.bfloat16, device=dev)
    gen = torch.Generator(device=dev).manual_seed(seed)
    for i in range(0, POOL, 50_000):
        pool[i:i + 50_000].normal_(generator=gen)
    pages_needed = [(n + layout.slots - 1) // layout.slots for n in nb]
    perm = torch.randperm(POOL, generator=torch.Generator().manual_seed(seed))
    width = max(pages_needed)
    tables = torch.full((NSEQ, width), 0, dtype=torch.long)
    off = 0
    for sidx, n in enumerate(pages_needed):
        tables[sidx, :n] = perm[off:off + n]
        off += n
    raw_count = [S + t + 1 for t in tails]                       # sinks + tail + current token
    raw_blocks = (max(raw_count) + 15) // 16
    raw_pool = torch.randn(NSEQ * raw_blocks, 16, 2, HKV, D, generator=gen, device=dev).to(torch.bfloat16)
    raw_tables = torch.randperm(NSEQ * raw_blocks, generator=torch.Generator().manual_seed(seed + 1))
    cpu = torch.Generator().manual_seed(seed + 2)
    up_k = block_diagonal([orthonormal_columns(D, r, cpu) for _ in range(HKV)]).to(dev, torch.bfloat16)
    up_v = block_diagonal([orthonormal_columns(D, r, cpu) for _ in range(HKV)]).to(dev, torch.bfloat16)
    q = torch.randn(NSEQ, 1, HQ, D, generator=gen, device=dev).to(torch.bfloat16)
    return dict(ctx=ctx, nb=nb, raw_count=raw_count, layout=layout, pool=pool, tables_cpu=tables,
                tables=tables.to(dev), raw_pool=raw_pool, raw_tables=raw_tables.view(NSEQ, raw_blocks).to(dev),
                lat_len=torch.tensor(nb, dtype=torch.int32, device=dev),
                raw_len=torch.tensor(raw_count, dtype=torch.int32, device=dev), up_k=up_k, up_v=up_v, q=q)


def paged(args):
    import torch
    from slimkv_amd import kernels
    from slimkv_amd.paged_cache import BeaconPages, RawPages
    c = PAGED_SHAPE
    NSEQ, HQ, HKV, D, RATIO, S, r, POOL = (c[k] for k in ('NSEQ', 'HQ', 'HKV', 'D', 'RATIO', 'S', 'r', 'POOL'))
    R = HKV * r
    dev = torch.device('cuda:0')
    pc = paged_case(torch, dev, args.seed)
    nb, raw_count, layout, pool, tables = pc['nb'], pc['raw_count'], pc['layout'], pc['pool'], pc['tables']
    raw_pool, raw_tables, lat_len, raw_len = pc['raw_pool'], pc['raw_tables'], pc['lat_len'], pc['raw_len']
    up_k, up_v, q = pc['up_k'], pc['up_v'], pc['q']
    beacons = BeaconPages(pool, layout)
    raw = RawPages(raw_pool)
    out = torch.empty(NSEQ, 1, HQ, D, dtype=torch.bfloat16, device=dev)
    scale = D ** -0.5
    max_nb, max_raw = max(nb), max(raw_count)
    lat_k = torch.zeros(NSEQ, max_nb, R, dtype=torch.bfloat16, device=dev)
    lat_v = torch.zeros_like(lat_k)
    raw_k = torch.zeros(NSEQ, HKV, max_raw, D, dtype=torch.bfloat16, device=dev)
    raw_v = torch.zeros_like(raw_k)
    # block-table index errors land here and are checked once after the timed
    # steps (the default per-call check would synchronise every step)
    status = torch.zeros(1, dtype=torch.int32, device=dev)

    def gather():
        beacons._move(tables, 0, lat_k, lat_v, False, lat_len, status)
        kernels.raw_pages(raw.pages, raw_tables, raw_k, raw_v, start=0, count=max_raw, to_pages=False,
                          lengths=raw_len, status=status)

    def decode():
        kernels.latent_decode(q, raw_k.transpose(1, 2), raw_v.transpose(1, 2), lat_k, lat_v, up_k, up_v, scale,
                              block_diagonal=True, raw_lengths=raw_len, lat_lengths=lat_len, out=out)

    def restore_step():
        gather()
        decode()

    def paged_call(stages=_STAGE_ALL, workspace=None):
        # beacon rows and raw rows (sinks, tail, current token) both read by
        # the decode through their block tables: no gather step
        kernels.paged_latent_decode(q, None, None, pool, tables, lat_len, max_nb, layout, up_k, up_v, scale,
                                    rows_total=sum(nb), block_diagonal=True, raw_lengths=raw_len, out=out,
                                    status=status, stages=stages, workspace=workspace, raw_pages=raw.pages,
                                    raw_tables=raw_tables, raw_keys=max_raw)

    def direct_step():
        paged_call()

    def raw_gather_step():
        # the raw rows gathered into a small dense buffer first
        kernels.raw_pages(raw.pages, raw_tables, raw_k, raw_v, start=0, count=max_raw, to_pages=False,
                          lengths=raw_len, status=status)
        kernels.paged_latent_decode(q, raw_k.transpose(1, 2), raw_v.transpose(1, 2), pool, tables, lat_len, max_nb,
                                    layout, up_k, up_v, scale, rows_total=sum(nb), block_diagonal=True,
                                    raw_lengths=raw_len, out=out, status=status)

    seconds = _time_steps(torch, direct_step, args.steps, args.warmup)
    replays, clocks = _replays(torch, direct_step)
    raw_gather_s = _time_steps(torch, raw_gather_step, args.steps, args.warmup)
    restore_s = _time_steps(torch, restore_step, args.steps, args.warmup)
    decode_s = _time_steps(torch, decode, args.steps, args.warmup)
    # the split kernel alone (attend stage): the pool (2.4 GB) is far larger
    # than the MALL, so back-to-back launches over it read HBM
    ws = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    attend_s = staged_attend_seconds(torch, [lambda st: paged_call(st, ws)] * 4, _STAGE_PROLOGUE, _STAGE_ATTEND)
    del ws
    kernels.check_status(status)
    # the access pattern's own ceiling: the beacon slots of every page the
    # decode reads (2 KB a page at its page offset), in table order
    ids = torch.cat([pc['tables_cpu'][b, :(n + layout.slots - 1) // layout.slots] for b, n in enumerate(nb)]).to(dev)
    gather = gather_probe(torch, pool, ids, pool.stride(0) * 2, layout.sink_elements * 2,
                          layout.slots * layout.width * 2)
    del ids
    algo = sum(n * 2 * R * 2 + c * HKV * D * 2 * 2 for n, c in zip(nb, raw_count)) + NSEQ * 2 * HQ * D * 2 \
        + 2 * HKV * D * R * 2
    split_bytes = sum(n * 2 * R * 2 + c * HKV * D * 2 * 2 for n, c in zip(nb, raw_count)) + NSEQ * HQ * D * 2 \
        + HKV * D * R * 2
    gbps = algo / seconds / 1e9
    achieved = split_bytes / attend_s / 1e9
    result = _result('paged latent decode GB/s, 64 seqs ctx U[1K,128K] t8', gbps, 'GB/s', args, seconds, 'bf16',
                     {'workload': 'paged decode: beacon and raw rows read from their pages by the fused latent '
                                  'decode, t8, rank 32',
                      'sequences': NSEQ, 'page_layout': [16, RATIO, R, R, HKV * D], 'pool_pages': POOL,
                      'beacons_total': sum(nb)},
                     hbm_frac=round(gbps / HBM_PEAK_GBPS, 4), bytes_per_step=algo,
                     roofline={'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBPS, 'unit': 'GB/s',
                               'frac': round(achieved / HBM_PEAK_GBPS, 4), 'traffic': PAGED_TRAFFIC_BYTES,
                               'traffic_source': TRAFFIC_SOURCE,
                               'kernel': 'split_kernel<KA,8,paged,0,raw pages> (attend stage)', 'avg_us': round(attend_s * 1e6, 2),
                               'bytes_per_launch': split_bytes,
                               'ceiling': {'gather_gbps': max(gather.values()), 'by_waves_per_cu': gather,
                                           'frac_of_gather': round(achieved / max(gather.values()), 4),
                                           'source': 'slimkv_probe_gather_read (libslimkv_probe.so): the 2 KB '
                                                     'beacon slots of every page the decode reads, in table order'}},
                     raw_gather_path_gbps=round(algo / raw_gather_s / 1e9, 1),
                     raw_gather_path_ms=round(raw_gather_s * 1e3, 4),
                     restore_path_gbps=round(algo / restore_s / 1e9, 1), restore_path_ms=round(restore_s * 1e3, 4),
                     dense_decode_only_gbps=round(algo / decode_s / 1e9, 1), replays=replays, clocks=clocks)
    if not args.no_cpu:
        result['cpu_baseline'] = _paged_cpu(torch, pc, raw_k, raw_v, scale)
    return result


def _paged_cpu(torch, pc, raw_k, raw_v, scale, sample=4):
    """restore_memory's gather (BeaconPages._indices + advanced indexing,
    paged_cache.py:60-73) and the eager latent decode (fa2_decode.py:143-164 in
    fp32) on the host, for the `sample` sequences of median length; their
    pages are copied to a host pool first (table entries renumbered)."""
    import numpy as np
    from oracle import eager_torch
    from oracle import paged as opaged
    c = PAGED_SHAPE
    layout = pc['layout']
    olayout = opaged.Layout(layout.raw_block_size, layout.token_ratio, layout.key_rank, layout.value_rank,
                            layout.raw_width)
    nb = pc['nb']
    order = sorted(range(len(nb)), key=lambda b: nb[b])
    picks = order[len(nb) // 2 - sample // 2:len(nb) // 2 - sample // 2 + sample]
    tables = pc['tables_cpu']
    seqs = []
    for b in picks:
        used = (nb[b] + layout.slots - 1) // layout.slots
        host_pool = pc['pool'][tables[b, :used].to(pc['pool'].device)].float().cpu()
        seqs.append((b, nb[b], host_pool, np.arange(used, dtype=np.int64)))
    up_k, up_v = pc['up_k'].float().cpu(), pc['up_v'].float().cpu()
    q = pc['q'].float().cpu().transpose(1, 2)                       # [B, H, 1, D]
    rk, rv = raw_k.float().cpu().transpose(1, 2), raw_v.float().cpu().transpose(1, 2)
    width = torch.arange(layout.width)

    def run():
        for b, n, host_pool, table in seqs:
            page, first = opaged.beacon_indices(olayout, table, 0, n)
            rows = host_pool[torch.from_numpy(page)[:, None], torch.from_numpy(first)[:, None] + width[None]]
            lk, lv = rows[:, :layout.key_rank], rows[:, layout.key_rank:]
            m = pc['raw_count'][b]
            eager_torch.latent_layer(q[b:b + 1], rk[b:b + 1, :m], rv[b:b + 1, :m], lk[None, :, None],
                                     lv[None, :, None], up_k, up_v, scale, c['HKV'])
    work = sum(n * 2 * layout.width + pc['raw_count'][b] * c['HKV'] * c['D'] * 2 * 2 for b, n, _, _ in seqs)
    return cpu_baseline(torch, run, work, 'GB/s', 1e9,
                        f'{sample} sequences of median length ({", ".join(str(nb[b]) for b in picks)} beacons): '
                        f'page gather + torch fp32 eager latent decode')


# ----------------------------------------------------------------------------- HBM ceiling

CEILING_CONFIGS = [(4, 8), (8, 4), (16, 1), (16, 2), (32, 1)]     # (resident waves per CU, loads in flight)


def ceiling_probe(torch, dev, gib=4, reps=10):
    """Read rate of slimkv_probe_stream_read over a `gib` GiB buffer (far past
    the 256 MB MALL) for each (waves per CU, loads in flight) configuration,
    plain and non-temporal loads: {config: GB/s} and the best of each kind."""
    import ctypes
    from slimkv_amd import _lib
    nbytes = gib << 30
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    # filled 256 MiB a launch: writes of a known size for scaling the
    # rocprofv3 WRITE_SIZE counter (as the stream reads scale FETCH_SIZE)
    for chunk in buf.split(256 << 20):
        chunk.fill_(1)
    cu = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.empty(cu * 64 * 64, dtype=torch.int32, device=dev)
    lib = _lib.probe_lib()
    stream = _lib.stream_handle(dev)
    rates = {}
    for nt in (0, 1):
        for waves, depth in CEILING_CONFIGS:
            def launch():
                _lib.probe_check(lib.slimkv_probe_stream_read(ctypes.c_void_p(buf.data_ptr()), nbytes,
                                                        ctypes.c_void_p(sink.data_ptr()), sink.numel(), waves,
                                                        depth, nt, stream))
            for _ in range(3):
                launch()
            a, b = _events(torch)
            a.record()
            for _ in range(reps):
                launch()
            b.record()
            torch.cuda.synchronize()
            rates[f"{'nt' if nt else 'plain'}_w{waves}_d{depth}"] = round(nbytes * reps / (a.elapsed_time(b) * 1e-3) / 1e9, 1)
    del buf
    best = {kind: max(v for k, v in rates.items() if k.startswith(kind)) for kind in ('plain', 'nt')}
    return rates, best


def gather_probe(torch, buf, ids, stride_bytes, offset_bytes, chunk_bytes, reps=10):
    """Read rate of slimkv_probe_gather_read over `buf` at the chunks `ids`
    (device int64), for 8 to 64 resident waves a CU: {config: GB/s}."""
    import ctypes
    from slimkv_amd import _lib
    dev = buf.device
    cu = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.empty(cu * 16 * 256, dtype=torch.int32, device=dev)
    lib, stream = _lib.probe_lib(), _lib.stream_handle(dev)
    nbytes = buf.numel() * buf.element_size()
    rates = {}
    for waves in (8, 16, 32, 64):
        def launch():
            _lib.probe_check(lib.slimkv_probe_gather_read(
                ctypes.c_void_p(buf.data_ptr()), nbytes, ctypes.c_void_p(ids.data_ptr()), ids.numel(), stride_bytes,
                offset_bytes, chunk_bytes, ctypes.c_void_p(sink.data_ptr()), sink.numel(), waves, stream))
        for _ in range(2):
            launch()
        a, b = _events(torch)
        a.record()
        for _ in range(reps):
            launch()
        b.record()
        torch.cuda.synchronize()
        rates[f'w{waves}'] = round(ids.numel() * chunk_bytes * reps / (a.elapsed_time(b) * 1e-3) / 1e9, 1)
    return rates


def launch_floor_probe(torch, dev, workgroups=512, launches=64):
    """Microseconds a launch of slimkv_probe_touch (`workgroups` one-wave
    workgroups, one store each) costs when `launches` of them are captured back
    to back in a graph: the dispatch-and-hand-off floor every launch of a
    decode layer pays.  512 workgroups is the batch-16 combine's grid."""
    import ctypes
    from slimkv_amd import _lib
    sink = torch.zeros(workgroups, dtype=torch.int32, device=dev)
    lib = _lib.probe_lib()

    def body():
        stream = _lib.stream_handle(dev)
        for _ in range(launches):
            _lib.probe_check(lib.slimkv_probe_touch(ctypes.c_void_p(sink.data_ptr()), sink.numel(), workgroups,
                                                    stream))
    return round(_timed_graph(torch, body) / launches * 1e6, 2)


def lds_probe(torch, dev, iters=256, reps=5):
    """LDS read rate of a CU (slimkv_probe_lds_read): 8- and 16-byte reads, one
    and two 256-thread workgroups a CU.  {config: GB/s a CU} and, at the shader
    clock the driver reports, bytes a clock a CU."""
    import ctypes
    from slimkv_amd import _lib
    cu = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.empty(cu * 2 * 256, dtype=torch.int32, device=dev)
    lib, stream = _lib.probe_lib(), _lib.stream_handle(dev)
    rates = {}
    for width in (8, 16):
        for wgs in (1, 2):
            def launch():
                _lib.probe_check(lib.slimkv_probe_lds_read(ctypes.c_void_p(sink.data_ptr()), sink.numel(), wgs,
                                                           iters, width, stream))
            launch()
            a, b = _events(torch)
            a.record()
            for _ in range(reps):
                launch()
            b.record()
            torch.cuda.synchronize()
            nbytes = cu * wgs * 256 * iters * 16 * width
            rates[f'b{8 * width}_wg{wgs}'] = round(nbytes * reps / (a.elapsed_time(b) * 1e-3) / 1e9 / cu, 1)
    clocks = _replays_clocks() or {}
    mhz = float(clocks['sclk'].rstrip('Mhz')) if clocks.get('sclk', '').rstrip('Mhz').isdigit() else None
    per_clk = {k: round(v * 1e9 / (mhz * 1e6), 1) for k, v in rates.items()} if mhz else None
    return {'gbps_per_cu': rates, 'bytes_per_clock_per_cu': per_clk, 'sclk_mhz': mhz,
            'source': 'slimkv_probe_lds_read (libslimkv_probe.so), conflict-free consecutive reads'}


def ceiling(args):
    """The HBM read ceiling of this GPU: a grid-stride stream of 16-byte loads
    (slimkv_probe_stream_read) over 4 GiB, the best of several resident-wave /
    loads-in-flight configurations, plain and non-temporal; the LDS read rate
    of a CU (slimkv_probe_lds_read); and the per-launch floor of a graph of
    back-to-back launches (slimkv_probe_touch)."""
    import torch
    dev = torch.device('cuda:0')
    t0 = time.perf_counter()
    rates, best = ceiling_probe(torch, dev)
    seconds = time.perf_counter() - t0
    return _result('HBM read ceiling GB/s (grid-stride stream, 4 GiB)', best['plain'], 'GB/s', args, seconds,
                   'u8', {'workload': 'stream read of a 4 GiB buffer, 16-byte loads',
                          'configs': [list(c) for c in CEILING_CONFIGS]},
                   hbm_frac=round(best['plain'] / HBM_PEAK_GBPS, 4), nt_gbps=best['nt'],
                   nt_frac=round(best['nt'] / HBM_PEAK_GBPS, 4), rates=rates, lds=lds_probe(torch, dev),
                   launch_floor_us=launch_floor_probe(torch, dev), clocks=_replays_clocks())


def _replays_clocks():
    from bench import gpu_clocks
    return gpu_clocks()


# ----------------------------------------------------------------------------- batch 1

# The reference's published attention GPU kernel time per token, 32 layers,
# batch 1, SlimKV t4f4 latent decode on H20 (README.md:276-280), by context.
REFERENCE_B1_MS = {32768: 4.81, 65536: 6.52, 98304: 8.10, 131072: 9.69, 262144: 16.03}
# ... and of its reconstruction decode (README.md:276-280, "Recon t4f4").
REFERENCE_B1_RECON_MS = {32768: 10.40, 65536: 17.30, 98304: 24.14, 131072: 31.27, 262144: 57.99}


def b1(args):
    """Batch-1 latent decode attention, 32 layers per token, at the contexts the
    reference publishes: ms per token (graph replay of the 32 layers' fused
    decode, own buffers per layer, RoPE rows gathered once per token)."""
    import torch
    import bench
    from slimkv_amd import kernels
    from slimkv_amd.workloads import block_diagonal, orthonormal_columns, rope_tables
    HQ, HKV, D, SINKS, TAIL, LAYERS = 32, 8, 128, 4, 128, 32
    dev = torch.device('cuda:0')
    ranks = bench.draw_ranks(LAYERS, args.seed)
    scale = D ** -0.5
    per_context = {}
    for ctx in sorted(REFERENCE_B1_MS):
        nb, raw = ctx // 4, SINKS + TAIL + 1
        cos, sin = rope_tables(ctx + 1, D, 500000.0, dev)
        layers = []
        for i, r in enumerate(ranks):
            gen = torch.Generator(device=dev).manual_seed(args.seed * 1000 + i)
            cpu = torch.Generator().manual_seed(args.seed * 1000 + i + 1)
            rnd = lambda *sh: torch.randn(*sh, generator=gen, device=dev).to(torch.bfloat16)
            layers.append(dict(
                q=rnd(1, 1, HQ, D), raw_k=rnd(1, raw, HKV, D), raw_v=rnd(1, raw, HKV, D),
                lat_k=rnd(1, nb, HKV * r), lat_v=rnd(1, nb, HKV * r),
                up_k=block_diagonal([orthonormal_columns(D, r, cpu) for _ in range(HKV)]).to(dev, torch.bfloat16),
                up_v=block_diagonal([orthonormal_columns(D, r, cpu) for _ in range(HKV)]).to(dev, torch.bfloat16),
                out=torch.empty(1, 1, HQ, D, dtype=torch.bfloat16, device=dev),
                lse=torch.empty(1, HQ, 1, dtype=torch.float32, device=dev)))
        pos = torch.full((1, 1), ctx, dtype=torch.int64, device=dev)
        ws = torch.empty(max(kernels.latent_decode_workspace_bytes(
            L['q'], L['raw_k'], L['raw_v'], L['lat_k'], L['lat_v'], L['up_k'], L['up_v'], block_diagonal=True,
            q_positions=pos, cos=cos, sin=sin) for L in layers), dtype=torch.uint8, device=dev)

        def token():
            rows = kernels.query_rope_rows(cos, sin, pos)
            for L in layers:
                kernels.latent_decode(L['q'], L['raw_k'], L['raw_v'], L['lat_k'], L['lat_v'], L['up_k'], L['up_v'],
                                      scale, block_diagonal=True, cos=rows[0], sin=rows[1], out=L['out'],
                                      lse=L['lse'], workspace=ws)
        token()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            token()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            token()
        seconds = _time_steps(torch, graph.replay, args.steps, args.warmup)
        replays, clocks = _replays(torch, graph.replay)
        ms = seconds * 1e3
        per_context[ctx] = {'ms_per_token': round(ms, 4), 'median_ms': replays['median_ms'],
                            'context_reference_h20_ms': REFERENCE_B1_MS[ctx]}
        del graph

        # The reference's per-token scope (README.md:284): the same 32 layers
        # with their QKV projection, the new token's K RoPE and its appends to
        # the raw cache (rotated K, plain K, V) -- one kernels.decode_qkv
        # launch over the concatenated q/k/v weights, as StaticDecode runs it --
        # the fused decode and the output projection (kernels.linear_rows); no
        # norm, MLP or LM head.  Weights are synthetic (Llama-3.1-8B shapes,
        # hidden 4096, q 4096, k/v 1024).
        hidden = HQ * D
        slot = torch.full((1,), raw - 1, dtype=torch.int64, device=dev)
        for i, L in enumerate(layers):
            gen = torch.Generator(device=dev).manual_seed(args.seed * 1000 + 700 + i)
            L['x'] = torch.randn(1, 1, hidden, generator=gen, device=dev).to(torch.bfloat16)
            L['w_qkv'] = (torch.randn(hidden + 2 * HKV * D, hidden, generator=gen, device=dev) * hidden ** -0.5
                          ).to(torch.bfloat16)
            L['w_o'] = (torch.randn(hidden, hidden, generator=gen, device=dev) * hidden ** -0.5).to(torch.bfloat16)
            L['plain_k'] = L['raw_k'].clone()
            L['q_new'] = torch.empty(1, hidden, dtype=torch.bfloat16, device=dev)
            L['o'] = torch.empty(1, hidden, dtype=torch.bfloat16, device=dev)
        token_pos = pos.view(1)
        status = torch.zeros(1, dtype=torch.int32, device=dev)     # slot errors, checked after the timing

        def full_token():
            rows = kernels.query_rope_rows(cos, sin, pos)
            for L in layers:
                q = kernels.decode_qkv(L['x'].view(1, hidden), L['w_qkv'], None, HQ, HKV, cos, sin, token_pos,
                                       L['raw_k'], L['raw_v'], slot, plain_k=L['plain_k'], q_out=L['q_new'],
                                       status=status)
                kernels.latent_decode(q.view(1, 1, HQ, D), L['raw_k'], L['raw_v'], L['lat_k'], L['lat_v'],
                                      L['up_k'], L['up_v'], scale, block_diagonal=True, cos=rows[0], sin=rows[1],
                                      out=L['out'], lse=L['lse'], workspace=ws)
                kernels.linear_rows(L['out'].view(1, hidden), L['w_o'], out=L['o'])
        full_token()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            full_token()
        torch.cuda.current_stream().wait_stream(side)
        full_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(full_graph):
            full_token()
        full_ms = _time_steps(torch, full_graph.replay, args.steps, args.warmup) * 1e3
        kernels.check_status(status)
        per_context[ctx]['readme_scope_ms_per_token'] = round(full_ms, 4)
        del layers, ws, full_graph
        torch.cuda.empty_cache()

        # Reconstruction decode of the same token: beacon K rebuilt and rotated
        # at the beacon slot positions inside the attention kernel, rank 32 in
        # every layer (the fused route's V ranks are 32 and 64).
        rec_layers = []
        for i in range(LAYERS):
            gen = torch.Generator(device=dev).manual_seed(args.seed * 1000 + 500 + i)
            cpu = torch.Generator().manual_seed(args.seed * 1000 + 501 + i)
            rnd = lambda *sh: torch.randn(*sh, generator=gen, device=dev).to(torch.bfloat16)
            rec_layers.append(dict(
                q=rnd(1, 1, HQ, D), raw_k=rnd(1, raw, HKV, D), raw_v=rnd(1, raw, HKV, D),
                lat_k=rnd(1, nb, HKV * 32), lat_v=rnd(1, nb, HKV * 32),
                up_k=block_diagonal([orthonormal_columns(D, 32, cpu) for _ in range(HKV)]).to(dev, torch.bfloat16),
                up_v=block_diagonal([orthonormal_columns(D, 32, cpu) for _ in range(HKV)]).to(dev, torch.bfloat16),
                out=torch.empty(1, 1, HQ, D, dtype=torch.bfloat16, device=dev)))
        bpos = (SINKS + torch.arange(nb, device=dev))[None].contiguous()

        def rec_token():
            for L in rec_layers:
                kernels.recon_decode(L['q'], L['raw_k'], L['raw_v'], L['lat_k'], L['lat_v'], L['up_k'], L['up_v'],
                                     scale, beacon_positions=bpos, block_diagonal=True, q_positions=pos, cos=cos,
                                     sin=sin, out=L['out'])
        rec_token()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            rec_token()
        torch.cuda.current_stream().wait_stream(side)
        rec_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(rec_graph):
            rec_token()
        rec_ms = _time_steps(torch, rec_graph.replay, args.steps, args.warmup) * 1e3
        per_context[ctx].update(recon_ms_per_token=round(rec_ms, 4),
                                context_reference_h20_recon_ms=REFERENCE_B1_RECON_MS[ctx])
        del rec_layers, rec_graph
        torch.cuda.empty_cache()
    first = per_context[32768]
    return _result('latent decode attention ms/token, 32 layers, B1, t4f4', first['ms_per_token'], 'ms', args,
                   first['ms_per_token'] * 1e-3, 'bf16',
                   {'workload': 'batch-1 latent beacon decode, 32 layers per token, Llama-3.1-8B layer shape, '
                                'per-layer rank drawn from {16, 32, 48}', 'contexts': sorted(REFERENCE_B1_MS),
                    'layer_ranks': ranks},
                   higher_is_better=False, vs_baseline=None,
                   per_context={str(k): v for k, v in per_context.items()},
                   readme_scope_ms_per_token=first['readme_scope_ms_per_token'],
                   context_reference_source='README.md:276-284, "Attention GPU kernel time" on an H20: per-token '
                                            'times including the QKV/O projections, cache operations and RoPE. '
                                            'readme_scope_ms_per_token times that scope here (value: the '
                                            'attention core alone); a different GPU, so context only',
                   clocks=clocks)


# ----------------------------------------------------------------------------- batched paged decode step

STEP_SHAPE = dict(NREQ=64, HIDDEN=4096, HQ=32, HKV=8, D=128, RATIO=8, WINDOW=1024, SINK=1, r=32)


class _RotaryTables:
    """Rotary module stand-in with the name the decode paths recognise."""
    def __init__(self, cos, sin):
        self.cos_cached, self.sin_cached = cos, sin
        self.max_seq_len_cached = cos.shape[0]


def paged_step(args):
    """One decode step of one Llama-3.1-8B attention layer (32/8 heads, t8,
    per-head rank 32, window 1024, one sink) for 64 vLLM requests whose
    contexts are drawn from [1024, 131072]: slimkv_amd.paged_step's
    paged_decode_layer over the requests' beacon pages (BeaconPageLayout(16, 8,
    256, 256, 1024)) and raw pages, the module's q/k/v/o and beacon
    projections included (random-init nn.Linear layers of the layer's
    shapes).  The step plan (plan_paged_step) is made once per decode step
    for all layers and is not timed.  Beside it the same layer runs once per
    request (groups of one), the shape of the reference's per-request loop
    (SlimKVLlamaForCausalLM._paged_forward, vllm_plugin/model.py:114-142)."""
    import random
    from types import SimpleNamespace
    import torch
    from slimkv_amd import kernels
    from slimkv_amd.paged_cache import BeaconPageLayout
    from slimkv_amd.paged_step import paged_decode_layer, plan_paged_step
    from slimkv_amd.workloads import block_diagonal, orthonormal_columns, rope_tables
    c = STEP_SHAPE
    NREQ, HID, HQ, HKV, D, RATIO, W, SINK, r = (c[k] for k in ('NREQ', 'HIDDEN', 'HQ', 'HKV', 'D', 'RATIO', 'WINDOW',
                                                               'SINK', 'r'))
    R = HKV * r
    dev = torch.device('cuda:0')
    rng = random.Random(args.seed)
    processed = [rng.randint(1024, 131072) for _ in range(NREQ)]
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    cpu = torch.Generator().manual_seed(args.seed + 1)

    def linear(i, o, weight=None):
        lin = torch.nn.Linear(i, o, bias=False, device=dev, dtype=torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_(weight if weight is not None else torch.randn(o, i, generator=gen, device=dev) / i ** 0.5)
        return lin

    cos, sin = rope_tables(max(processed) + 4096, D, 500000.0, dev)
    up = [block_diagonal([orthonormal_columns(D, r, cpu) for _ in range(HKV)]).to(dev, torch.bfloat16)
          for _ in range(2)]
    att = SimpleNamespace(
        config=SimpleNamespace(beacon_param=['q', 'k', 'v'], beacon_skip_rope_for_beacon_k=True),
        num_heads=HQ, num_key_value_heads=HKV, head_dim=D, hidden_size=HID,
        q_proj=linear(HID, HQ * D), k_proj=linear(HID, HKV * D), v_proj=linear(HID, HKV * D),
        beacon_q_proj=linear(HID, HQ * D), beacon_k_down_proj=linear(HID, R), beacon_v_down_proj=linear(HID, R),
        beacon_k_up_proj=linear(R, HKV * D, up[0]), beacon_v_up_proj=linear(R, HKV * D, up[1]),
        o_proj=linear(HQ * D, HID), rotary_emb=_RotaryTables(cos, sin))
    att._use_shared_kv_down_proj = lambda: False
    att.o_proj_with_beacon = lambda output, size, roles: att.o_proj(output)

    # beacon pages: each request's beacons (and the step's new one) on a permuted pool
    layout = BeaconPageLayout(16, RATIO, R, R, HKV * D)
    need = [(p // RATIO + 1 + layout.slots - 1) // layout.slots for p in processed]
    pool_pages = sum(need) + 64
    pool = torch.empty(pool_pages, layout.page_elements, dtype=torch.bfloat16, device=dev)
    for i in range(0, pool_pages, 50_000):
        pool[i:i + 50_000].normal_(generator=gen)
    perm = torch.randperm(pool_pages, generator=cpu)
    btables = torch.zeros(NREQ, max(need), dtype=torch.long)
    off = 0
    for i, n in enumerate(need):
        btables[i, :n] = perm[off:off + n]
        off += n
    # raw pages: blocks of the open window and the step's token; earlier
    # positions map to block 0, which the step neither reads nor writes
    cols = max((p + 1) // 16 + 1 for p in processed)
    win_blocks = [list(range((p - p % W) // 16, p // 16 + 1)) for p in processed]
    raw_blocks = 1 + sum(len(x) for x in win_blocks)
    raw_pool = torch.randn(raw_blocks, 16, 2, HKV, D, generator=gen, device=dev).to(torch.bfloat16)
    rtables = torch.zeros(NREQ, cols, dtype=torch.long)
    nxt = 1
    for i, blocks in enumerate(win_blocks):
        for blk in blocks:
            rtables[i, blk] = nxt
            nxt += 1
    btables, rtables = btables.to(dev), rtables.to(dev)
    groups = plan_paged_step(processed, W, RATIO, SINK, dev)
    hidden = {g.size: (0.5 * torch.randn(len(g.index), 1 + g.size, HID, generator=gen, device=dev)).to(torch.bfloat16)
              for g in groups}
    tables = {g.size: (rtables[g.tensors['index']], btables[g.tensors['index']]) for g in groups}
    status = torch.zeros(1, dtype=torch.int32, device=dev)

    def layer():
        with torch.no_grad():
            for g in groups:
                rt, bt = tables[g.size]
                paged_decode_layer(att, hidden[g.size], g, raw_pool, pool, rt, bt, 16, status=status)

    # the same layer one request at a time (groups of one)
    row_of = {i: (g.size, row) for g in groups for row, i in enumerate(g.index)}
    singles = []
    for i, p in enumerate(processed):
        (g1,) = plan_paged_step([p], W, RATIO, SINK, dev)
        size, row = row_of[i]
        singles.append((g1, hidden[size][row:row + 1], rtables[i:i + 1], btables[i:i + 1]))

    def per_request():
        with torch.no_grad():
            for g1, h1, rt, bt in singles:
                paged_decode_layer(att, h1, g1, raw_pool, pool, rt, bt, 16, status=status)

    seconds = _time_steps(torch, layer, args.steps, args.warmup)
    replays, clocks = _replays(torch, layer)
    graph_s = _timed_graph(torch, layer)          # the layer's GPU time without host launch gaps
    loop_s = _time_steps(torch, per_request, max(3, args.steps // 4), 1)
    kernels.check_status(status)
    weights = sum(x.weight.numel() for x in (att.q_proj, att.k_proj, att.v_proj, att.o_proj, att.beacon_k_up_proj,
                                             att.beacon_v_up_proj)) * 2
    inserting = [g for g in groups if g.size]
    if inserting:
        weights += sum(x.weight.numel() for x in (att.beacon_q_proj, att.beacon_k_down_proj,
                                                  att.beacon_v_down_proj)) * 2
    beacon_bytes = sum(g.rows_total for g in groups) * 2 * R * 2
    raw_bytes = sum((SINK + rc) * HKV * D * 2 * 2 for g in groups for rc in g.raw_counts)
    step_bytes = weights + beacon_bytes + raw_bytes
    tokens_per_s = NREQ / (32 * seconds)
    return _result('batched paged decode step, one Llama-3.1-8B attention layer, 64 requests ctx U[1K,128K] t8',
                   step_bytes / seconds / 1e9, 'GB/s', args, seconds, 'bf16',
                   {'workload': 'vLLM decode step of 64 paged requests through paged_decode_layer (projections, '
                                'page appends, raw gather and RoPE, paged latent decode, flush writes)',
                    'requests': NREQ, 'window': W, 'ratio': RATIO, 'sink': SINK, 'per_head_rank': r,
                    'groups': {str(g.size): len(g.index) for g in groups}, 'beacon_pool_pages': pool_pages},
                   hbm_frac=round(step_bytes / seconds / 1e9 / HBM_PEAK_GBPS, 4), bytes_per_step=step_bytes,
                   bytes_note='algorithmic: layer weights once, beacon latents and raw window rows of every request',
                   attention_layers_tokens_per_s=round(tokens_per_s, 1),
                   graph_replay_ms=round(graph_s * 1e3, 4),
                   graph_replay_gbps=round(step_bytes / graph_s / 1e9, 1),
                   per_request_loop_ms=round(loop_s * 1e3, 4),
                   batched_speedup=round(loop_s / seconds, 2), replays=replays, clocks=clocks)


def run_workload(args):
    from slimkv_amd._lib import library_identity
    result = {'prefill': prefill, 'recon': recon, 'paged': paged, 'paged_step': paged_step, 'b1': b1,
              'ceiling': ceiling}[args.workload](args)
    result['library'] = library_identity()
    return result
