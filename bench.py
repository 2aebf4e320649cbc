"""Benchmark of the fused NVFP4 sparse-attention decode on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload gqa_decode_b32] [--layers L] [--splits S]

A step is one layer-step of batched GQA sparse decode: batch 32, 32 query / 4 KV heads, head size 128, context
32768 per request, top-2048 sorted unique indices per request, NVFP4 paged KV (page 64, shuffled pages) built from
bf16 N(0,1) with 1% outlier channels x8. Exactly K layer-steps are timed: HIP graphs of L layer-steps, each on its own
layer's pool (distinct HBM, as the layers of a decode step, so the gathered rows come from HBM rather than from the
previous step's cache lines), replayed K // L times, plus one graph of the remaining K mod L steps. ms_per_step is
the event-timed mean over the K steps; `timing` gives the median and p10 / p90 over the full replays.

Prints one JSON line: value = achieved algorithmic HBM bandwidth (gathered KV payload + scales per step / step
time), plus the µs per layer-step, the roofline record, and the torch CPU restatement timed on the host's cores as a
reported baseline.
"""
import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = 'NVFP4-KV sparse-attn decode µs/layer-step + achieved HBM GB/s (% peak)'


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def emit(record):
    """Prints the record as one JSON line, with the GPU it ran on: name, architecture, compute units and the shader
    clock read right after the timed region (xt_clock_probe)."""
    import torch

    from xtier_amd import ops
    props = torch.cuda.get_device_properties(0)
    try:
        mhz = ops.clock_mhz()
    except Exception as e:  # noqa: BLE001 - the record is printed without the clock rather than not at all
        log(f'clock probe failed: {e}')
        mhz = None
    record['device'] = {'name': props.name, 'arch': getattr(props, 'gcnArchName', None),
                        'compute_units': props.multi_processor_count,
                        'shader_clock_mhz': None if mhz is None else round(mhz, 1),
                        'clock_read': 'core clock ticks over 100 MHz ticks while one wavefront runs, after the timed '
                                      'region'}
    print(json.dumps(record), flush=True)


def cpu_model():
    try:
        for line in open('/proc/cpuinfo'):
            if line.startswith('model name'):
                return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or 'unknown'


def cpu_threads():
    """Host threads for the CPU baseline: every core, capped by OMP_NUM_THREADS where the host sets it (a shared GPU
    box gives each GPU's jobs a share of its cores)."""
    n = os.cpu_count() or 1
    env = os.environ.get('OMP_NUM_THREADS')
    return max(1, min(n, int(env))) if env and env.isdigit() else n


def time_steps(step, layers, steps, warmup):
    """Times exactly `steps` layer-steps. After `warmup` eager steps, a graph of g layer-steps (layer l on its own
    pool) is replayed steps // g times and a graph of the remaining steps once, with HIP events on the launching stream
    around each replay. g = min(layers, max(8, steps // 5), steps): at least 8 pools when there are (a rotation of the
    decode workloads then gathers more than the 256 MB MALL holds, so no launch finds the previous replay's records
    there), and up to steps // 5, so that longer runs time at least five full replays. Returns (ms per layer-step over
    the whole timed region, per-layer-step µs of each full replay, g: the pools the timed region rotates)."""
    import torch
    g_len = max(1, min(layers, max(8, steps // 5), steps))
    for i in range(warmup):
        step(i % g_len)
    torch.cuda.synchronize()
    full, rest = divmod(steps, g_len)
    graphs = []
    for n in (g_len if full else 0, rest):
        g = None
        if n:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for layer in range(n):
                    step(layer)
            g.replay()   # the first replay of a graph is not timed
        graphs.append(g)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(full + 2)]
    ev[0].record()
    for i in range(full):
        graphs[0].replay()
        ev[i + 1].record()
    if graphs[1] is not None:
        graphs[1].replay()
    ev[-1].record()
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) * 1e3 / g_len for i in range(full)]
    return ev[0].elapsed_time(ev[-1]) / steps, per, g_len


def timeline_summary(stamps, waves, phases, loop_phase='main loop done'):
    """Phase times of one decode launch from its per-wave stamps (100 MHz ticks, rows g * waves + w): per phase the
    p10 / p50 / p90 / max over the waves that reached it, in µs from the earliest wave's entry; and the spread of the
    main loop's end within a workgroup (its last wave minus its first)."""
    import numpy as np
    st = np.asarray(stamps, dtype=np.int64)
    st = st[: (st.shape[0] // waves) * waves].reshape(-1, waves, len(phases))
    st = st[(st[:, :, 0] > 0).all(1)]
    t0 = st[:, :, 0].min()
    out = {'unit': 'µs from the first wave entry of the launch (100 MHz clock)', 'phases': {}}
    for i, name in enumerate(phases):
        if name.startswith('('):
            continue
        col = st[:, :, i].ravel()
        col = col[col > 0]
        if col.size == 0:
            continue
        rel = (col - t0) / 100.0
        out['phases'][name] = {'waves': int(col.size), 'p10': round(float(np.percentile(rel, 10)), 2),
                               'p50': round(float(np.percentile(rel, 50)), 2),
                               'p90': round(float(np.percentile(rel, 90)), 2), 'max': round(float(rel.max()), 2)}
    loop = st[:, :, list(phases).index(loop_phase)]
    ok = (loop > 0).all(1)
    if ok.any():
        d = (loop[ok].max(1) - loop[ok].min(1)) / 100.0
        out['main_loop_done_spread_within_workgroup'] = {'p50': round(float(np.percentile(d, 50)), 2),
                                                         'p90': round(float(np.percentile(d, 90)), 2)}
    return out


def spread(per_step_us, launches_per_replay):
    """Median and p10 / p90 of the per-layer-step times of the full replays."""
    import numpy as np
    if not per_step_us:
        return None
    a = np.asarray(per_step_us)
    return {'median_us': round(float(np.median(a)), 3), 'p10_us': round(float(np.percentile(a, 10)), 3),
            'p90_us': round(float(np.percentile(a, 90)), 3), 'replays': len(a),
            'launches_per_replay': launches_per_replay, 'unit': 'µs per layer-step, per graph replay'}


def build_layer(w, gen, layout, workloads, KVPool):
    """One layer's pool: K and V drawn as bf16 N(0,1) with 1% outlier channels x8, per-tensor global scales
    amax / 2688, quantized on the GPU into every slot."""
    import torch
    pool = KVPool(w.slots, w.kv_heads, w.dim, 'cuda', layout=layout)
    k = workloads.kv_tensor(w.slots, w.kv_heads, w.dim, gen, 'cuda')
    v = workloads.kv_tensor(w.slots, w.kv_heads, w.dim, gen, 'cuda')
    pool.set_global_scales(k, v)
    pool.append(k, v, torch.arange(w.slots, device='cuda'), saturate=False)
    return pool.raw


def cpu_baseline(raw, q, pt, idx, seq, w, scale, runs=20, warm=3):
    """The torch CPU restatement of the decode (oracle/torch_cpu.py: slots through the page table, NVFP4 dequant of
    the gathered rows, FP32 softmax attention), batched over the whole layer-step on the host's cores: 3 warm-ups,
    then the median of 20 runs."""
    import numpy as np
    import torch

    from oracle import torch_cpu

    threads = cpu_threads()
    torch.set_num_threads(threads)
    pool = tuple(t.cpu() for t in raw[:4]) + (raw[4].item(), raw[5].item())
    qf, pt_h, idx_h, seq_h = q.float().cpu(), pt.cpu(), idx.cpu(), seq.cpu()

    def run():
        slots = torch_cpu.slots_of(pt_h, w.page, idx_h, seq_h)
        return torch_cpu.sparse_decode(qf, pool, slots, scale)

    for _ in range(warm):
        run()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {'value': round(w.algorithmic_bytes() / med / 1e9, 4), 'unit': 'GB/s', 'cores': threads, 'kind': 'port',
            'us_per_layer_step': round(med * 1e6, 1), 'p10_us': round(float(np.percentile(times, 10)) * 1e6, 1),
            'p90_us': round(float(np.percentile(times, 90)) * 1e6, 1),
            'tokens_per_s': round(w.batch / med, 1),
            'sample': f'the whole layer-step ({w.batch} requests, full size): torch CPU restatement (page-table slots, '
                      f'NVFP4 dequant, FP32 softmax attention), {threads} threads of {os.cpu_count()} host cores '
                      f'({cpu_model()}), {warm} warm-ups, median of {runs}'}


def timed_sample(stage, run, total, seconds):
    """A bounded CPU sample on one thread: stage(rows) copies what rows need to the host (untimed), run(data) is the
    oracle's work on them. One row first, then as many rows (up to `total`) as fit in about `seconds`. Returns
    (rows timed, seconds)."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    with threadpool_limits(1):
        one = stage(np.array([0]))
        t0 = time.perf_counter()
        run(one)
        per_row = time.perf_counter() - t0
        n = int(max(1, min(total, seconds / max(per_row, 1e-6))))
        data = stage(np.arange(n))
        t0 = time.perf_counter()
        run(data)
        return n, time.perf_counter() - t0


def port_record(value, unit, n, total, what, oracle):
    return {'value': round(value, 6), 'unit': unit, 'cores': 1, 'kind': 'port',
            'sample': f'{n} of {total} {what} (oracle: {oracle}, one thread, {cpu_model()}, {os.cpu_count()} host '
                      'cores)'}


def compact_rows(device_tensors, slots):
    """Host copies of the rows `slots` (any shape) of each device tensor (BF16 ones as float32), and slots renumbered
    into them."""
    import numpy as np
    import torch
    uniq, inv = np.unique(np.asarray(slots), return_inverse=True)
    sel = torch.from_numpy(uniq.astype(np.int64)).cuda()
    host = []
    for t in device_tensors:
        r = t.index_select(0, sel)
        host.append((r.float() if r.dtype == torch.bfloat16 else r).cpu().numpy())
    return host, inv.reshape(np.shape(slots))


def measured_traffic(workload, splits, layout):
    """HBM bytes per launch of the decode kernel from the committed rocprofv3 counter summary (FETCH_SIZE and
    WRITE_SIZE, each scaled by the counter's reading for a copy of known size), when it was taken on this exact
    configuration; None otherwise."""
    path = ROOT / 'profiles' / f'decode_split_{workload}_traffic.json'
    try:
        rec = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    if rec.get('workload') != workload or rec.get('splits') != splits or rec.get('pool_layout') != layout:
        return None
    return rec.get('traffic_bytes')


MFMA_PEAK_TFLOPS = 2500.0   # dense FP16 / BF16


def run_prefill(args, w, ops, workloads, KVPool):
    """A step of chunked sparse prefill: quantize-on-append of the chunk's K and V rows into the pool, then the
    attention of every chunk query over its own causal top-k positions. One JSON line: attention TFLOP/s against the
    dense FP16 MFMA peak (the step's MFMA roofline), and the gathered-bytes rate."""
    import torch
    torch.cuda.set_device(0)
    gen = workloads.generator('cuda', 20261029)
    t0 = time.time()
    inp = workloads.prefill_inputs(w, 20261029, device='cuda')
    pool = KVPool(w.slots, w.kv_heads, w.dim, 'cuda', layout=args.layout)
    pool.set_global_scales(inp.k, inp.v)
    pos = torch.arange(w.ctx, device='cuda')
    slot_of = inp.page_table[0, pos // w.page].long() * w.page + pos % w.page
    pool.append(inp.k[:w.ctx0], inp.v[:w.ctx0], slot_of[:w.ctx0], saturate=False)
    k_new, v_new, new_slots = inp.k[w.ctx0:].contiguous(), inp.v[w.ctx0:].contiguous(), slot_of[w.ctx0:].contiguous()
    rows = w.chunk
    row_req = torch.zeros(rows, dtype=torch.int64, device='cuda')
    seq = torch.full((rows,), w.ctx, dtype=torch.int32, device='cuda')
    out = torch.empty(rows, w.q_heads, w.dim, dtype=torch.bfloat16, device='cuda')
    splits = args.splits or 1
    ws = ops.new_workspace('cuda', rows, w.q_heads, w.dim, splits)
    scale = 1.0 / math.sqrt(w.dim)
    del gen
    torch.cuda.synchronize()
    log(f'built the {w.ctx}-slot pool and {rows} causal index lists in {time.time() - t0:.1f} s')

    def step():
        pool.append(k_new, v_new, new_slots, saturate=False)
        ops.sparse_decode(inp.q, pool.raw, inp.page_table, inp.indices, seq, scale, page_size=w.page, row_req=row_req,
                          query_pos=inp.q_pos, out=out, splits=splits, ws=ws)

    steps = max(1, args.steps)
    ms, per, rot = time_steps(lambda layer: step(), 1, steps, max(1, args.warmup))
    tflops = w.flops() / (ms * 1e-3) / 1e12
    gbs = w.algorithmic_bytes() / (ms * 1e-3) / 1e9
    log(f'{w.name}: {ms * 1e3:.1f} us per step, {tflops:.1f} TFLOP/s ({tflops / MFMA_PEAK_TFLOPS:.1%} of '
        f'{MFMA_PEAK_TFLOPS:.0f}), gathered {gbs:.0f} GB/s')
    record = {
        'metric': 'NVFP4-KV sparse prefill attention TFLOP/s (chunk with quantize-on-append)', 'value': round(tflops, 2),
        'unit': 'TFLOP/s', 'n_gpus': 1, 'steps': steps, 'warmup': args.warmup, 'ms_per_step': round(ms, 6), 'timing': spread(per, rot),
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f16', 'data': 'synthetic',
        'config': {'workload': w.name, 'q_heads': w.q_heads, 'kv_heads': w.kv_heads, 'head_dim': w.dim,
                   'context': w.ctx0, 'chunk': w.chunk, 'topk': w.topk, 'recent': w.recent, 'page': w.page,
                   'kv_format': 'nvfp4', 'splits': splits, 'pool_layout': args.layout},
        'us_per_step': round(ms * 1e3, 2), 'gathered_gbs': round(gbs, 1),
        'roofline': {'bound': 'mfma', 'achieved': round(tflops, 2), 'peak': MFMA_PEAK_TFLOPS, 'unit': 'TFLOP/s',
                     'frac': round(tflops / MFMA_PEAK_TFLOPS, 4), 'traffic': None},
        'cpu_baseline': None if args.no_cpu_baseline else prefill_cpu(pool, inp, w, scale, args.cpu_seconds),
    }
    emit(record)


def prefill_cpu(pool, inp, w, scale, seconds):
    """The oracle's causal sparse attention (gather through the page table, NVFP4 dequant, FP32 softmax) on a sample
    of the chunk's query rows, after the step (the pool holds the chunk's rows)."""
    import numpy as np
    from oracle import attention
    pt = inp.page_table[0].cpu().numpy()
    idx, q_pos = inp.indices.cpu().numpy(), inp.q_pos.cpu().numpy()
    qf = inp.q.float().cpu().numpy()

    def stage(rows):
        pos = idx[rows]
        slots = pt[pos // w.page].astype(np.int64) * w.page + pos % w.page
        (k, v, ksf, vsf), inv = compact_rows(pool.raw[:4], slots)
        table = np.zeros((1, w.ctx), np.int32)
        table[0, pos] = inv
        host = (k, v, ksf, vsf, pool.raw[4].item(), pool.raw[5].item())
        return rows, host, table

    def run(data):
        rows, host, table = data
        attention.sparse_decode(qf[rows], host, table, 1, np.zeros(len(rows), np.int64), idx[rows], None,
                                np.full(len(rows), w.ctx), scale, query_pos=q_pos[rows], dtype=np.float32)

    n, dt = timed_sample(stage, run, w.chunk, seconds)
    flops = n * w.q_heads * w.topk * 4 * w.dim
    return port_record(flops / dt / 1e12, 'TFLOP/s', n, w.chunk, 'query rows of the chunk',
                       'numpy gather + NVFP4 dequant + FP32 causal softmax attention')


def build_latent_pool(w, seed, layout, workloads, LatentPool, chunk=1 << 20):
    """One layer's latent cache of w.slots tokens, generated in chunks of `chunk` rows (seed + chunk index each): a
    first pass takes the latent amax for g = amax / 2688, a second quantizes the rows into the pool."""
    import torch
    pool = LatentPool(w.slots, w.latent, w.rope, 'cuda', layout=layout)
    amax = torch.zeros((), device='cuda')
    starts = list(range(0, w.slots, chunk))
    for i, st in enumerate(starts):
        lat, _ = workloads.mla_cache_rows(w, workloads.generator('cuda', seed * 1000 + i), 'cuda', st,
                                          min(chunk, w.slots - st))
        amax = torch.maximum(amax, lat.abs().max().float())
    pool.g = torch.clamp(amax / 2688.0, min=1e-12).reshape(1).to(torch.float32)
    for i, st in enumerate(starts):
        n = min(chunk, w.slots - st)
        lat, rope = workloads.mla_cache_rows(w, workloads.generator('cuda', seed * 1000 + i), 'cuda', st, n)
        pool.append(lat, rope, torch.arange(st, st + n, device='cuda'), saturate=False)
    return pool


def run_mla(args, w, ops, workloads):
    """Sparse MLA steps (decode: one query per request; prefill: a causal chunk) over NVFP4 latent caches, rotating
    `layers` distinct caches for decode. One JSON line: TFLOP/s against the dense FP16 MFMA peak."""
    import torch
    from xtier_amd.pool import LatentPool
    torch.cuda.set_device(0)
    t0 = time.time()
    layers = 1 if w.causal else max(1, min(args.layers, 6))
    if w.fmt == 'fp8_v4':
        pools = [workloads.v4_pages(w.slots, w.page, workloads.generator('cuda', 17 + l), 'cuda') for l in range(layers)]
    else:
        pools = [build_latent_pool(w, 17 + l, args.layout, workloads, LatentPool) for l in range(layers)]
    inp = workloads.mla_inputs(w, 20261029, 'cuda')
    scale = 1.0 / math.sqrt(inp.q.shape[-1])
    splits = args.splits or ops.default_mla_splits(w.rows, w.topk, w.fmt == 'fp8_v4')
    ws = ops.workspace('cuda', ops.mla_workspace_bytes(w.rows, w.heads, splits, v4=w.fmt == 'fp8_v4'))
    out = torch.empty(w.rows, w.heads, 512, dtype=torch.bfloat16, device='cuda')
    lse = torch.empty(w.rows, w.heads, dtype=torch.float32, device='cuda')
    lengths = torch.full((w.rows,), w.topk, dtype=torch.int32, device='cuda') if args.mla_lengths else None
    torch.cuda.synchronize()
    log(f'built {layers} latent caches of {w.slots} tokens in {time.time() - t0:.1f} s')

    def step(layer):
        ops.sparse_mla(inp.q, pools[layer], inp.slots, lengths, None, scale, out=out, lse=lse, splits=splits, ws=ws)

    steps = max(1, args.steps)
    ms, per, rot = time_steps(step, layers, steps, max(1, args.warmup))
    tflops = w.flops() / (ms * 1e-3) / 1e12
    gbs = w.algorithmic_bytes() / (ms * 1e-3) / 1e9
    log(f'{w.name}: {ms * 1e3:.1f} us per step, {tflops:.1f} TFLOP/s ({tflops / MFMA_PEAK_TFLOPS:.1%} of '
        f'{MFMA_PEAK_TFLOPS:.0f}), {gbs:.0f} GB/s gathered, splits {splits}')
    timeline = None
    if args.timeline:   # one more launch (decode: on the cache used half a rotation ago) with the per-wave stamps
        units = w.rows * splits
        torch.cuda.synchronize()
        with ops.decode_timeline(units * 8, kind='mla') as tl:
            step(rot // 2)
        timeline = timeline_summary(tl.stamps, 8, ops.MLA_TIMELINE_PHASES)
        timeline['shape'] = {'waves_per_workgroup': 8, 'workgroups': units, 'splits': splits}
        log('timeline: ' + json.dumps(timeline))
    record = {
        'metric': 'NVFP4 sparse MLA attention TFLOP/s', 'value': round(tflops, 2), 'unit': 'TFLOP/s', 'n_gpus': 1,
        'steps': steps, 'warmup': args.warmup, 'ms_per_step': round(ms, 6), 'timing': spread(per, rot), 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16' if w.fmt == 'fp8_v4' else 'f16', 'data': 'synthetic',
        'config': {'workload': w.name, 'rows': w.rows, 'heads': w.heads, 'latent': w.latent, 'rope': w.rope,
                   'context': w.ctx, 'topk': w.topk, 'causal': w.causal,
                   'kv_format': 'fp8 v4 pages' if w.fmt == 'fp8_v4' else 'nvfp4 latent + bf16 rope',
                   'layers_rotated': rot, 'splits': splits, 'cache_layout': args.layout,
                   'list_lengths': bool(args.mla_lengths)},
        'us_per_step': round(ms * 1e3, 2), 'gathered_gbs': round(gbs, 1),
        'roofline': {'bound': 'mfma', 'achieved': round(tflops, 2), 'peak': MFMA_PEAK_TFLOPS, 'unit': 'TFLOP/s',
                     'frac': round(tflops / MFMA_PEAK_TFLOPS, 4), 'traffic': None},
        'cpu_baseline': None if args.no_cpu_baseline else mla_cpu(pools[0], inp, w, scale, args.cpu_seconds),
    }
    if timeline is not None:
        record['timeline'] = timeline
    emit(record)


def mla_cpu(cache, inp, w, scale, seconds):
    """The oracle's sparse MLA (key decoding from the cache bytes, FP32 softmax over the row's keys) on a sample of
    rows: the NVFP4 latent + rope cache, or the V4 FP8 pages."""
    import numpy as np
    import torch
    from oracle import attention
    slots = inp.slots.cpu().numpy()
    qf = inp.q.float().cpu().numpy()
    v4 = w.fmt == 'fp8_v4'
    if v4:
        stride = w.page * 584
        flat = torch.as_strided(cache, (cache.shape[0] * stride,), (1,))

    def stage(rows):
        tok = slots[rows]
        if not v4:
            (pay, sc, rope), inv = compact_rows((cache.pay, cache.scales, cache.rope), tok)
            return rows, (pay, sc, rope, np.float32(cache.g.item())), inv
        uniq, inv = np.unique(tok, return_inverse=True)
        t = torch.from_numpy(uniq.astype(np.int64)).cuda()
        base = (t // w.page) * stride
        row = t % w.page
        data = flat[(base + row * 576)[:, None] + torch.arange(576, device='cuda')[None, :]]
        sc = flat[(base + w.page * 576 + row * 8)[:, None] + torch.arange(8, device='cuda')[None, :]]
        return rows, torch.cat([data, sc], 1).cpu().numpy(), inv.reshape(tok.shape)

    def run(data):
        rows, cache_h, inv = data
        if v4:
            keys = attention.v4_keys(cache_h.reshape(-1), 1, 584, tokens=cache_h.shape[0])
            attention.sparse_mla_v4(qf[rows], keys, inv, None, None, scale)
        else:
            attention.sparse_mla(qf[rows], *cache_h, inv, None, None, scale, dtype=np.float32)

    n, dt = timed_sample(stage, run, w.rows, seconds)
    flops = w.flops() / w.rows * n
    what = 'numpy V4 FP8 page decoding + FP64' if v4 else 'numpy NVFP4 latent dequant + FP32'
    return port_record(flops / dt / 1e12, 'TFLOP/s', n, w.rows, 'rows', what + " softmax attention over the row's keys")


def build_block_pool(w, gen, workloads, ops):
    """One layer's head-major NVFP4 pages (unit global scale) from bf16 K/V of w.batch * w.ctx tokens."""
    import torch
    slots = w.batch * w.ctx
    one = torch.ones(1, dtype=torch.float32, device='cuda')
    out = []
    for _ in range(2):
        x = workloads.kv_tensor(slots, w.kv_heads, w.dim, gen, 'cuda')
        pay = torch.empty(slots, w.kv_heads, w.dim // 2, dtype=torch.uint8, device='cuda')
        sc = torch.empty(slots, w.kv_heads, w.dim // 16, dtype=torch.uint8, device='cuda')
        ops.quantize_append(x, torch.arange(slots, device='cuda'), one, pay, sc)
        del x
        out += list(workloads.head_major_pages(pay, sc, w.block))
    return out   # k_pay, k_sc, v_pay, v_sc


def run_block(args, w, ops, workloads):
    """Block-sparse decode steps over head-major NVFP4 pages (MiniMax layout), rotating `layers` distinct pools.
    One JSON line: GB/s of read KV bytes against the HBM peak."""
    import torch
    torch.cuda.set_device(0)
    t0 = time.time()
    gen = workloads.generator('cuda', 20261103)
    layers = max(1, min(args.layers, 8))
    pools = [build_block_pool(w, gen, workloads, ops) for _ in range(layers)]
    inp = workloads.block_decode_inputs(w, 20261104, 'cuda')
    splits = args.splits or ops.default_splits(w.batch, w.kv_heads, w.keys, False)
    ws = ops.new_workspace('cuda', w.batch, w.q_heads, w.dim, splits)
    out = torch.empty(w.batch, w.q_heads, w.dim, dtype=torch.bfloat16, device='cuda')
    torch.cuda.synchronize()
    log(f'built {layers} page pools ({w.pages} pages each) in {time.time() - t0:.1f} s')

    def step(layer):
        k_pay, k_sc, v_pay, v_sc = pools[layer]
        ops.fp4_sparse_decode(inp.q, k_pay, k_sc, v_pay, v_sc, inp.req_to_token, inp.slot_ids, inp.topk_idx,
                              inp.seq_lens, w.block, out=out, splits=splits, ws=ws)

    steps = max(1, args.steps)
    ms, per, rot = time_steps(step, layers, steps, max(1, args.warmup))
    gbs = w.algorithmic_bytes() / (ms * 1e-3) / 1e9
    log(f'{w.name}: {ms * 1e3:.2f} us per layer-step, {gbs:.0f} GB/s algorithmic ({gbs / HBM_PEAK_GBS:.1%} of '
        f'{HBM_PEAK_GBS:.0f}), splits {splits}')
    timeline = None
    if args.timeline:   # one launch on the pool used half a rotation ago, as for the token-index decode
        hpw, waves, units = ops.decode_shape(w.batch, w.kv_heads, splits, w.dim, shared_lists=False)
        torch.cuda.synchronize()
        with ops.decode_timeline(units * waves) as tl:
            step(rot // 2)
        timeline = timeline_summary(tl.stamps, waves, ops.TIMELINE_PHASES)
        timeline['shape'] = {'kv_heads_per_workgroup': hpw, 'waves_per_workgroup': waves, 'workgroups': units}
        log('timeline: ' + json.dumps(timeline))
    record = {
        'metric': 'NVFP4-KV block-sparse decode HBM GB/s', 'value': round(gbs, 1), 'unit': 'GB/s', 'n_gpus': 1,
        'steps': steps, 'warmup': args.warmup, 'ms_per_step': round(ms, 6), 'timing': spread(per, rot), 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f16', 'data': 'synthetic',
        'config': {'workload': w.name, 'batch': w.batch, 'q_heads': w.q_heads, 'kv_heads': w.kv_heads,
                   'head_dim': w.dim, 'context': w.ctx, 'topk_blocks': w.topk_blocks, 'block': w.block,
                   'kv_format': 'nvfp4 head-major pages', 'layers_rotated': rot, 'splits': splits},
        'us_per_layer_step': round(ms * 1e3, 3), 'tokens_per_s': round(w.batch / (ms * 1e-3), 1),
        'roofline': {'bound': 'hbm', 'achieved': round(gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': round(gbs / HBM_PEAK_GBS, 4), 'traffic': None},
        'cpu_baseline': None if args.no_cpu_baseline else block_cpu(pools[0], inp, w, args.cpu_seconds),
    }
    if timeline is not None:
        record['timeline'] = timeline
    emit(record)


def block_cpu(pool, inp, w, seconds):
    """The oracle's block-sparse decode (per KV head: the listed blocks' NVFP4 rows dequantized, FP32 softmax) on a
    sample of the requests of one layer-step."""
    import numpy as np
    from oracle import attention
    host = [t.cpu().numpy() for t in pool]          # k_pay, k_sc, v_pay, v_sc pages
    r2t, sid = inp.req_to_token.cpu().numpy(), inp.slot_ids.cpu().numpy()
    idx, seq = inp.topk_idx.cpu().numpy(), inp.seq_lens.cpu().numpy()
    qf = inp.q.float().cpu().numpy()
    f32 = lambda q, k, v, valid, sc: attention.softmax_attention(q, k, v, valid, sc, np.float32)

    def run(rows):
        attention.block_sparse_decode(qf[rows], *host, r2t, sid[rows], idx[:, rows], seq[rows], w.block,
                                      w.dim ** -0.5, attend=f32)

    n, dt = timed_sample(lambda rows: rows, run, w.batch, seconds)
    nbytes = w.algorithmic_bytes() / w.batch * n
    return port_record(nbytes / dt / 1e9, 'GB/s', n, w.batch, 'requests of one layer-step',
                       'numpy NVFP4 block dequant + FP32 softmax attention per KV head')


def run_block_prefill(args, w, ops, workloads):
    """Causal block-sparse prefill chunks over head-major NVFP4 pages (MiniMax layout), rotating `layers` distinct
    pools; also times the BF16 context copy (main K, V and index K) the prefill entry makes for contexts that fit.
    One JSON line: TFLOP/s of the attention against the MFMA peak."""
    import torch
    torch.cuda.set_device(0)
    t0 = time.time()
    gen = workloads.generator('cuda', 20261201)
    layers = max(1, min(args.layers, 8))
    shape = workloads.BlockDecodeWorkload(w.name, 1, w.q_heads, w.kv_heads, w.dim, w.ctx, w.topk_blocks, w.block)
    pools = [build_block_pool(shape, gen, workloads, ops) for _ in range(layers)]
    ik = build_block_pool(workloads.BlockDecodeWorkload(w.name, 1, 1, 1, w.dim, w.ctx, 1, w.block), gen, workloads,
                          ops)[:2]
    ik = [t[:, 0] for t in ik]
    inp = workloads.block_prefill_inputs(w, 20261202, 'cuda')
    splits = args.splits or ops.default_splits(w.q_len, w.kv_heads, w.topk_blocks * w.block, False)
    ws = ops.new_workspace('cuda', w.q_len, w.q_heads, w.dim, splits)
    out = torch.empty_like(inp.q)
    rows = -(-w.ctx // 128) * 128
    copies = [torch.empty(rows, w.kv_heads, w.dim, dtype=torch.bfloat16, device='cuda') for _ in range(2)]
    copies.append(torch.empty(rows, 1, w.dim, dtype=torch.bfloat16, device='cuda'))
    torch.cuda.synchronize()
    log(f'built {layers} page pools ({w.pages} pages each) in {time.time() - t0:.1f} s')

    def step(layer):
        k_pay, k_sc, v_pay, v_sc = pools[layer]
        ops.fp4_prefill_gqa_share_sparse(inp.q, k_pay, v_pay, None, inp.req_to_token, inp.slot_ids, inp.topk_idx, 1,
                                         w.block, inp.cu_seqlens, inp.seq_lens, inp.prefix_lens, w.q_len, k_sc=k_sc,
                                         v_sc=v_sc, out=out, splits=splits, ws=ws)

    def copy(layer):
        k_pay, k_sc, v_pay, v_sc = pools[layer]
        for (pay, sc), dst in zip(((k_pay, k_sc), (v_pay, v_sc), ik), copies):
            ops.dequantize_context(pay, sc, inp.req_to_token, inp.slot_ids, inp.seq_lens, rows, out=dst)

    steps = max(1, args.steps)
    ms, per, rot = time_steps(step, layers, steps, max(1, args.warmup))
    copy_ms, _, _ = time_steps(copy, layers, steps, max(1, args.warmup))
    tflops = w.flops() / (ms * 1e-3) / 1e12
    gbs = w.algorithmic_bytes() / (ms * 1e-3) / 1e9
    copy_gbs = w.copy_bytes() / (copy_ms * 1e-3) / 1e9
    log(f'{w.name}: {ms * 1e3:.1f} us per chunk, {tflops:.1f} TFLOP/s ({tflops / MFMA_PEAK_TFLOPS:.1%} of '
        f'{MFMA_PEAK_TFLOPS:.0f}), {gbs:.0f} GB/s of listed KV, splits {splits}; context copy {copy_ms * 1e3:.1f} us '
        f'= {copy_gbs:.0f} GB/s ({copy_gbs / HBM_PEAK_GBS:.1%})')
    record = {
        'metric': 'NVFP4-KV block-sparse prefill TFLOP/s', 'value': round(tflops, 2), 'unit': 'TFLOP/s',
        'n_gpus': 1, 'steps': steps, 'warmup': args.warmup, 'ms_per_step': round(ms, 6), 'timing': spread(per, rot), 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f16', 'data': 'synthetic',
        'config': {'workload': w.name, 'q_len': w.q_len, 'prefix': w.prefix, 'q_heads': w.q_heads,
                   'kv_heads': w.kv_heads, 'head_dim': w.dim, 'topk_blocks': w.topk_blocks, 'block': w.block,
                   'block_size_q': 1, 'kv_format': 'nvfp4 head-major pages', 'layers_rotated': rot,
                   'splits': splits},
        'us_per_chunk': round(ms * 1e3, 2), 'listed_kv_gbs': round(gbs, 1),
        'context_copy': {'us': round(copy_ms * 1e3, 2), 'bytes': w.copy_bytes(), 'gbs': round(copy_gbs, 1),
                         'frac_hbm': round(copy_gbs / HBM_PEAK_GBS, 4)},
        'roofline': {'bound': 'mfma', 'achieved': round(tflops, 2), 'peak': MFMA_PEAK_TFLOPS, 'unit': 'TFLOP/s',
                     'frac': round(tflops / MFMA_PEAK_TFLOPS, 4), 'traffic': None},
        'cpu_baseline': None if args.no_cpu_baseline else block_prefill_cpu(pools[0], inp, w, args.cpu_seconds),
    }
    emit(record)


def block_prefill_cpu(pool, inp, w, seconds):
    """The oracle's causal block-sparse prefill (per-token slot lookups, NVFP4 dequant, FP32 softmax) on a sample of
    the chunk's query rows."""
    import numpy as np
    from oracle import attention
    host = [t.cpu().numpy() for t in pool]
    r2t = inp.req_to_token.cpu().numpy()
    idx = inp.topk_idx.cpu().numpy()
    qf = inp.q.float().cpu().numpy()
    f32 = lambda q, k, v, valid, sc: attention.softmax_attention(q, k, v, valid, sc, np.float32)

    def run(rows):
        n = len(rows)
        one = np.arange(n + 1)
        attention.block_sparse_prefill(qf[rows], *host, r2t, np.zeros(n, np.int64), idx[:, rows], one, one,
                                       np.full(n, w.ctx), w.prefix + rows, 1, w.block, w.dim ** -0.5, attend=f32)

    n, dt = timed_sample(lambda rows: rows, run, w.q_len, seconds)
    flops = w.flops() / w.q_len * n
    return port_record(flops / dt / 1e12, 'TFLOP/s', n, w.q_len, 'query rows of the chunk',
                       'numpy per-token slot lookup + NVFP4 dequant + FP32 causal softmax attention')


GATHER_WORKLOADS = {
    # the decode workload's rows (batch 32, 4 KV heads x 128, context 32768, top-2048, page 64) gathered into BF16
    'qsa_gather_b32': ('gather', 32, 32768, 2048),
    # one request's 65536-token prefix packed into BF16 rows (4 KV heads x 128)
    'qsa_pack_ctx65536': ('pack', 1, 65536, 65536),
}


def run_gather(args, name, ops, workloads, KVPool):
    """The QSA gather (decode rows through the page table) or prefix pack into BF16 rows, rotating `layers` pools of
    SGLang's four buffers. One JSON line: GB/s of pool bytes read plus BF16 rows written against the HBM peak."""
    import torch
    mode, batch, ctx, topk = GATHER_WORKLOADS[name]
    kv_heads, dim, page = 4, 128, 64
    torch.cuda.set_device(0)
    gen = workloads.generator('cuda', 20261203)
    layers = max(1, min(args.layers, 4))
    w = workloads.DecodeWorkload(name, batch, 32, kv_heads, dim, ctx, topk, page)
    t0 = time.time()
    pools = [build_layer(w, gen, 'split', workloads, KVPool) for _ in range(layers)]
    r2t = workloads.token_table(workloads.page_table(batch, ctx, page, gen, 'cuda'), page)
    req = torch.arange(batch, dtype=torch.int64, device='cuda')
    cu = (torch.arange(batch + 1, dtype=torch.int32, device='cuda') * topk)
    seq = torch.full((batch,), ctx, dtype=torch.int32, device='cuda')
    idx = workloads.index_lists(batch, ctx, topk, gen, 'cuda') if mode == 'gather' else None
    out_k = torch.empty(batch * topk, kv_heads, dim, dtype=torch.bfloat16, device='cuda')
    out_v = torch.empty_like(out_k)
    torch.cuda.synchronize()
    log(f'built {layers} pools ({w.slots} slots each) in {time.time() - t0:.1f} s')

    def step(layer):
        if mode == 'gather':
            ops.gather(pools[layer], r2t, req, idx, seq, cu, out_k, out_v, batch, topk)
        else:
            ops.pack(pools[layer], r2t, req, cu, batch * topk, topk, torch.bfloat16)

    steps = max(1, args.steps)
    ms, per, rot = time_steps(step, layers, steps, max(1, args.warmup))
    rows = batch * topk * kv_heads
    nbytes = rows * 2 * (dim // 2 + dim // 16) + rows * 2 * dim * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f'{name}: {ms * 1e3:.2f} us per layer-step, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of {HBM_PEAK_GBS:.0f})')
    record = {
        'metric': f'NVFP4-KV {mode} into BF16 rows HBM GB/s', 'value': round(gbs, 1), 'unit': 'GB/s', 'n_gpus': 1,
        'steps': steps, 'warmup': args.warmup, 'ms_per_step': round(ms, 6), 'timing': spread(per, rot), 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16', 'data': 'synthetic',
        'config': {'workload': name, 'batch': batch, 'kv_heads': kv_heads, 'head_dim': dim, 'context': ctx,
                   'rows_per_request': topk, 'page': page, 'kv_format': 'nvfp4 (SGLang buffers)',
                   'layers_rotated': rot},
        'us_per_layer_step': round(ms * 1e3, 3), 'bytes_per_step': nbytes,
        'roofline': {'bound': 'hbm', 'achieved': round(gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': round(gbs / HBM_PEAK_GBS, 4), 'traffic': None},
        'cpu_baseline': None if args.no_cpu_baseline else gather_cpu(mode, pools[0], r2t, idx, w, args.cpu_seconds),
    }
    emit(record)


def gather_cpu(mode, raw, r2t, idx, w, seconds):
    """The oracle's gather (decode rows) or pack (a prefix) into BF16 rows on a sample: requests of the decode
    workload, or the first positions of the prefix."""
    import numpy as np
    from oracle import attention
    r2t_h = r2t.cpu().numpy()
    per_row = w.kv_heads * (2 * (w.dim // 2 + w.dim // 16) + 2 * w.dim * 2)   # bytes per (request column, all heads)
    if mode == 'gather':
        idx_h = idx.cpu().numpy()

        def stage(rows):
            pos = idx_h[rows]
            (k, v, ksf, vsf), inv = compact_rows(raw[:4], r2t_h[rows[:, None], pos])
            table = np.zeros((len(rows), w.ctx), np.int32)
            table[np.arange(len(rows))[:, None], pos] = inv
            return rows, (k, v, ksf, vsf, raw[4].item(), raw[5].item()), table

        def run(data):
            rows, host, table = data
            n = len(rows)
            out = np.zeros((n * w.topk, w.kv_heads, w.dim), np.uint16)
            attention.gather_qsa(host, table, np.arange(n), idx_h[rows], np.full(n, w.ctx),
                                 np.arange(n + 1) * w.topk, out, out.copy(), n, w.topk)

        n, dt = timed_sample(stage, run, w.batch, seconds)
        return port_record(n * w.topk * per_row / dt / 1e9, 'GB/s', n, w.batch, 'requests',
                           'numpy NVFP4 dequant into BF16 rows')
    chunk = 512

    def stage(rows):
        m = len(rows) * chunk
        (k, v, ksf, vsf), inv = compact_rows(raw[:4], r2t_h[0, :m])
        return m, (k, v, ksf, vsf, raw[4].item(), raw[5].item()), inv[None, :].astype(np.int32)

    def run(data):
        m, host, table = data
        attention.pack_qsa(host, table, np.zeros(1, np.int64), np.array([0, m]), m)

    n, dt = timed_sample(stage, run, w.ctx // chunk, seconds)
    return port_record(n * chunk * per_row / dt / 1e9, 'GB/s', n * chunk, w.ctx, 'positions of the prefix',
                       'numpy NVFP4 dequant into BF16 rows')


def run_varlen(args, w, ops, workloads):
    """Split-K decode over packed BF16 rows, rotating `layers` distinct K/V buffers. One JSON line: GB/s of K/V rows
    read against the HBM peak."""
    import torch
    torch.cuda.set_device(0)
    gen = workloads.generator('cuda', 20261105)
    layers = max(1, min(args.layers, 16))
    n = w.rows * w.keys
    kv = [(workloads.kv_tensor(n, w.kv_heads, w.dim, gen, 'cuda'), workloads.kv_tensor(n, w.kv_heads, w.dim, gen, 'cuda'))
          for _ in range(layers)]
    q = torch.randn(w.rows, w.q_heads, w.dim, generator=gen, device='cuda').to(torch.bfloat16)
    cu_q = torch.arange(w.rows + 1, dtype=torch.int32, device='cuda')
    cu_k = cu_q * w.keys
    splits = args.splits or ops.varlen_splits(w.rows, w.kv_heads, w.q_heads // w.kv_heads, w.keys)
    ws = torch.zeros(ops.varlen_workspace_bytes(w.rows, w.q_heads, w.dim, splits), dtype=torch.uint8, device='cuda')
    out = torch.empty_like(q)
    scale = w.dim ** -0.5

    def step(layer):
        ops.varlen_decode(q, kv[layer][0], kv[layer][1], cu_q, cu_k, 1, w.keys, scale, out=out, splits=splits, ws=ws)

    steps = max(1, args.steps)
    ms, per, rot = time_steps(step, layers, steps, max(1, args.warmup))
    gbs = w.algorithmic_bytes() / (ms * 1e-3) / 1e9
    log(f'{w.name}: {ms * 1e3:.2f} us per layer-step, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of {HBM_PEAK_GBS:.0f}), '
        f'splits {splits}')
    record = {
        'metric': 'BF16 varlen split-K decode HBM GB/s', 'value': round(gbs, 1), 'unit': 'GB/s', 'n_gpus': 1,
        'steps': steps, 'warmup': args.warmup, 'ms_per_step': round(ms, 6), 'timing': spread(per, rot), 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16', 'data': 'synthetic',
        'config': {'workload': w.name, 'rows': w.rows, 'q_heads': w.q_heads, 'kv_heads': w.kv_heads,
                   'head_dim': w.dim, 'keys_per_row': w.keys, 'kv_format': 'bf16 packed rows',
                   'layers_rotated': rot, 'splits': splits},
        'us_per_layer_step': round(ms * 1e3, 3),
        'roofline': {'bound': 'hbm', 'achieved': round(gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': round(gbs / HBM_PEAK_GBS, 4), 'traffic': None},
        'cpu_baseline': None if args.no_cpu_baseline else varlen_cpu(q, kv[0], w, scale, args.cpu_seconds),
    }
    emit(record)


def varlen_cpu(q, kv, w, scale, seconds):
    """The oracle's split-K decode over packed BF16 rows (128-key partials, FP64 merge) on a sample of rows."""
    import numpy as np
    from oracle import attention
    qf = q.float().cpu().numpy()

    def stage(rows):
        n = len(rows)
        k, v = (t[:n * w.keys].float().cpu().numpy() for t in kv)
        return rows, k, v

    def run(data):
        rows, k, v = data
        n = len(rows)
        attention.varlen_decode(qf[rows], k, v, np.arange(n + 1), np.arange(n + 1) * w.keys, scale)

    n, dt = timed_sample(stage, run, w.rows, seconds)
    return port_record(w.algorithmic_bytes() / w.rows * n / dt / 1e9, 'GB/s', n, w.rows, 'rows',
                       'numpy split-K softmax attention with FP64 merge')


INDEXER_WORKLOADS = {
    # QSA indexer prefill logits deep in a 380K prompt: 352 rows x 95088 compressed keys, 4 heads x 128, BF16 (the
    # first case of the reference's tests/qsa_prefill_check.py:25-53; 2.40 -> 0.61 ms on an RTX PRO 5000,
    # docs/reports/2026-10-23-prefill.md:48-53)
    'qsa_logits_352x95088': dict(kind='qsa', rows=352, heads=4, dim=128, prefix=380000, ratio=4),
    # DSA indexer prefill logits: 4096 queries x 16384 keys, 32 heads x 128, FP8 E4M3 with FP32 key scales and head
    # weights (the shapes of the reference's tests/glm_indexer_torch_check.py:27-43, at prefill size)
    'dsa_logits_4096x16384': dict(kind='dsa', num_q=4096, heads=32, dim=128, num_kv=16384),
    # top-2048 selection over the QSA case's logits (352 rows x 95088 columns)
    'topk_352x95088_k2048': dict(kind='topk', rows=352, cols=95088, topk=2048),
    # MiniMax decode index scores: batch 32, context 32768, 4 index heads x 128 over the NVFP4 index pool, blocks of
    # 128 (the shapes of tests/minimax_kv_fp4_check.py:29, :81-108 at batch 32)
    'minimax_decode_scores_b32': dict(kind='mm_decode', batch=32, ctx=32768, heads=4, dim=128, block=128),
    # MiniMax prefill index scores: one 8192-token prompt, 4 index heads x 128, blocks of 128
    'minimax_prefill_scores_8k': dict(kind='mm_prefill', ext=8192, heads=4, dim=128, block=128),
}


def run_indexer(args, name, ops):
    """The top-k producers: the QSA and DSA indexer logits, the top-k selection and the MiniMax index block scores,
    each timed over exactly K launches (HIP graphs), against the bound its algorithmic bytes or flops set."""
    import numpy as np
    import torch

    from oracle import topk as ref

    torch.cuda.set_device(0)
    cfg = INDEXER_WORKLOADS[name]
    kind = cfg['kind']
    gen = torch.Generator(device='cuda').manual_seed(20261023)
    seconds = args.cpu_seconds

    def bf16(*shape, std=1.0):
        return (torch.randn(*shape, device='cuda', generator=gen) * std).bfloat16()

    if kind == 'qsa':
        rows, heads, dim = cfg['rows'], cfg['heads'], cfg['dim']
        keys = (cfg['prefix'] + rows) // cfg['ratio']
        q, k = bf16(rows, heads, dim), bf16(keys, 1, dim)
        # one key buffer per launch of a graph replay (8 x 24 MB, with the 134 MB of logits written between two reads
        # of one of them), so the keys come from HBM, not from the 256 MB MALL
        kcopies = [k] + [k.clone() for _ in range(7)]
        starts = torch.zeros(rows, dtype=torch.int32, device='cuda')
        ends = ((torch.arange(cfg['prefix'], cfg['prefix'] + rows, device='cuda') + 1) // cfg['ratio']).int()
        out = torch.empty(rows, keys, device='cuda')
        lib = ops._lib.lib()

        def step(layer):
            kl = kcopies[layer % len(kcopies)]
            ops._lib.check(lib.xt_qsa_indexer_logits(q.data_ptr(), q.stride(0), q.stride(1), rows, heads, dim,
                                                     kl.data_ptr(), kl.stride(0), keys, starts.data_ptr(),
                                                     ends.data_ptr(), math.sqrt(dim), ops._lib.XT_DTYPE_BF16,
                                                     out.data_ptr(), out.stride(0),
                                                     torch.cuda.current_stream().cuda_stream), 'qsa')
        nbytes = q.numel() * 2 + k.numel() * 2 + rows * keys * 4 + rows * 8
        flops = 2 * rows * heads * keys * dim
        conf = {'rows': rows, 'keys': keys, 'heads': heads, 'dim': dim, 'dtype': 'bf16'}
        qh, kh, eh = q.float().cpu().numpy(), k[:, 0].float().cpu().numpy(), ends.cpu().numpy()

        def cpu(n):
            ref.qsa_indexer_logits(qh[:n], kh, np.zeros(n, np.int64), eh[:n])
        cpu_total, cpu_unit = rows, 'rows'
    elif kind == 'dsa':
        nq, heads, dim, nkv = cfg['num_q'], cfg['heads'], cfg['dim'], cfg['num_kv']
        q = (torch.randn(nq, heads, dim, device='cuda', generator=gen) * 2).to(torch.float8_e4m3fn)
        k = (torch.randn(nkv, dim, device='cuda', generator=gen) * 2).to(torch.float8_e4m3fn)
        ksc = torch.rand(nkv, device='cuda', generator=gen) + 0.5
        w = torch.randn(nq, heads, device='cuda', generator=gen)
        ks = torch.zeros(nq, dtype=torch.int32, device='cuda')
        ke = torch.full((nq,), nkv, dtype=torch.int32, device='cuda')

        def step(_):
            ops.dsa_mqa_logits(q, (k, ksc), w, ks, ke)
        ld = (nkv + 3) // 4 * 4
        nbytes = q.numel() + k.numel() + nkv * 4 + w.numel() * 4 + nq * ld * 4
        flops = 2 * nq * heads * nkv * dim
        conf = {'num_q': nq, 'num_kv': nkv, 'heads': heads, 'dim': dim, 'dtype': 'e4m3'}
        qh, kh, kch, wh = q.float().cpu().numpy(), k.float().cpu().numpy(), ksc.cpu().numpy(), w.cpu().numpy()

        def cpu(n):
            ref.dsa_mqa_logits(qh[:n], kh, kch, wh[:n], np.zeros(n, np.int64), np.full(n, nkv))
        cpu_total, cpu_unit = nq, 'queries'
    elif kind == 'topk':
        rows, cols, kk = cfg['rows'], cfg['cols'], cfg['topk']
        x = torch.randn(rows, cols, device='cuda', generator=gen)
        # three inputs of 134 MB in turn: two others (268 MB, more than the 256 MB MALL) are read between two reads of
        # one, so each launch reads its input from HBM
        xs = [x] + [torch.randn(rows, cols, device='cuda', generator=gen) for _ in range(2)]
        out = torch.empty(rows, kk, dtype=torch.int32, device='cuda')

        def step(layer):
            ops.topk_rows(xs[layer % len(xs)], kk, out=out)
        nbytes = rows * cols * 4 + rows * kk * 4
        flops = 0
        conf = {'rows': rows, 'cols': cols, 'topk': kk, 'dtype': 'f32'}
        xh = x.cpu().numpy()

        def cpu(n):
            ref.topk_rows(xh[:n], kk)
        cpu_total, cpu_unit = rows, 'rows'
    else:
        page = 128
        heads, dim, bs = cfg['heads'], cfg['dim'], cfg['block']
        if kind == 'mm_decode':
            batch, ctx = cfg['batch'], cfg['ctx']
            lens, pre, ext = [ctx] * batch, [0] * batch, None
        else:
            batch, ext = 1, [cfg['ext']]
            lens, pre = ext, [0]
        blocks = [-(-n // page) for n in lens]
        pages = sum(blocks) + 1
        perm = torch.randperm(pages - 1, device='cuda', generator=gen) + 1
        width = max(blocks) * page
        r2t = torch.zeros(batch, width, dtype=torch.int32, device='cuda')
        off = 0
        for r, n in enumerate(blocks):
            pg = perm[off:off + n].int()
            r2t[r, :n * page] = (pg[:, None] * page + torch.arange(page, device='cuda', dtype=torch.int32)).view(-1)
            off += n
        # decode: 4 index pools (320 MB together, more than the 256 MB MALL), rotated over the launches of a graph
        npools = 4 if kind == 'mm_decode' else 1
        pays = [torch.randint(0, 256, (pages, page, dim // 2), device='cuda', generator=gen, dtype=torch.uint8)
                for _ in range(npools)]
        scs = [torch.randint(0x28, 0x40, (pages, page, dim // 16), device='cuda', generator=gen, dtype=torch.uint8)
               for _ in range(npools)]
        pay, sc = pays[0], scs[0]
        seq = torch.tensor(lens, dtype=torch.int32, device='cuda')
        sid = torch.arange(batch, dtype=torch.int32, device='cuda')
        nblk = -(-max(lens) // bs)
        if kind == 'mm_decode':
            q = bf16(batch, heads, dim)
            score = torch.empty(heads, batch, nblk, device='cuda')

            def step(layer):
                ops.minimax_decode_scores(q, pays[layer % npools], scs[layer % npools], r2t, score, seq, sid, bs,
                                          dim ** -0.5, 1.0, 0, 1)
            keys = sum(lens)
            nbytes = keys * (dim // 2 + dim // 16 + 4) + q.numel() * 2 + score.numel() * 4
            flops = 2 * keys * heads * dim
            conf = {'batch': batch, 'context': ctx, 'heads': heads, 'dim': dim, 'block': bs, 'dtype': 'bf16'}

            def cpu(n):
                ref.minimax_block_scores_decode(qh[:n], payh, sch, r2th, np.arange(n), lens[:n], bs, dim ** -0.5,
                                                1.0, 0, 1)
            cpu_total, cpu_unit = batch, 'requests'
        else:
            total = ext[0]
            q = bf16(total, heads, dim)
            score = torch.empty(heads, total, nblk, device='cuda')
            cu = torch.tensor([0, total], dtype=torch.int32, device='cuda')
            pre_t = torch.zeros(1, dtype=torch.int32, device='cuda')

            def step(_):
                ops.minimax_prefill_scores(q, pay, sc, r2t, score, cu, seq, pre_t, sid, bs, dim ** -0.5, 1.0, total)
            # the keys each row's 64-row tile visits, every head
            visited = sum(min(total, 64 * (t // 64 + 1)) for t in range(total))
            nbytes = total * heads * dim * 2 + sum(lens) * (dim // 2 + dim // 16 + 4) + total * heads * nblk * 4
            flops = 2 * visited * heads * dim
            conf = {'prompt': total, 'heads': heads, 'dim': dim, 'block': bs, 'dtype': 'bf16'}

            def cpu(n):
                # the prompt's last n rows (prefix total - n), each against its causal keys
                ref.minimax_block_scores_prefill(qh[total - n:], payh, sch, r2th, [0], [0, n], [total], [total - n],
                                                 bs, dim ** -0.5, 1.0)

            def cpu_work(n):
                # keys visited by the last n rows, as a fraction of the whole prompt's
                return sum(min(total, total - n + 64 * (t // 64 + 1)) for t in range(n)) / visited
            cpu_total, cpu_unit = total, 'prompt rows (the last ones, scaled by the keys they visit)'
        qh, payh, sch, r2th = q.float().cpu().numpy(), pay.cpu().numpy(), sc.cpu().numpy(), r2t.cpu().numpy()
    # 8 launches per graph replay (a replay of one short launch would time the graph launch); the HBM-bound ones rotate
    # their inputs (QSA keys, top-k rows, decode-score pools) so that no launch reads its input from the MALL
    steps = max(1, args.steps)
    ms, per, rot = time_steps(step, 8, steps, max(1, args.warmup))
    t = ms * 1e-3
    gbs, tflops = nbytes / t / 1e9, flops / t / 1e12
    t_hbm, t_mfma = nbytes / (HBM_PEAK_GBS * 1e9), flops / (MFMA_PEAK_TFLOPS * 1e12)
    bound = 'mfma' if t_mfma > t_hbm else 'hbm'
    if bound == 'mfma':
        roof = {'bound': 'mfma', 'achieved': round(tflops, 1), 'peak': MFMA_PEAK_TFLOPS, 'unit': 'TFLOP/s',
                'frac': round(tflops / MFMA_PEAK_TFLOPS, 4), 'traffic': None}
    else:
        roof = {'bound': 'hbm', 'achieved': round(gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                'frac': round(gbs / HBM_PEAK_GBS, 4), 'traffic': None}
    log(f'{name}: {ms * 1e3:.1f} us per launch, {gbs:.0f} GB/s, {tflops:.1f} TFLOP/s ({bound}-bound, '
        f'{roof["frac"]:.1%} of peak)')
    # CPU baseline: the oracle on a bounded prefix of the rows, one thread
    from threadpoolctl import threadpool_limits
    with threadpool_limits(1):
        t0 = time.perf_counter()
        cpu(1)
        one = time.perf_counter() - t0
        n = int(max(1, min(cpu_total, seconds / max(one, 1e-6))))
        t0 = time.perf_counter()
        cpu(n)
        dt = time.perf_counter() - t0
    frac = cpu_work(n) if kind == 'mm_prefill' else n / cpu_total
    cpu_ms = dt / frac * 1e3
    record = {'metric': f'{name} µs per launch', 'value': round(ms * 1e3, 3), 'unit': 'µs', 'n_gpus': 1,
              'steps': steps, 'warmup': args.warmup, 'ms_per_step': round(ms, 6), 'timing': spread(per, rot),
              'higher_is_better': False, 'scaling': 'weak', 'vs_baseline': None, 'dtype': conf.pop('dtype'),
              'data': 'synthetic', 'config': dict(workload=name, **conf),
              'algorithmic_bytes': nbytes, 'algorithmic_flops': flops,
              'roofline': roof,
              'cpu_baseline': {'value': round(cpu_ms * 1e3, 1), 'unit': 'µs per launch (extrapolated)', 'cores': 1,
                               'kind': 'port',
                               'sample': f'{n} of {cpu_total} {cpu_unit}: the numpy oracle (oracle/topk.py) on one '
                                         f'thread of {cpu_model()}, scaled to the whole launch'}}
    emit(record)


CEILING_WORKLOADS = ('mfma_ceiling', 'gather_ceiling_b32', 'gather_pieces_ceiling_b32', 'launch_ceiling',
                     'split_merge_ceiling')


def run_launch_ceilings(args, name, ops, cus):
    """The floors under the short kernels: an empty launch of one workgroup per CU (xt_ceiling_launch), and the
    decode kernels' split arrival alone (xt_ceiling_split_merge) on the batch-32 decode's grid: one workgroup per CU,
    each writing its partial (32 rows x 2 splits x 8 heads x 132 floats = 4224 bytes per workgroup at 2 splits),
    counting its arrival, the last of each row reloading and merging; the fenced form and 4 / 8 splits beside it.
    16 launches per graph replay; microseconds per launch, lower is better."""
    import torch
    steps, warm = max(1, args.steps), max(1, args.warmup)
    if name == 'launch_ceiling':
        ms, per, rot = time_steps(lambda _: ops.ceiling_launch(cus), 16, steps, warm)
        log(f'launch ceiling: {ms * 1e3:.2f} us per empty launch of {cus} workgroups x 512 threads')
        config = {'workload': name, 'workgroups': cus, 'threads': 512}
        metric, variants = 'empty kernel launch in a graph, us per launch', None
    else:
        part = torch.zeros(cus * 16896, dtype=torch.uint8, device='cuda')
        counters = torch.zeros(1024, dtype=torch.int32, device='cuda')
        out = torch.zeros(cus * 512, dtype=torch.int32, device='cuda')
        variants = []
        for splits, nbytes, fenced in ((2, 4224, False), (2, 4224, True), (4, 8448, False), (8, 16896, False),
                                       (8, 16896, True)):
            def step(_, splits=splits, nbytes=nbytes, fenced=fenced):
                ops.ceiling_split_merge(part, counters, out, splits, nbytes, cus, fenced)
            vms, vper, rot = time_steps(step, 16, steps, warm)
            torch.cuda.synchronize()
            cols = [range(t * 16, nbytes, 8192) for t in range(512)]
            want = torch.tensor([(splits * sum(o + 1 for o in c)) & 0xFFFFFFFF for c in cols], dtype=torch.int64)
            got = out[:cus // splits * 512].view(cus // splits, 512).cpu().long() & 0xFFFFFFFF
            assert bool((got == want).all()), f'xt_ceiling_split_merge returned wrong sums ({splits} splits)'
            assert int(counters.abs().sum()) == 0, 'xt_ceiling_split_merge left arrival counters set'
            variants.append({'splits': splits, 'bytes_per_workgroup': nbytes, 'fenced': fenced,
                             'us_per_launch': round(vms * 1e3, 3), 'timing': spread(vper, rot)})
            log(f'split merge: {splits} splits of {nbytes} B{" fenced" if fenced else ""}: {vms * 1e3:.2f} us per launch')
            if len(variants) == 1:
                ms, per = vms, vper
        config = {'workload': name, 'workgroups': cus, 'threads': 512, 'splits': 2, 'bytes_per_workgroup': 4224}
        metric = 'split arrival and merge alone (write-through, system-scope count, reload), us per launch'
    record = {'metric': metric, 'value': round(ms * 1e3, 3), 'unit': 'us', 'n_gpus': 1, 'steps': steps,
              'warmup': args.warmup, 'ms_per_step': round(ms, 6), 'timing': spread(per, rot),
              'higher_is_better': False, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'u32',
              'data': 'synthetic', 'config': config, 'roofline': None, 'cpu_baseline': None}
    if variants:
        record['variants'] = variants
    emit(record)


def run_ceiling(args, name, ops, workloads):
    """The ceilings the roofline fractions are read against (xt_ceiling_mfma / xt_ceiling_gather): the sustained dense
    MFMA rate, and the batch-32 decode's exact gather (batch 32, context 32768, top-2048, pages of 64, 576-byte
    interleaved records, 16 rotated pools) with no dequantization or math."""
    import torch
    torch.cuda.set_device(0)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    steps = max(1, args.steps)
    if name in ('launch_ceiling', 'split_merge_ceiling'):
        return run_launch_ceilings(args, name, ops, cus)
    if name == 'mfma_ceiling':
        blocks, iters = 4 * cus, 2000

        def step(_):
            ops.ceiling_mfma(iters, blocks)

        ms, per, rot = time_steps(step, 1, steps, max(1, args.warmup))
        check = ops.ceiling_mfma(iters, blocks)
        assert bool((check == 64.0 * iters).all()), 'xt_ceiling_mfma returned wrong sums'
        flops = blocks * 4 * iters * 4 * 32 * 32 * 16 * 2
        tflops = flops / (ms * 1e-3) / 1e12
        log(f'mfma ceiling: {tflops:.0f} TFLOP/s ({tflops / MFMA_PEAK_TFLOPS:.1%} of {MFMA_PEAK_TFLOPS:.0f})')
        record = {'metric': 'sustained dense FP16 MFMA TFLOP/s', 'value': round(tflops, 1), 'unit': 'TFLOP/s',
                  'n_gpus': 1, 'steps': steps, 'warmup': args.warmup, 'ms_per_step': round(ms, 6),
                  'timing': spread(per, rot), 'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None,
                  'dtype': 'f16', 'data': 'synthetic',
                  'config': {'workload': name, 'workgroups': blocks, 'mfma_per_wave': iters * 4,
                             'instruction': 'v_mfma_f32_32x32x16_f16'},
                  'roofline': {'bound': 'mfma', 'achieved': round(tflops, 1), 'peak': MFMA_PEAK_TFLOPS,
                               'unit': 'TFLOP/s', 'frac': round(tflops / MFMA_PEAK_TFLOPS, 4), 'traffic': None},
                  'cpu_baseline': None}
        emit(record)
        return
    w = workloads.WORKLOADS['gqa_decode_b32']
    gen = workloads.generator('cuda', 20261029)
    pools = [torch.randint(0, 256, (w.slots, 576), dtype=torch.uint8, device='cuda', generator=gen)
             for _ in range(args.layers)]
    pt = workloads.page_table(w.batch, w.ctx, w.page, gen, 'cuda')
    idx = workloads.index_lists(w.batch, w.ctx, w.topk, gen, 'cuda', w.index_mode)
    pieces = name == 'gather_pieces_ceiling_b32'
    splits = args.splits or 2
    words = (w.batch * 4 * splits * 512 if pieces else
             int(ops._lib.lib().xt_ceiling_gather_sink_words(w.batch, w.topk)))
    sink = torch.empty(words, dtype=torch.int32, device='cuda')

    def step(layer):
        if pieces:
            ops.ceiling_gather_pieces(pools[layer], pt, idx, w.page, splits, sink=sink)
        else:
            ops.ceiling_gather(pools[layer], pt, idx, w.page, sink=sink)

    ms, per, rot = time_steps(step, args.layers, steps, max(1, args.warmup))
    nbytes = w.batch * w.topk * 576
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f'{name}: {ms * 1e3:.2f} us per layer-step, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of '
        f'{HBM_PEAK_GBS:.0f})')
    what = ('decode gather pattern alone, per-head pieces as the decode reads them' if pieces else
            'decode gather pattern alone, whole records')
    record = {'metric': f'{what}, GB/s', 'value': round(gbs, 1), 'unit': 'GB/s', 'n_gpus': 1,
              'steps': steps, 'warmup': args.warmup, 'ms_per_step': round(ms, 6), 'timing': spread(per, rot),
              'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'u8', 'data': 'synthetic',
              'config': {'workload': name, 'batch': w.batch, 'context': w.ctx, 'topk': w.topk, 'page': w.page,
                         'record_bytes': 576, 'layers_rotated': rot,
                         **({'splits': splits, 'kv_heads_per_workgroup': 1} if pieces else {})},
              'us_per_layer_step': round(ms * 1e3, 3),
              'roofline': {'bound': 'hbm', 'achieved': round(gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                           'frac': round(gbs / HBM_PEAK_GBS, 4), 'traffic': None},
              'cpu_baseline': None}
    emit(record)


def main():
    p = argparse.ArgumentParser()
    p.add_argument('--gpus', type=int, default=1)
    p.add_argument('--steps', type=int, default=512)
    p.add_argument('--warmup', type=int, default=64)
    p.add_argument('--workload', default='gqa_decode_b32',
                   help='gqa_decode_b32 (default), cpu_ref_decode, long_ctx_decode_b4, gqa_prefill_chunk4096, '
                        'minimax_decode_b32, minimax_prefill_chunk4096, qsa_varlen_b32, qsa_gather_b32, qsa_pack_ctx65536, '
                        'mla_decode_b64, mla_prefill_2048, mla_v4_decode_b64, the top-k producers '
                        'qsa_logits_352x95088, dsa_logits_4096x16384, topk_352x95088_k2048, '
                        'minimax_decode_scores_b32, minimax_prefill_scores_8k, or the ceilings mfma_ceiling, '
                        'gather_ceiling_b32, gather_pieces_ceiling_b32, launch_ceiling and split_merge_ceiling')
    p.add_argument('--layers', type=int, default=16)
    p.add_argument('--splits', type=int, default=None)
    p.add_argument('--layout', default='interleaved', choices=['interleaved', 'split'],
                   help='pool layout: interleaved (one 576-B record per slot: per head [K pay | V pay], then per '
                        'head [K sf | V sf]) or split (SGLang buffers)')
    p.add_argument('--cpu-seconds', type=float, default=10.0)
    p.add_argument('--no-cpu-baseline', action='store_true')
    p.add_argument('--no-layout-compare', action='store_true',
                   help='decode workloads: skip timing the same step on the other pool layout')
    p.add_argument('--mla-lengths', action='store_true',
                   help='sparse-MLA workloads: pass per-row list lengths (every list full), as the DeepSeek hook '
                        'passes topk_length')
    p.add_argument('--timeline', action='store_true',
                   help='decode and sparse-MLA workloads: after the timed region, one more launch with the '
                        'per-wave timeline '
                        '(xt_decode_timeline, xt_mla_timeline) and its phase times in the record')
    p.add_argument('--copy-calibration', type=int, default=0, metavar='MIB',
                   help='only copy MIB MiB between two device buffers 8 times (the known-size kernel that scales the '
                        'FETCH_SIZE / WRITE_SIZE counters), then exit')
    args = p.parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print(json.dumps({'error': 'this benchmark runs on one GPU only: the sparse decode shards by request or KV '
                                   'head with no exchange, and no multi-GPU figure is produced'}))
        sys.exit(2)

    import torch

    if args.copy_calibration:
        src = torch.empty(args.copy_calibration << 20, dtype=torch.uint8, device='cuda')
        dst = torch.empty_like(src)
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({'copy_calibration_bytes': args.copy_calibration << 20, 'launches': 8}))
        return

    from xtier_amd import ops, workloads
    from xtier_amd.pool import KVPool

    if args.workload in CEILING_WORKLOADS:
        return run_ceiling(args, args.workload, ops, workloads)
    if args.workload in INDEXER_WORKLOADS:
        return run_indexer(args, args.workload, ops)
    if args.workload in workloads.VARLEN_WORKLOADS:
        return run_varlen(args, workloads.VARLEN_WORKLOADS[args.workload], ops, workloads)
    if args.workload in workloads.BLOCK_WORKLOADS:
        return run_block(args, workloads.BLOCK_WORKLOADS[args.workload], ops, workloads)
    if args.workload in GATHER_WORKLOADS:
        return run_gather(args, args.workload, ops, workloads, KVPool)
    if args.workload in workloads.BLOCK_PREFILL_WORKLOADS:
        return run_block_prefill(args, workloads.BLOCK_PREFILL_WORKLOADS[args.workload], ops, workloads)
    if args.workload in workloads.MLA_WORKLOADS:
        return run_mla(args, workloads.MLA_WORKLOADS[args.workload], ops, workloads)
    if args.workload in workloads.PREFILL_WORKLOADS:
        return run_prefill(args, workloads.PREFILL_WORKLOADS[args.workload], ops, workloads, KVPool)
    w = workloads.WORKLOADS[args.workload]
    torch.cuda.set_device(0)
    gen = workloads.generator('cuda', 20261029)
    t0 = time.time()
    layers = [build_layer(w, gen, args.layout, workloads, KVPool) for _ in range(args.layers)]
    q = (torch.randn(w.batch, w.q_heads, w.dim, generator=gen, device='cuda') * w.q_std).to(torch.bfloat16)
    pt = workloads.page_table(w.batch, w.ctx, w.page, gen, 'cuda')
    idx = workloads.index_lists(w.batch, w.ctx, w.topk, gen, 'cuda', w.index_mode)
    seq = torch.full((w.batch,), w.ctx, dtype=torch.int32, device='cuda')
    torch.cuda.synchronize()
    log(f'built {args.layers} layer pools ({w.slots} slots each) in {time.time() - t0:.1f} s')
    scale = 1.0 / math.sqrt(w.dim)
    splits = args.splits or ops.default_splits(w.batch, w.kv_heads, w.topk)
    ws = ops.new_workspace('cuda', w.batch, w.q_heads, w.dim, splits)
    out = torch.empty(w.batch, w.q_heads, w.dim, dtype=torch.bfloat16, device='cuda')

    def step(layer):
        ops.sparse_decode(q, layers[layer], pt, idx, seq, scale, page_size=w.page, out=out, splits=splits, ws=ws)

    steps = max(1, args.steps)
    ms, per, rot = time_steps(step, args.layers, steps, args.warmup)
    nbytes = w.algorithmic_bytes()
    gbs = nbytes / (ms * 1e-3) / 1e9
    props = torch.cuda.get_device_properties(0)
    log(f'{w.name}: {ms * 1e3:.2f} us per layer-step, {gbs:.0f} GB/s algorithmic ({gbs / HBM_PEAK_GBS:.1%} of '
        f'{HBM_PEAK_GBS:.0f}), splits {splits}, {args.layout} pool, {props.multi_processor_count} CUs')
    timeline = None
    if args.timeline:
        # one launch on the pool used half a rotation ago (its records are out of the MALL by now, as in the timed
        # region)
        hpw, waves, units = ops.decode_shape(w.batch, w.kv_heads, splits, w.dim)
        torch.cuda.synchronize()
        with ops.decode_timeline(units * waves) as tl:
            step(rot // 2)
        timeline = timeline_summary(tl.stamps, waves, ops.TIMELINE_PHASES)
        timeline['shape'] = {'kv_heads_per_workgroup': hpw, 'waves_per_workgroup': waves, 'workgroups': units,
                             'pool_layout': args.layout}
        log('timeline: ' + json.dumps(timeline))
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(layers[0], q, pt, idx, seq, w, scale)
        log(f'cpu baseline: {cpu}')
    other = None
    if not args.no_layout_compare:
        # the same step on the other pool layout (SGLang's split buffers are what the drop-in hook receives)
        alt = 'split' if args.layout == 'interleaved' else 'interleaved'
        del layers
        torch.cuda.empty_cache()
        layers = [build_layer(w, gen, alt, workloads, KVPool) for _ in range(args.layers)]
        ms_alt, per_alt, rot_alt = time_steps(step, args.layers, steps, args.warmup)
        other = {'pool_layout': alt, 'us_per_layer_step': round(ms_alt * 1e3, 3), 'timing': spread(per_alt, rot_alt),
                 'achieved_gbs': round(nbytes / (ms_alt * 1e-3) / 1e9, 1),
                 'frac': round(nbytes / (ms_alt * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f'{alt} pool: {ms_alt * 1e3:.2f} us per layer-step')
    traffic = measured_traffic(w.name, splits, args.layout)
    record = {
        'metric': METRIC, 'value': round(gbs, 1), 'unit': 'GB/s', 'n_gpus': 1, 'steps': steps,
        'warmup': args.warmup, 'ms_per_step': round(ms, 6), 'timing': spread(per, rot), 'higher_is_better': True, 'scaling': 'weak',
        'vs_baseline': None, 'dtype': 'f16', 'data': 'synthetic',
        'config': {'workload': w.name, 'batch': w.batch, 'q_heads': w.q_heads, 'kv_heads': w.kv_heads,
                   'head_dim': w.dim, 'context': w.ctx, 'topk': w.topk, 'page': w.page, 'kv_format': 'nvfp4',
                   'layers_rotated': rot, 'splits': splits, 'pool_layout': args.layout},
        'us_per_layer_step': round(ms * 1e3, 3),
        'tokens_per_s': round(w.batch / (ms * 1e-3), 1),
        'hbm_frac': round(gbs / HBM_PEAK_GBS, 4),
        'roofline': {'bound': 'hbm', 'achieved': round(gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': round(gbs / HBM_PEAK_GBS, 4), 'traffic': traffic,
                     'traffic_source': None if traffic is None else
                     f'profiles/decode_split_{w.name}_hbm_traffic.txt: rocprofv3 FETCH_SIZE and WRITE_SIZE of this '
                     'workload, split count and pool layout (one counter per run, scaled by a copy of known size), '
                     'committed with the kernel build; not measured in this run'},
        'cpu_baseline': cpu,
        'other_layout': other,
    }
    if timeline is not None:
        record['timeline'] = timeline
    emit(record)


if __name__ == '__main__':
    main()
