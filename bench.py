#!/usr/bin/env python3
"""Benchmark the fused Avey / Avey-B forward contextualizer on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config C2] [--all-configs]

A step is one call of the hot path (``avey`` / ``avey_b``) on one batch of the
configuration's synthetic, seeded inputs, already resident in HBM. The timed
region replays a HIP graph that holds exactly K back-to-back calls, bracketed
by ``torch.cuda.synchronize()``; HIP events on the launch stream give the
per-call duration used for the roofline. Prints ONE JSON line on stdout.

Work accounting (see avey_kernel_amd/workloads.py): useful flops
F = 4 * D * (allowed query-key pairs); compulsory bytes M = z_tr + z_tl + out
(+ V, bias, valid). The headline C2 config (AI = 85 flop/B) sits below the
MI355X ridge (315 flop/B), so its roofline is HBM.

The CPU baseline times the numpy oracle (oracle/avey_oracle.py, fp32 like the
reference's eager path) on the host cores, on the full config for about
``--cpu-seconds`` of work; it is a reported baseline only.
"""

import argparse
import json
import math
import os
import statistics
import sys
import time

METRIC = 'contextualizer fwd µs/call + TFLOP/s (MFMA util %), bf16 B16×N256×D768'
PEAK_BF16_TFLOPS = 2516.6
PEAK_HBM_GBPS = 8000.0
RIDGE = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBPS * 1e9)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split('\n\n')[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=200)
    ap.add_argument('--warmup', type=int, default=20)
    ap.add_argument('--config', default='C2')
    ap.add_argument('--cpu-seconds', type=float, default=10.0)
    ap.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline')
    ap.add_argument('--cold-calls', type=int, default=0,
                    help='also time this many calls with the MALL flushed before each (off by default so that '
                         'every traced dispatch of the default run is a warm one)')
    ap.add_argument('--all-configs', action='store_true',
                    help='also measure every configuration (table on stderr, --report JSON)')
    ap.add_argument('--report', default=None, help='write all measurements to this JSON file')
    ap.add_argument('--dispatches', type=int, default=0,
                    help='profiling run: launch the config this many times (eager, no timing, no JSON) '
                         'after one plain copy of --copy-mib MiB, whose HBM counters calibrate the '
                         'per-dispatch FETCH_SIZE / WRITE_SIZE readings')
    ap.add_argument('--copy-mib', type=int, default=256)
    ap.add_argument('--backward', action='store_true',
                    help='also time the fused backward (avey_bwd) and forward+backward through autograd '
                         'against autograd over the eager path, for every configuration')
    return ap.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def measure_graph(torch, fn, steps, warmup):
    """Warm up, capture `steps` back-to-back calls in one HIP graph, time one replay."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(steps):
            fn()
    graph.replay()  # untimed: first replay uploads the graph
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = start.elapsed_time(end)
    del graph
    return ev_ms / steps, wall * 1e3 / steps


def measure_eager(torch, fn, steps):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def measure_cold(torch, fn, calls):
    """Per-call kernel span with the 256 MB MALL flushed by a 512 MiB write before each call."""
    scratch = torch.empty(512 << 20, dtype=torch.uint8, device='cuda')
    spans = []
    evs = []
    for i in range(calls):
        scratch.fill_(i & 0xFF)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        evs.append((a, b))
    torch.cuda.synchronize()
    for a, b in evs:
        spans.append(a.elapsed_time(b))
    del scratch
    return statistics.median(spans)


def cpu_baseline(cfg, inputs_cpu, seconds):
    """Time the numpy oracle (fp32, the reference's eager arithmetic) on the host."""
    import numpy as np
    from oracle import avey_oracle as orc
    try:
        from threadpoolctl import threadpool_info
        cores = max([d.get('num_threads', 1) for d in threadpool_info()] or [1])
    except Exception:  # pragma: no cover - reporting only
        cores = os.cpu_count() or 1
    z = inputs_cpu['z_tr'].float().numpy()
    gate = inputs_cpu['z_tl'].float().numpy()
    bias = inputs_cpu['bias'].float().numpy()
    v = inputs_cpu['v'].float().numpy()
    valid = None if inputs_cpu['valid'] is None else inputs_cpu['valid'].numpy()
    normalize = cfg.op == 'avey_b'

    def once():
        return orc.contextualize(z, None if normalize else v, gate, bias, valid, eps=1e-6, norm_eps=1e-12,
                                 causal=cfg.causal, normalize=normalize, activation='identity', acc=np.float32)

    once()  # warm caches / thread pools
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
        if len(times) >= 200:
            break
    return statistics.median(times), cores, len(times)


def measure_config(torch, wl, tag, steps, warmup, cold_calls):
    cfg = wl.CONFIGS[tag]
    inp = wl.make_inputs(cfg, device='cuda')
    flops = wl.useful_flops(cfg, inp['valid'])
    nbytes = wl.compulsory_bytes(cfg)

    def fn():
        return wl.call(cfg, inp, backend='hip')

    per_call_ms, wall_ms = measure_graph(torch, fn, steps, warmup)
    eager_ms = measure_eager(torch, fn, max(steps // 4, 10))
    cold_ms = measure_cold(torch, fn, cold_calls) if cold_calls > 0 else None
    return cfg, inp, flops, nbytes, per_call_ms, wall_ms, eager_ms, cold_ms


def measure_backward(torch, wl, tag, steps, warmup):
    """Fused backward alone (HIP graph), and forward + backward through autograd for
    the fused op and for the eager path (the reference's gradient path, ops.py:96-106)."""
    cfg = wl.CONFIGS[tag]
    inp = wl.make_inputs(cfg, device='cuda')
    g = torch.Generator().manual_seed(100 + cfg.seed)
    dout = torch.randn(inp['z_tr'].shape, generator=g).to(cfg.dtype).to('cuda')
    v = inp['v'] if cfg.op == 'avey' else None
    normalize = cfg.op == 'avey_b'
    op = torch.ops.avey_kernels.contextualize_backward

    def bwd():
        return op(dout, inp['z_tr'], v, inp['z_tl'], inp['bias'], inp['valid'], 1e-6, 1e-12, cfg.causal, normalize,
                  'identity', True, True, True)

    bwd_ms, _ = measure_graph(torch, bwd, steps, warmup)
    leaves = {k: (t.clone().requires_grad_() if k in ('z_tr', 'z_tl', 'v', 'bias') else t) for k, t in inp.items()}

    def fwd_bwd(backend):
        def run():
            for t in leaves.values():
                if t is not None and t.requires_grad:
                    t.grad = None
            wl.call(cfg, leaves, backend=backend).backward(dout)
        return run

    fused = fwd_bwd('hip')
    eager = fwd_bwd('torch')
    for fn in (fused, eager):
        for _ in range(3):
            fn()
    reps = max(steps // 4, 10)
    fused_ms = measure_eager(torch, fused, reps)
    eager_ms = measure_eager(torch, eager, reps)
    # Useful backward work: S, num, dP, dS zhat, dS^T zhat and P^T dnum once each,
    # 2 * D flops per allowed pair apiece (the kernels recompute S and num on top).
    flops = 3 * wl.useful_flops(cfg, inp['valid'])
    row = {'config': cfg.name, 'bwd_us': round(bwd_ms * 1e3, 2),
           'bwd_tflops_useful': round(flops / (bwd_ms * 1e-3) / 1e12, 2),
           'fwd_bwd_autograd_us_fused': round(fused_ms * 1e3, 1),
           'fwd_bwd_autograd_us_eager': round(eager_ms * 1e3, 1),
           'speedup_vs_eager': round(eager_ms / fused_ms, 2)}
    del inp, leaves
    torch.cuda.empty_cache()
    return row


def roofline_block(flops, nbytes, per_call_ms, traffic):
    ai = flops / nbytes
    if ai < RIDGE:
        achieved = nbytes / (per_call_ms * 1e-3) / 1e9
        return {'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': PEAK_HBM_GBPS, 'unit': 'GB/s',
                'frac': round(achieved / PEAK_HBM_GBPS, 4), 'traffic': traffic}
    achieved = flops / (per_call_ms * 1e-3) / 1e12
    return {'bound': 'mfma', 'achieved': round(achieved, 2), 'peak': PEAK_BF16_TFLOPS, 'unit': 'TFLOP/s',
            'frac': round(achieved / PEAK_BF16_TFLOPS, 4), 'traffic': traffic}


def load_traffic(tag):
    """HBM bytes per dispatch from the committed rocprofv3 PMC summary for this config, if present.

    profiles/<kernel>_<tag>_hbm_traffic.txt holds FETCH_SIZE + WRITE_SIZE per dispatch, each scaled
    by what the same counter reads for a plain copy of known size.
    """
    import glob
    root = os.path.dirname(os.path.abspath(__file__))
    for path in sorted(glob.glob(os.path.join(root, 'profiles', f'*_{tag}_hbm_traffic.txt'))):
        with open(path) as fh:
            for line in fh:
                if line.startswith('traffic_bytes_per_dispatch:'):
                    return int(float(line.split(':', 1)[1]))
    return None


def profile_dispatches(torch, wl, tag, n, copy_mib):
    """Launch sequence for rocprofv3 counter runs: one copy of known size, then n calls."""
    src = torch.empty(copy_mib << 20, dtype=torch.uint8, device='cuda').fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)  # reads and writes exactly copy_mib MiB each
    torch.cuda.synchronize()
    del src, dst
    cfg = wl.CONFIGS[tag]
    inp = wl.make_inputs(cfg, device='cuda')
    for _ in range(n):
        wl.call(cfg, inp, backend='hip')
    torch.cuda.synchronize()
    log(f'[bench] profiled {n} dispatches of {cfg.name} after a {copy_mib} MiB copy; '
        f'compulsory bytes {wl.compulsory_bytes(cfg)}')


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f'bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path.',
              file=sys.stderr)
        sys.exit(2)
    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from avey_kernel_amd import _hip
    from avey_kernel_amd import workloads as wl

    _hip.load()
    if not torch.cuda.is_available():
        print('bench.py needs a GPU', file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    props = torch.cuda.get_device_properties(0)
    log(f'[bench] device {props.name} {getattr(props, "gcnArchName", "")} CUs {props.multi_processor_count}')
    if args.dispatches > 0:
        profile_dispatches(torch, wl, args.config, args.dispatches, args.copy_mib)
        return

    cfg, inp, flops, nbytes, per_call_ms, wall_ms, eager_ms, cold_ms = measure_config(
        torch, wl, args.config, args.steps, args.warmup, args.cold_calls)
    tflops = flops / (per_call_ms * 1e-3) / 1e12
    plan = _hip.plan(tuple(inp['z_tr'].shape), cfg.dtype, causal=cfg.causal, normalize=cfg.op == 'avey_b')
    log(f'[bench] {cfg.name}: {per_call_ms * 1e3:.2f} us/call (graph), {eager_ms * 1e3:.2f} us/call (eager), '
        f'cold {cold_ms * 1e3 if cold_ms else float("nan"):.2f} us, {tflops:.1f} TFLOP/s, plan {plan}')

    extra = {
        'us_per_call_graph_warm': round(per_call_ms * 1e3, 3),
        'us_per_call_eager': round(eager_ms * 1e3, 3),
        'us_per_call_cold_mall_flushed': None if cold_ms is None else round(cold_ms * 1e3, 3),
        'tflops_cold': None if cold_ms is None else round(flops / (cold_ms * 1e-3) / 1e12, 2),
        'wall_ms_per_step': round(wall_ms, 5),
        'useful_flops': flops,
        'compulsory_bytes': nbytes,
        'plan': plan,
    }

    cpu = None
    if not args.no_cpu:
        inputs_cpu = wl.make_inputs(cfg, device='cpu')
        secs, cores, reps = cpu_baseline(cfg, inputs_cpu, args.cpu_seconds)
        cpu = {'value': round(flops / secs / 1e12, 5), 'unit': 'TFLOP/s', 'cores': cores, 'kind': 'port',
               'sample': f'numpy oracle (fp32, dense N x N like ops.py:61-91) on the full {cfg.tag} inputs, '
                         f'median of {reps} calls = {secs * 1e3:.1f} ms/call; useful-flop rate'}
        log(f'[bench] cpu baseline {cpu}')

    all_rows = []
    if args.all_configs:
        for tag in wl.CONFIGS:
            c2, i2, f2, b2, ms2, _, eg2, cold2 = measure_config(torch, wl, tag, max(args.steps // 2, 20),
                                                                args.warmup, args.cold_calls)
            row = {'config': c2.name, 'us_per_call': round(ms2 * 1e3, 3), 'us_eager': round(eg2 * 1e3, 3),
                   'us_cold': None if cold2 is None else round(cold2 * 1e3, 3),
                   'tflops_useful': round(f2 / (ms2 * 1e-3) / 1e12, 2),
                   'pct_bf16_peak': round(100 * f2 / (ms2 * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
                   'roofline': roofline_block(f2, b2, ms2, load_traffic(tag)),
                   'plan': _hip.plan(tuple(i2['z_tr'].shape), c2.dtype, causal=c2.causal,
                                     normalize=c2.op == 'avey_b')}
            all_rows.append(row)
            log(f'[bench] {json.dumps(row)}')
            del i2
            torch.cuda.empty_cache()

    bwd_rows = []
    if args.backward:
        for tag in wl.CONFIGS:
            row = measure_backward(torch, wl, tag, max(args.steps // 4, 20), min(args.warmup, 5))
            bwd_rows.append(row)
            log(f'[bench] backward {json.dumps(row)}')

    line = {
        'metric': METRIC,
        'value': round(tflops, 3),
        'unit': 'TFLOP/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(per_call_ms, 6),
        'us_per_call': round(per_call_ms * 1e3, 3),
        'mfma_util_pct': round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'bf16' if cfg.dtype == torch.bfloat16 else str(cfg.dtype).replace('torch.', ''),
        'data': f'synthetic: seeded inputs of BASELINE config {cfg.tag} (x, gate ~ N(0,1), V ~ U(+-1/sqrt(N)), '
                f'bias 0), resident in HBM',
        'config': {'workload': cfg.name, 'op': cfg.op, 'batch': cfg.batch, 'context': cfg.context,
                   'features': cfg.features, 'causal': cfg.causal, 'gate': True, 'bias': 'zeros',
                   'activation': 'identity', 'parallelism': 'single GPU',
                   'timing': f'one HIP graph of {args.steps} back-to-back calls; HIP events on the launch stream',
                   'flops': 'useful: 4*D*allowed pairs'},
        'roofline': roofline_block(flops, nbytes, per_call_ms, load_traffic(cfg.tag)),
        'cpu_baseline': cpu,
        'extra': extra,
    }
    if args.report:
        with open(args.report, 'w') as fh:
            json.dump({'headline': line, 'configs': all_rows, 'backward': bwd_rows}, fh, indent=1)
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
