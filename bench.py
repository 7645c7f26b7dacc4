#!/usr/bin/env python3
"""Benchmark the fused Avey / Avey-B forward contextualizer on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config C2] [--headline-only]

A step is one call of the hot path (``avey`` / ``avey_b``) on one batch of the
configuration's synthetic, seeded inputs, already resident in HBM. The timed
region replays a HIP graph that holds exactly K back-to-back calls, bracketed
by ``torch.cuda.synchronize()``; HIP events on the launch stream give the
per-call duration used for the roofline. Prints ONE JSON line on stdout.

Work accounting (see avey_kernel_amd/workloads.py): useful flops
F = 4 * D * (allowed query-key pairs); compulsory bytes M = z_tr + z_tl + out
(+ V, bias, valid). The headline C2 config (AI = 85 flop/B) sits below the
MI355X ridge (315 flop/B), so its roofline is HBM.

Besides the warm (back-to-back, MALL-resident) figure, every configuration is
also timed cold: each of ``--cold-calls`` calls follows a 512 MiB write that
evicts the 256 MB MALL and the L2s. The calls are queued behind a spin kernel,
so that the GPU never waits for the host inside a span; a single call's event
span still carries the per-launch overhead the graph hides, so the cold kernel
time is the warm graph time plus the difference between cold and warm
single-call spans measured the same way (warm: a 4 KiB write instead).

The CPU baseline times the torch-eager restatement of the reference's path
(oracle/avey_torch_ref.py, what the reference runs on ROCm, fp32 accumulation,
dense N x N) under ``torch.inference_mode()`` on the host cores, at the default
thread count and at one thread; it is a reported baseline only.
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
SPANS = {}  # config tag -> (cold, warm) median single-call event spans in us


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split('\n\n')[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=200)
    ap.add_argument('--warmup', type=int, default=20)
    ap.add_argument('--config', default='C2')
    ap.add_argument('--cpu-seconds', type=float, default=6.0,
                    help='bound on the CPU baseline time per thread setting (at least 10 calls are timed)')
    ap.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline')
    ap.add_argument('--cold-calls', type=int, default=20,
                    help='calls timed with the MALL and L2s flushed before each (0: skip)')
    ap.add_argument('--headline-only', action='store_true',
                    help='skip the per-configuration table (C1-C5) in extra.configs')
    ap.add_argument('--all-configs', action='store_true', help=argparse.SUPPRESS)  # the table is on by default
    ap.add_argument('--report', default=None, help='write all measurements to this JSON file')
    ap.add_argument('--dispatches', type=int, default=0,
                    help='profiling run: launch the config this many times (eager, no timing, no JSON) '
                         'after one plain copy of --copy-mib MiB, whose HBM counters calibrate the '
                         'per-dispatch FETCH_SIZE / WRITE_SIZE readings')
    ap.add_argument('--copy-mib', type=int, default=256)
    ap.add_argument('--enriched', action='store_true',
                    help='also time avey_fwd_enriched (the enricher gate formed in the kernel) against '
                         'the gate GEMM + activation + contextualizer, for C2-C5 behind a d = D/2 enricher')
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


def measure_single_calls(torch, fn, calls, flush):
    """Median event span of single calls, each after a 512 MiB write (flush=True,
    which evicts the 256 MB MALL and every L2) or after a small write on the
    same stream (flush=False: a 4 KiB write, the inputs stay resident)."""
    scratch = torch.empty((512 << 20) if flush else 4096, dtype=torch.uint8, device='cuda')
    evs = []
    # Every call is enqueued while the GPU spins (about 4 ms at 2.4 GHz), so no span
    # waits for the host to launch its call, with a small write before it or a large one.
    torch.cuda.synchronize()
    torch.cuda._sleep(10_000_000)
    for i in range(calls):
        scratch.fill_(i & 0xFF)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        evs.append((a, b))
    torch.cuda.synchronize()
    del scratch
    return statistics.median(a.elapsed_time(b) for a, b in evs)


def host_cpu_model():
    try:
        import subprocess
        out = subprocess.run(['lscpu'], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith('Model name:'):
                return line.split(':', 1)[1].strip()
    except Exception:  # pragma: no cover - reporting only
        pass
    return 'unknown'


def cpu_baseline(torch, cfg, inputs_cpu, seconds, threads):
    """Median seconds per call of the torch-eager restatement of the reference's path
    (oracle/avey_torch_ref.py) on the CPU at `threads` threads: 2 warm-up calls, then
    at least 10 timed calls and at least one second, bounded by `seconds`."""
    from oracle import avey_torch_ref as tref
    normalize = cfg.op == 'avey_b'
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        def once():
            return tref.contextualize(inputs_cpu['z_tr'], None if normalize else inputs_cpu['v'],
                                      inputs_cpu['z_tl'], inputs_cpu['bias'], inputs_cpu['valid'], eps=1e-6,
                                      norm_eps=1e-12, causal=cfg.causal, normalize=normalize,
                                      activation='identity')
        with torch.inference_mode():
            for _ in range(2):
                once()
            times = []
            t_start = time.perf_counter()
            while len(times) < 10 or (time.perf_counter() - t_start < 1.0):
                t0 = time.perf_counter()
                once()
                times.append(time.perf_counter() - t0)
                if time.perf_counter() - t_start > seconds and len(times) >= 3:
                    break
        return statistics.median(times), len(times)
    finally:
        torch.set_num_threads(prev)


def measure_config(torch, wl, tag, steps, warmup, cold_calls):
    """Warm graph time per call, eager time per call, and the cold kernel estimate."""
    cfg = wl.CONFIGS[tag]
    inp = wl.make_inputs(cfg, device='cuda')
    flops = wl.useful_flops(cfg, inp['valid'])
    nbytes = wl.compulsory_bytes(cfg)

    def fn():
        return wl.call(cfg, inp, backend='hip')

    per_call_ms, wall_ms = measure_graph(torch, fn, steps, warmup)
    eager_ms = measure_eager(torch, fn, max(steps // 4, 10))
    cold_ms = None
    if cold_calls > 0:
        span_cold = measure_single_calls(torch, fn, cold_calls, flush=True)
        span_warm = measure_single_calls(torch, fn, cold_calls, flush=False)
        # A negative difference (the kernel hides its HBM fetch) counts as no penalty.
        cold_ms = per_call_ms + max(span_cold - span_warm, 0.0)
        SPANS[tag] = (round(span_cold * 1e3, 3), round(span_warm * 1e3, 3))
    return cfg, inp, flops, nbytes, per_call_ms, wall_ms, eager_ms, cold_ms


def measure_enriched(torch, wl, tag, steps, warmup):
    """avey_fwd_enriched (z_tl formed per row block in the kernel, never stored) against
    the composition it replaces: the enricher's gate GEMM (hipBLASLt, bf16 out), its
    ReLU, then the contextualizer reading z_tl. Model width d = D / 2; both in one HIP
    graph of back-to-back calls. Also the contextualizer alone with a stored z_tl."""
    import torch.nn.functional as F
    from avey_kernel_amd import avey_b_enriched, avey_enriched
    cfg = wl.CONFIGS[tag]
    inp = wl.make_inputs(cfg, device='cuda')
    d = cfg.features // 2
    g = torch.Generator().manual_seed(200 + cfg.seed)
    x = torch.randn(cfg.batch, cfg.context, d, generator=g).to(cfg.dtype).to('cuda')
    w = (torch.randn(cfg.features, d, generator=g) / d ** 0.5).to(cfg.dtype).to('cuda')
    bg = (torch.randn(cfg.features, generator=g) * 0.1).to(cfg.dtype).to('cuda')
    normalize = cfg.op == 'avey_b'
    v = inp['v'] if not normalize else None
    kw = dict(bias=inp['bias'], valid=inp['valid'])

    def fused():
        if normalize:
            return avey_b_enriched(x, w, inp['z_tr'], b_gate=bg, gate_activation='relu', backend='hip', **kw)
        return avey_enriched(x, w, inp['z_tr'], v, b_gate=bg, gate_activation='relu', causal=cfg.causal,
                             backend='hip', **kw)

    def unfused():
        gate = F.relu(F.linear(x, w, bg))
        return wl.call(cfg, dict(inp, z_tl=gate), backend='hip')

    def op_only():
        return wl.call(cfg, inp, backend='hip')

    with torch.inference_mode():
        fused_ms, _ = measure_graph(torch, fused, steps, warmup)
        unfused_ms, _ = measure_graph(torch, unfused, steps, warmup)
        op_ms, _ = measure_graph(torch, op_only, steps, warmup)
    es = 2
    n = cfg.batch * cfg.context
    row = {'config': cfg.name, 'model_dim': d, 'fused_us': round(fused_ms * 1e3, 2),
           'gemm_act_op_us': round(unfused_ms * 1e3, 2), 'op_alone_us': round(op_ms * 1e3, 2),
           'speedup': round(unfused_ms / fused_ms, 3),
           'hbm_bytes_removed': 2 * n * cfg.features * es,  # z_tl written by the GEMM, read by the op
           'hbm_bytes_added': n * d * es}                   # x read by the op
    del inp, x, w
    torch.cuda.empty_cache()
    return row


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


def roofline_block(flops, nbytes, per_call_ms, traffic, cold_ms=None):
    """Roofline of one call: HBM-bound below the ridge (compulsory bytes / time),
    MFMA-bound above it (useful flops / time). `frac_cold` applies the same to the
    cold (MALL-flushed) kernel time."""
    ai = flops / nbytes
    if ai < RIDGE:
        rate = lambda ms: nbytes / (ms * 1e-3) / 1e9
        block = {'bound': 'hbm', 'achieved': round(rate(per_call_ms), 1), 'peak': PEAK_HBM_GBPS, 'unit': 'GB/s'}
        peak = PEAK_HBM_GBPS
    else:
        rate = lambda ms: flops / (ms * 1e-3) / 1e12
        block = {'bound': 'mfma', 'achieved': round(rate(per_call_ms), 2), 'peak': PEAK_BF16_TFLOPS,
                 'unit': 'TFLOP/s'}
        peak = PEAK_BF16_TFLOPS
    block['frac'] = round(rate(per_call_ms) / peak, 4)
    block['traffic'] = traffic
    if cold_ms is not None:
        block['achieved_cold'] = round(rate(cold_ms), 2)
        block['frac_cold'] = round(rate(cold_ms) / peak, 4)
    return block


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


def load_mfma_busy(tag):
    """Counter-measured MFMA busy percentage (rocprofv3 derived counter MfmaUtil =
    SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs)) from the committed summary
    profiles/fused_fwd_counters.md, if present."""
    root = os.path.dirname(os.path.abspath(__file__))
    path = os.path.join(root, 'profiles', 'fused_fwd_counters.md')
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        for line in fh:
            if line.startswith(f'mfma_util_pct {tag}:'):
                return float(line.split(':', 1)[1])
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


def config_row(torch, wl, _hip, tag, steps, warmup, cold_calls):
    cfg, inp, flops, nbytes, ms, _, eager_ms, cold_ms = measure_config(torch, wl, tag, steps, warmup, cold_calls)
    row = {'config': cfg.name, 'us_per_call': round(ms * 1e3, 3), 'us_eager': round(eager_ms * 1e3, 3),
           'us_cold': None if cold_ms is None else round(cold_ms * 1e3, 3),
           'tflops_useful': round(flops / (ms * 1e-3) / 1e12, 2),
           'pct_bf16_peak': round(100 * flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
           'mfma_busy_pct_counter': load_mfma_busy(tag),
           'roofline': roofline_block(flops, nbytes, ms, load_traffic(tag), cold_ms),
           'single_call_spans_us_cold_warm': SPANS.get(tag),
           'plan': _hip.plan(tuple(inp['z_tr'].shape), cfg.dtype, causal=cfg.causal, normalize=cfg.op == 'avey_b')}
    del inp
    torch.cuda.empty_cache()
    return row


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
    log(f'[bench] {cfg.name}: {per_call_ms * 1e3:.2f} us/call (graph, warm), {eager_ms * 1e3:.2f} us/call (eager), '
        f'cold {cold_ms * 1e3 if cold_ms else float("nan"):.2f} us, {tflops:.1f} TFLOP/s, plan {plan}')
    del inp
    torch.cuda.empty_cache()

    extra = {
        'us_per_call_graph_warm': round(per_call_ms * 1e3, 3),
        'us_per_call_eager': round(eager_ms * 1e3, 3),
        'us_per_call_cold_mall_flushed': None if cold_ms is None else round(cold_ms * 1e3, 3),
        'tflops_cold': None if cold_ms is None else round(flops / (cold_ms * 1e-3) / 1e12, 2),
        'cold_method': f'median of {args.cold_calls} single calls after a 512 MiB write, minus the median of '
                       f'{args.cold_calls} single calls after a 4 KiB write, added to the warm graph time; '
                       f'both sets queued behind a spin kernel so that no span includes host launch time',
        'single_call_spans_us_cold_warm': SPANS.get(cfg.tag),
        'wall_ms_per_step': round(wall_ms, 5),
        'useful_flops': flops,
        'compulsory_bytes': nbytes,
        'pct_bf16_peak_useful': round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        'mfma_busy_pct_counter': load_mfma_busy(cfg.tag),
        'plan': plan,
    }

    cpu = None
    if not args.no_cpu:
        inputs_cpu = wl.make_inputs(cfg, device='cpu')
        threads = torch.get_num_threads()
        secs, reps = cpu_baseline(torch, cfg, inputs_cpu, args.cpu_seconds, threads)
        secs1, reps1 = cpu_baseline(torch, cfg, inputs_cpu, args.cpu_seconds, 1)
        dense = wl.dense_flops(cfg)
        cpu = {'value': round(flops / secs / 1e12, 5), 'unit': 'TFLOP/s', 'cores': threads, 'kind': 'port',
               'sample': f'torch-eager restatement of the reference path (oracle/avey_torch_ref.py, fp32, dense '
                         f'N x N, inference_mode) on the full {cfg.tag} inputs: median of {reps} calls = '
                         f'{secs * 1e3:.2f} ms/call at {threads} threads; useful-flop rate',
               'ms_per_call': round(secs * 1e3, 3), 'ms_per_call_1_thread': round(secs1 * 1e3, 3),
               'calls_1_thread': reps1,
               'dense_equiv_tflops': round(dense / secs / 1e12, 5),
               'dense_equiv_tflops_1_thread': round(dense / secs1 / 1e12, 5),
               'torch_num_threads': threads, 'affinity_cpus': len(os.sched_getaffinity(0)),
               'cpu_model': host_cpu_model(),
               'gpu_speedup_warm': round(secs / (per_call_ms * 1e-3), 1)}
        log(f'[bench] cpu baseline {cpu}')

    rows = []
    if not args.headline_only:
        for tag in wl.CONFIGS:
            row = config_row(torch, wl, _hip, tag, max(args.steps // 2, 20), args.warmup, args.cold_calls)
            rows.append(row)
            log(f'[bench] {json.dumps(row)}')
    extra['configs'] = rows

    if args.enriched:
        enr_rows = []
        for tag in ('C2', 'C3', 'C4', 'C5'):
            row = measure_enriched(torch, wl, tag, max(args.steps // 2, 20), min(args.warmup, 5))
            enr_rows.append(row)
            log(f'[bench] enriched {json.dumps(row)}')
        extra['enriched'] = enr_rows

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
        'roofline': roofline_block(flops, nbytes, per_call_ms, load_traffic(cfg.tag), cold_ms),
        'cpu_baseline': cpu,
        'extra': extra,
    }
    if args.report:
        with open(args.report, 'w') as fh:
            json.dump({'headline': line, 'backward': bwd_rows}, fh, indent=1)
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
