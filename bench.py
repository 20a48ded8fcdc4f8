#!/usr/bin/env python3
"""Benchmark of the MI355X task-graph executor on BASELINE.json's headline configurations.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|gpt162m|decode|sched] [--no-cpu-baseline]

A "step" is one run of the workload's task graph (one persistent-kernel launch): one GPT-162M training step
(forward + backward + AdamW), or one Qwen3-8B-shape greedy decode token for every sequence of the batch. Inputs and
weights are synthetic (seeded, on the device) and resident in HBM before the timed region; the timed region is K
back-to-back launches bracketed by HIP events on the executor's stream. Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
METRIC = 'GPT-162M train step ms; Qwen3-8B-shape decode tok/s + HBM GB/s fraction'


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_executor(w, trace=False):
    from kvm_amd import bundle as bl
    from kvm_amd import compiler
    from kvm_amd.executor import Executor
    t0 = time.perf_counter()
    lb = bl.load(compiler.compile_spec(w.spec))
    t1 = time.perf_counter()
    ex = Executor(num_vars=max(1, len(lb.metadata['variables'])), trace=trace, timeout_s=60.0)
    for m in lb.metadata['buffers']:
        ex.add_buffer(m['name'], m['rows'], m['cols'], m['dtype'], init=w.init_override.get(m['name'], m['init']))
    for v in lb.metadata['variables']:
        ex.set_version(v['id'], v['base_version'])
    ex.submit(lb)
    ex.meta = lb.metadata
    log(f'  graph: {lb.ntasks} tasks, {lb.succ.size} edges (compile {t1 - t0:.1f}s, load {time.perf_counter() - t1:.1f}s)')
    return ex, lb


def time_steps(ex, steps, warmup):
    for _ in range(warmup):
        ex.relaunch()
        ex.finish()
    ms = ex.run_timed(steps)
    res = ex.finish()
    return ms / steps, res


def bench_decode(batch, steps, warmup, cpu):
    from kvm_amd.workloads import qwen3
    c = qwen3.Qwen3Config(batch=batch, max_new=max(64, steps + warmup + 8))
    w = qwen3.build(c)
    log(f'decode batch {batch}: building')
    ex, lb = build_executor(w)
    ms, res = time_steps(ex, steps, warmup)
    byts = w.info['weight_bytes'] + w.info['kv_bytes_per_step']
    gbs = byts / (ms / 1e3) / 1e9
    out = {'batch': batch, 'ms_per_token_step': round(ms, 4), 'tok_s': round(batch * 1e3 / ms, 2), 'hbm_gbs': round(gbs, 1),
           'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'bytes_per_step': byts, 'tasks': lb.ntasks}
    log(f'  decode batch {batch}: {ms:.3f} ms/step, {out["tok_s"]} tok/s, {gbs:.0f} GB/s ({out["hbm_frac"]:.1%} of peak)')
    ex.close()
    if cpu:
        out['cpu_baseline'] = cpu_decode(batch)
    return out


def cpu_decode(batch):
    """Oracle on a 1-layer full-width Qwen3 graph (+ LM head), scaled to 36 layers by weight elements."""
    import oracle
    from kvm_amd import bundle as bl
    from kvm_amd import compiler
    from kvm_amd.workloads import qwen3
    c1 = qwen3.Qwen3Config(batch=batch, layers=1, max_new=4)
    w = qwen3.build(c1)
    lb = bl.load(compiler.compile_spec(w.spec))
    bufs = [bl.materialize({**m, 'init': w.init_override.get(m['name'], m['init'])}) for m in lb.metadata['buffers']]
    r = oracle.run(lb, bufs)
    full = qwen3.weight_elems(qwen3.Qwen3Config(batch=batch))
    est = r['seconds'] * full / qwen3.weight_elems(c1)
    return {'value': round(batch / est, 4), 'unit': 'tok/s', 'cores': 1, 'kind': 'port',
            'sample': f'C++ oracle (restated reference CPU VM) on a 1-layer full-width graph + LM head, batch {batch}: '
                      f'{r["seconds"]:.2f} s, scaled x{full / qwen3.weight_elems(c1):.1f} by weight elements to 36 layers'}


def bench_sched():
    """Dependent-hop latency (a chain of noops) and fan-out/fan-in cost (wide noop phases)."""
    from kvm_amd.workloads import Builder, Workload
    b = Builder()
    prev = []
    for i in range(2000):
        prev = [b.task('noop', after=prev)]
    ex, lb = build_executor(Workload(b.spec()))
    ms, _ = time_steps(ex, 5, 2)
    hop_us = ms * 1e3 / 2000
    ex.close()
    b = Builder()
    prev = []
    for p in range(50):
        prev = [b.task('noop', after=prev) for _ in range(512)]
        prev = [b.task('noop', after=prev)]
    ex, lb = build_executor(Workload(b.spec()))
    ms2, _ = time_steps(ex, 5, 2)
    ex.close()
    out = {'hop_us': round(hop_us, 3), 'phase_us_512wide': round(ms2 * 1e3 / 50, 2), 'tasks_per_s_wide': round(50 * 513 / (ms2 / 1e3))}
    log(f'  sched: {hop_us:.2f} us per dependent hop; 512-wide noop phase + join: {out["phase_us_512wide"]} us')
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--workload', default='all', choices=['all', 'gpt162m', 'decode', 'sched'])
    ap.add_argument('--decode-batch', default='1,8')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    a = ap.parse_args()
    if a.gpus != 1:
        print(json.dumps({'error': 'this executor runs on one GPU; multi-GPU runs are not part of this build', 'n_gpus': a.gpus}))
        sys.exit(2)
    cpu = not a.no_cpu_baseline
    result = {'metric': METRIC, 'n_gpus': 1, 'steps': a.steps, 'warmup': a.warmup, 'scaling': 'weak', 'vs_baseline': None,
              'data': 'synthetic (seeded weights/KV/tokens generated on the device)'}
    extra = {}
    if a.workload in ('all', 'sched'):
        extra['sched'] = bench_sched()
    if a.workload in ('all', 'decode'):
        extra['decode'] = [bench_decode(int(bs), a.steps, a.warmup, cpu) for bs in a.decode_batch.split(',')]
    if a.workload in ('all', 'decode') and 'gpt162m' not in extra:
        d = extra['decode'][0]
        result.update({'value': d['tok_s'], 'unit': 'tok/s', 'higher_is_better': True, 'ms_per_step': d['ms_per_token_step'],
                       'dtype': 'bf16', 'config': {'workload': f'qwen3-8b-shape decode, batch {d["batch"]}, 4096-token KV cache'},
                       'roofline': {'bound': 'hbm', 'achieved': d['hbm_gbs'], 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                                    'frac': d['hbm_frac'], 'traffic': None}})
        if 'cpu_baseline' in d:
            result['cpu_baseline'] = d['cpu_baseline']
    result.update(extra)
    print(json.dumps(result))


if __name__ == '__main__':
    main()
