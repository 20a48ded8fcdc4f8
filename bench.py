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


def build_executor(w, trace=False, blocks=0):
    from kvm_amd import bundle as bl
    from kvm_amd import compiler
    from kvm_amd.executor import Executor
    t0 = time.perf_counter()
    lb = bl.load(compiler.compile_spec(w.spec))
    t1 = time.perf_counter()
    ex = Executor(num_vars=max(1, len(lb.metadata['variables'])), trace=trace, timeout_s=60.0, blocks=blocks)
    for m in lb.metadata['buffers']:
        ex.add_buffer(m['name'], m['rows'], m['cols'], m['dtype'], init=w.init_override.get(m['name'], m['init']))
    for v in lb.metadata['variables']:
        ex.set_version(v['id'], v['base_version'])
    ex.submit(lb)
    ex.meta = lb.metadata
    log(f'  graph: {lb.ntasks} tasks, {lb.succ.size} edges (compile {t1 - t0:.1f}s, load {time.perf_counter() - t1:.1f}s)')
    return ex, lb


def time_steps(ex, steps, warmup):
    """(ms per step for the whole job, ms per step of the persistent kernel alone, finish() of the last step)."""
    for _ in range(warmup):
        ex.relaunch()
        ex.finish()
    tot, exe = ex.run_timed_split(steps)
    res = ex.finish()
    return tot / steps, exe / steps, res


def bench_decode(batch, steps, warmup, cpu):
    from kvm_amd.workloads import qwen3
    c = qwen3.Qwen3Config(batch=batch, max_new=max(64, steps + warmup + 8))
    w = qwen3.build(c)
    log(f'decode batch {batch}: building')
    ex, lb = build_executor(w)
    ms, kms, res = time_steps(ex, steps, warmup)
    byts = w.info['weight_bytes'] + w.info['kv_bytes_per_step']
    gbs = byts / (kms / 1e3) / 1e9
    out = {'batch': batch, 'ms_per_token_step': round(ms, 4), 'kernel_ms': round(kms, 4), 'tok_s': round(batch * 1e3 / ms, 2),
           'hbm_gbs': round(gbs, 1), 'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'bytes_per_step': byts, 'tasks': lb.ntasks}
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


def gemm_task_flops(lb):
    """FLOPs of every GEMM tile task (2*tm*tn*K clipped to the matrix) and of the attention tasks (their share of
    the causal attention's algorithmic FLOPs: fwd 2 products, bwd 5), from the bundle's own arguments."""
    import numpy as np
    t, a = lb.tasks, lb.args
    fl = np.zeros(t.shape[0])
    for i in range(t.shape[0]):
        op, off = t[i, 0], t[i, 6]
        if op in (34, 114, 122):
            m0, n0, M, N, K, f = (int(x) for x in a[off + 6:off + 12])
            tm, tn = (128, 256) if op == 122 else ((256, 128) if f & 64 else (128, 128) if f & 32 else (64, 64))
            fl[i] = 2.0 * (min(M, m0 + tm) - m0) * (min(N, n0 + tn) - n0) * K
        elif op in (45, 47, 48):
            q0, T, hd = int(a[off + (7 if op != 48 else 10)]), int(a[off + (8 if op != 48 else 11)]), int(a[off + (11 if op != 48 else 13)])
            q1 = min(T, q0 + 128)
            if op == 48:   # keys [q0, q1) meet queries [k, T): sum over keys of (T - k)
                pairs = sum(T - k for k in range(q0, q1))
            else:
                pairs = sum(k + 1 for k in range(q0, q1))
            fl[i] = 2.0 * hd * pairs * (2 if op == 45 else 2.5)
    return fl


def bench_gpt(steps, warmup, cpu):
    import numpy as np
    from kvm_amd.workloads import gpt
    c = gpt.GPTConfig()
    log('gpt-162m bf16 training step: building')
    w = gpt.build(c)
    ex, lb = build_executor(w, trace=True)
    ms, kms, res = time_steps(ex, steps, warmup)
    flops = w.info['flops']['total']
    tflops = flops / (kms / 1e3) / 1e12
    # MFMA utilisation inside the GEMM / attention tasks, from the last run's per-task trace
    tr = ex.trace()
    dur = (tr['end'] - tr['start']).astype(np.float64) / 100e6     # s (wall_clock64 at 100 MHz)
    fl = gemm_task_flops(lb)
    ops = lb.tasks[:, 0]
    gm = np.isin(ops, [34, 114, 122]); at = np.isin(ops, [45, 47, 48])
    per_cu = BF16_PEAK_TFLOPS / 256 * 1e12
    in_task = {'gemm': float(fl[gm].sum() / dur[gm].sum() / per_cu), 'attention': float(fl[at].sum() / dur[at].sum() / per_cu)}
    busy = float(dur.sum() / (res['grid'] * (tr['end'].max() - tr['start'].min()) / 100e6))
    names = [m['name'] for m in lb.metadata['buffers']]
    loss = float(ex.read('loss')[0])
    out = {'ms_per_step': round(ms, 3), 'kernel_ms': round(kms, 3), 'tflops': round(tflops, 1), 'mfma_frac_step': round(tflops / BF16_PEAK_TFLOPS, 4),
           'mfma_frac_in_gemm_tasks': round(in_task['gemm'], 4), 'mfma_frac_in_attention_tasks': round(in_task['attention'], 4),
           'worker_busy_frac': round(busy, 4), 'tasks': lb.ntasks, 'edges': int(lb.succ.size), 'loss_after': loss,
           'step_flops': flops, 'params': w.info['params']}
    log(f'  gpt-162m: {ms:.2f} ms/step (persistent kernel {kms:.2f} ms), {tflops:.1f} TFLOP/s ({tflops / BF16_PEAK_TFLOPS:.1%} of bf16 peak); in-task MFMA: '
        f'GEMM {in_task["gemm"]:.1%}, attention {in_task["attention"]:.1%}; workers busy {busy:.1%}; loss {loss:.4f}')
    ex.close()
    if cpu:
        out['cpu_baseline'] = cpu_gpt(w, lb)
    return out


def cpu_gpt(w, lb, per_op=16, seed=0):
    """CPU reference time of the same GPT-162M step graph, sampled: the oracle (C++ restatement of the reference CPU VM
    and its operators) runs `per_op` tasks of every operator of the graph, drawn at random, on the step's initial
    buffers; the step estimate is the sum over operators of (task count x mean sampled task time). The sampled tasks run
    as a graph of their own with no edges, so the sample is bounded (about 10-30 s of CPU work) and its tasks read
    buffers as initialised (the operators' costs do not depend on the values). GEMM and attention tasks are scaled by
    their algorithmic FLOPs (tile sizes differ up to 60x across the graph), the others by task count."""
    import numpy as np
    import oracle
    from kvm_amd import bundle as bl
    rng = np.random.default_rng(seed)
    ops = lb.tasks[:, 0]
    pick = []
    for o in np.unique(ops):
        idx = np.nonzero(ops == o)[0]
        pick += list(rng.choice(idx, size=min(per_op, idx.size), replace=False))
    pick = np.array(sorted(pick))
    t = lb.tasks[pick].copy()
    t[:, 1] = 0; t[:, 2] = 0; t[:, 3] = 0          # no successors, no predecessors
    t[:, 8] = -1; t[:, 10] = -1                     # no version wait, no publish
    sub = bl.LoadedBundle({**lb.metadata, 'reads': [], 'publishers': []}, t, np.zeros(0, np.int32), lb.args, lb.root)
    bufs = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    r = oracle.run(sub, bufs)
    fl = gemm_task_flops(lb)            # GEMM and attention tasks: CPU time scales with the task's FLOPs
    est_s = 0.0
    for o in np.unique(ops):
        sel = ops[pick] == o
        us = r['task_us'][sel].astype(np.float64)
        if fl[pick][sel].sum() > 0:
            est_s += fl[ops == o].sum() * us.sum() / fl[pick][sel].sum() / 1e6
        else:
            est_s += (ops == o).sum() * us.mean() / 1e6
    return {'value': round(float(est_s) * 1e3, 1), 'unit': 'ms/step', 'cores': 1, 'kind': 'port',
            'sample': f'C++ oracle (restated reference CPU VM + ops, 1 thread) on {len(pick)} tasks of the same step graph '
                      f'({per_op} per operator, {r["seconds"]:.1f} s), scaled to the {lb.ntasks} tasks by FLOPs (GEMM, attention) or task count'}


def bench_sched():
    """Dependent-hop latency (a chain of noops) and fan-out/fan-in cost (wide noop phases)."""
    from kvm_amd.workloads import Builder, Workload
    b = Builder()
    prev = []
    for i in range(2000):
        prev = [b.task('noop', after=prev)]
    ex, lb = build_executor(Workload(b.spec()))
    _, ms, _ = time_steps(ex, 5, 2)
    hop_us = ms * 1e3 / 2000
    ex.close()
    b = Builder()
    prev = []
    for p in range(50):
        prev = [b.task('noop', after=prev) for _ in range(512)]
        prev = [b.task('noop', after=prev)]
    ex, lb = build_executor(Workload(b.spec()))
    _, ms2, _ = time_steps(ex, 5, 2)
    ex.close()
    out = {'hop_us': round(hop_us, 3), 'phase_us_512wide': round(ms2 * 1e3 / 50, 2), 'tasks_per_s_wide': round(50 * 513 / (ms2 / 1e3))}
    log(f'  sched: {hop_us:.2f} us per dependent hop; 512-wide noop phase + join: {out["phase_us_512wide"]} us')
    return out


def hbm_traffic(key):
    """HBM bytes per launch of the persistent kernel for a workload, from the committed counter summary
    (profiles/hbm_traffic.json: rocprofv3 FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by the same counter's
    reading for a plain copy of known size); None when the summary has no entry."""
    path = Path(__file__).resolve().parent / 'profiles' / 'hbm_traffic.json'
    try:
        return json.loads(path.read_text())[key]['bytes_per_launch']
    except (OSError, KeyError, ValueError):
        return None


def copy_probe(mib):
    """One plain copy kernel over `mib` MiB (reads mib MiB, writes mib MiB; the library's kvm_copy_probe): a dispatch
    whose HBM traffic is known, against which the byte counters of the executor's dispatches are calibrated."""
    from kvm_amd import executor
    executor.copy_probe(mib << 20)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--workload', default='all', choices=['all', 'gpt162m', 'decode', 'sched'])
    ap.add_argument('--decode-batch', default='1,8')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--copy-probe', type=int, default=0, metavar='MIB',
                    help='after the runs, one plain device copy of MIB MiB (reference dispatch for the HBM byte counters)')
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
    if a.workload in ('all', 'gpt162m'):
        extra['gpt162m'] = bench_gpt(a.steps, a.warmup, cpu)
    if a.workload in ('all', 'decode'):
        extra['decode'] = [bench_decode(int(bs), a.steps, a.warmup, cpu) for bs in a.decode_batch.split(',')]
    if 'gpt162m' in extra:
        g = extra['gpt162m']
        result.update({'value': g['ms_per_step'], 'unit': 'ms/step', 'higher_is_better': False, 'ms_per_step': g['ms_per_step'],
                       'dtype': 'bf16', 'config': {'workload': 'gpt-162m training step (12L d768 T1024 B4 V50304, tied, bf16 storage, '
                                                               'fp32 master AdamW)', 'global_batch': 4, 'seq_len': 1024},
                       'roofline': {'bound': 'mfma', 'achieved': g['tflops'], 'peak': BF16_PEAK_TFLOPS, 'unit': 'TFLOP/s',
                                    'frac': g['mfma_frac_step'], 'traffic': None}})
        if 'cpu_baseline' in g:
            result['cpu_baseline'] = g['cpu_baseline']
    elif 'decode' in extra:
        d = extra['decode'][0]
        result.update({'value': d['tok_s'], 'unit': 'tok/s', 'higher_is_better': True, 'ms_per_step': d['ms_per_token_step'],
                       'dtype': 'bf16', 'config': {'workload': f'qwen3-8b-shape decode, batch {d["batch"]}, 4096-token KV cache'},
                       'roofline': {'bound': 'hbm', 'achieved': d['hbm_gbs'], 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                                    'frac': d['hbm_frac'], 'traffic': None}})
        if 'cpu_baseline' in d:
            result['cpu_baseline'] = d['cpu_baseline']
    if 'roofline' in result:
        result['roofline']['traffic'] = hbm_traffic('gpt162m' if 'gpt162m' in extra else f'decode_b{extra["decode"][0]["batch"]}')
    result.update(extra)
    if a.copy_probe:
        copy_probe(a.copy_probe)
    print(json.dumps(result))


if __name__ == '__main__':
    main()
