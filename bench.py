#!/usr/bin/env python3
"""Benchmark of the MI355X task-graph executor on BASELINE.json's headline configurations.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|gpt162m|decode|sched|tiny|mlp8|gpt355m]
                    [--no-cpu-baseline]

A "step" is one run of the workload's task graph (one persistent-kernel launch): one GPT-162M training step
(forward + backward + AdamW), or one Qwen3-8B-shape greedy decode token for every sequence of the batch. The other
BASELINE configurations are reported beside the headline: tiny GPT (10 steps per graph) and the eight MLPs (50 steps
per graph) as time per training step and worker-busy fraction, GPT-355M f32 as step time against the fp32 peak. Inputs and
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
FP32_PEAK_TFLOPS = 157.3       # MI355X dense fp32 (matrix)
CPU_THREADS = int(os.environ.get('KVM_CPU_THREADS', '16'))   # oracle worker threads for the CPU baseline (the box's CPU share)
METRIC = 'GPT-162M train step ms; Qwen3-8B-shape decode tok/s + HBM GB/s fraction'


def log(*a):
    print(*a, file=sys.stderr, flush=True)


PATH_NAMES = {0: 'dynamic', 1: 'static'}


def build_executor(w, trace=False, blocks=0, path=2):
    """Executor with the workload's buffers and graph submitted. path 2 (auto): the static path for graphs of short tasks
    (mean estimated task cost at most KVM_STATIC_MAX_MEAN_US), the dynamic scheduler otherwise."""
    from kvm_amd import bundle as bl
    from kvm_amd import compiler
    from kvm_amd.executor import Executor
    t0 = time.perf_counter()
    lb = bl.load(compiler.compile_spec(w.spec))
    t1 = time.perf_counter()
    ex = Executor(num_vars=max(1, len(lb.metadata['variables'])), trace=trace, timeout_s=60.0, blocks=blocks, path=path)
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
    out = {'batch': batch, 'path': PATH_NAMES.get(ex.path()), 'ms_per_token_step': round(ms, 4), 'kernel_ms': round(kms, 4), 'tok_s': round(batch * 1e3 / ms, 2),
           'hbm_gbs': round(gbs, 1), 'hbm_frac': round(gbs / HBM_PEAK_GBS, 4), 'bytes_per_step': byts, 'tasks': lb.ntasks}
    log(f'  decode batch {batch}: {ms:.3f} ms/step, {out["tok_s"]} tok/s, {gbs:.0f} GB/s ({out["hbm_frac"]:.1%} of peak)')
    ex.close()
    if cpu:
        out['cpu_baseline'] = cpu_decode(batch)
    return out


_INIT_CACHE = {}


def _oracle_time(w, threads, reuse=False):
    """Wall time of the oracle (C++ restatement of the reference CPU VM + ops) on a whole graph with `threads` workers.
    reuse: initial buffers with the same name, shape and initialiser are generated once and copied (graphs of 1 and 2
    layers, or two batch sizes, share most of their weights)."""
    import oracle
    from kvm_amd import bundle as bl
    from kvm_amd import compiler
    lb = bl.load(compiler.compile_spec(w.spec))
    init = []
    for m in lb.metadata['buffers']:
        ini = w.init_override.get(m['name'], m['init'])
        key = (m['name'], m['rows'], m['cols'], m['dtype'], json.dumps(ini, sort_keys=True))
        if not reuse:
            init.append(oracle.materialize(m, ini))
            continue
        if key not in _INIT_CACHE:
            _INIT_CACHE[key] = oracle.materialize(m, ini)
        init.append(_INIT_CACHE[key].copy())
    return oracle.run(lb, init, threads=threads)['seconds']


def _layer_fit(make, layers_full, threads):
    """CPU time of the full-depth graph from whole-graph oracle timings at 1 and 2 layers: t1 + (L - 1) * (t2 - t1)."""
    t1 = _oracle_time(make(1), threads, reuse=True)
    t2 = _oracle_time(make(2), threads, reuse=True)
    return t1 + (layers_full - 1) * max(t2 - t1, 0.0), t1, t2


def cpu_decode(batch):
    """CPU reference time of one decode step: the oracle on the whole 36-layer graph (weights materialised outside the
    timed region)."""
    from kvm_amd.workloads import qwen3
    t = _oracle_time(qwen3.build(qwen3.Qwen3Config(batch=batch, max_new=4)), CPU_THREADS)
    return {'value': round(batch / t, 4), 'unit': 'tok/s', 'cores': CPU_THREADS, 'nproc': os.cpu_count(), 'kind': 'port',
            'sample': f'oracle (C++ restatement of the reference CPU VM + ops, {CPU_THREADS} worker threads) on the whole decode '
                      f'graph (36 layers + LM head, batch {batch}, 4096-token cache), one step: {t:.2f} s'}


GEMM_OPS = (34, 114, 122, 302, 304, 308)
ATTN_OPS = (45, 47, 48)


def gemm_task_flops(lb, executed_out=None):
    """FLOPs of every GEMM tile task (2*tm*tn*K clipped to the matrix; K is the task's own range for the split-K tiles
    of op 302) and of the attention tasks (their share of the causal attention's algorithmic FLOPs: fwd 2 products,
    bwd 5), from the bundle's own arguments. executed_out (array): the attention tasks' executed FLOPs (backward with
    the recomputed products)."""
    import numpy as np
    t, a = lb.tasks, lb.args
    fl = np.zeros(t.shape[0])
    for i in range(t.shape[0]):
        op, off = t[i, 0], t[i, 6]
        if op in GEMM_OPS:
            m0, n0, M, N, K, f = (int(x) for x in a[off + 6:off + 12])
            if op in (122, 308):
                tm, tn = 128, 256
            elif op == 304:
                tm, tn = 256, 256
            elif op == 302:
                tm, tn = (256, 256) if f & 64 else (128, 256)
            else:
                tm, tn = (256, 128) if f & 64 else (128, 128) if f & 32 else (64, 64)
            fl[i] = 2.0 * (min(M, m0 + tm) - m0) * (min(N, n0 + tn) - n0) * K
        elif op in (45, 47, 48):
            # argument positions of (q0 or k0, T, hd) in the registry signatures (mvm_ops_gpt.def)
            iq, it, ih = {45: (7, 8, 11), 47: (9, 10, 13), 48: (10, 11, 13)}[op]
            q0, T, hd = int(a[off + iq]), int(a[off + it]), int(a[off + ih])
            q1 = min(T, q0 + 128)
            if op == 48:   # keys [q0, q1) meet queries [k, T): sum over keys of (T - k)
                pairs = sum(T - k for k in range(q0, q1))
            else:
                pairs = sum(k + 1 for k in range(q0, q1))
            # per (query, key) pair the algorithmic work is forward 4 hd (S, P V) and backward 10 hd (S, dP, dV, dQ, dK:
            # 2.5x the forward); the backward tasks execute 6 hd (dQ: S, dP, dS K) and 8 hd (dK / dV: S, dP, P^T dO,
            # dS^T Q), recomputing S and dP in both, so the algorithmic 10 hd is split between them as 6:8
            executed = 2.0 * hd * pairs * {45: 2, 47: 3, 48: 4}[op]
            fl[i] = executed if op == 45 else executed * 10.0 / 14.0
            if executed_out is not None:
                executed_out[i] = executed
    return fl


def critical_path(lb, tr):
    """From a traced launch: the graph's critical path with the measured task durations and no hop latency (the
    longest chain of dependent task times: a lower bound on the launch for these task times), and the chain the launch
    actually ran (from the last task to finish, each step to the predecessor that finished last): its task count, the
    time its tasks ran and the time they waited (dependency release, queueing, dispatch). Times in us."""
    import numpy as np
    st, en = tr['start'].astype(np.int64), tr['end'].astype(np.int64)
    t0 = int(st.min())
    dur = (en - st) / 100.0
    n = lb.ntasks
    off, cnt = lb.tasks[:, 1], lb.tasks[:, 2]
    ef = np.zeros(n)
    rel = np.zeros(n)
    last = np.full(n, -1)
    for i in np.argsort(st, kind='stable'):          # start order is a topological order of the executed graph
        ef[i] += dur[i]
        e = (en[i] - t0) / 100.0
        for j in lb.succ[off[i]:off[i] + cnt[i]]:
            if ef[i] > ef[j]:
                ef[j] = ef[i]
            if e > rel[j]:
                rel[j], last[j] = e, i
    chain, i = [], int(np.argmax(en))
    while i >= 0:
        chain.append(i)
        i = int(last[i])
    run = float(dur[chain].sum())
    span = (int(en.max()) - t0) / 100.0
    return {'span_us': round(span, 1), 'critical_path_us': round(float(ef.max()), 1), 'chain_tasks': len(chain),
            'chain_running_us': round(run, 1), 'chain_waiting_us': round(span - run, 1)}


def bench_gpt(steps, warmup, cpu):
    import numpy as np
    from kvm_amd.workloads import gpt
    c = gpt.GPTConfig()
    log('gpt-162m bf16 training step: building')
    w = gpt.build(c)
    ex, lb = build_executor(w, trace=True)
    check = first_step_invariants(ex, lb, c.vocab)
    ex.set_trace(False)                   # timed runs untraced; one traced run afterwards for the per-task statistics
    ms, kms, res = time_steps(ex, steps, warmup)
    flops = w.info['flops']['total']
    tflops = flops / (kms / 1e3) / 1e12
    ex.set_trace(True)
    ex.relaunch()
    res = ex.finish()
    # MFMA utilisation inside the GEMM / attention tasks, from the traced run's per-task record
    tr = ex.trace()
    dur = (tr['end'] - tr['start']).astype(np.float64) / 100e6     # s (wall_clock64 at 100 MHz)
    fx = np.zeros(lb.ntasks)
    fl = gemm_task_flops(lb, fx)
    ops = lb.tasks[:, 0]
    gm = np.isin(ops, GEMM_OPS); at = np.isin(ops, ATTN_OPS)
    per_cu = BF16_PEAK_TFLOPS / 256 * 1e12
    in_task = {'gemm': float(fl[gm].sum() / dur[gm].sum() / per_cu), 'attention': float(fl[at].sum() / dur[at].sum() / per_cu),
               'attention_executed': float(fx[at].sum() / dur[at].sum() / per_cu)}
    busy = float(dur.sum() / (res['grid'] * (tr['end'].max() - tr['start'].min()) / 100e6))
    crit = critical_path(lb, tr)
    names = [m['name'] for m in lb.metadata['buffers']]
    loss = float(ex.read('loss')[0])
    out = {'ms_per_step': round(ms, 3), 'path': PATH_NAMES.get(ex.path()), 'kernel_ms': round(kms, 3), 'tflops': round(tflops, 1), 'mfma_frac_step': round(tflops / BF16_PEAK_TFLOPS, 4),
           'mfma_frac_in_gemm_tasks': round(in_task['gemm'], 4), 'mfma_frac_in_attention_tasks': round(in_task['attention'], 4),
           'mfma_frac_in_attention_tasks_executed': round(in_task['attention_executed'], 4),
           'worker_busy_frac': round(busy, 4), 'tasks': lb.ntasks, 'edges': int(lb.succ.size), 'loss_after': loss,
           'step_flops': flops, 'params': w.info['params'], 'first_step_check': check, 'critical_path_traced': crit}
    log(f'  gpt-162m: {ms:.2f} ms/step (persistent kernel {kms:.2f} ms), {tflops:.1f} TFLOP/s ({tflops / BF16_PEAK_TFLOPS:.1%} of bf16 peak); in-task MFMA: '
        f'GEMM {in_task["gemm"]:.1%}, attention {in_task["attention"]:.1%}; workers busy {busy:.1%}; loss {loss:.4f}')
    ex.close()
    if cpu:
        out['cpu_baseline'] = cpu_gpt_whole()
    return out


# Operator classes of the GPT step for the per-class byte-counter attribution (--phases).
PHASE_OPS = {
    'gemm': (34, 114, 122, 302, 303, 304, 308),
    'attention': (45, 46, 47, 48),
    'cross_entropy': (51, 52, 53, 127),
    'optimizer': (54, 55, 56, 59, 60, 113, 115, 116, 305),
}


def phase_subgraph(lb, keep):
    """The tasks of lb selected by the boolean mask `keep`, with the edges among them (edges through dropped tasks
    are lost, so kept tasks may run in another order: for byte counts, not results) and no version waits or
    publications."""
    import numpy as np
    from kvm_amd import bundle as bl
    idx = np.nonzero(keep)[0]
    new = -np.ones(lb.ntasks, np.int64)
    new[idx] = np.arange(idx.size)
    t = lb.tasks[idx].copy()
    succ, indeg = [], np.zeros(idx.size, np.int64)
    for k, u in enumerate(idx):
        s = [int(new[v]) for v in lb.succ[lb.tasks[u, 1]:lb.tasks[u, 1] + lb.tasks[u, 2]] if new[v] >= 0]
        t[k, 1], t[k, 2] = len(succ), len(s)
        succ += s
        for v in s:
            indeg[v] += 1
    t[:, 3] = indeg
    t[:, 8], t[:, 9], t[:, 10], t[:, 11] = -1, 0, -1, 0
    meta = dict(lb.metadata, variables=[], reads=[], publishers=[])
    return bl.LoadedBundle(meta, t, np.array(succ or [0], np.int32)[:len(succ)], lb.args, lb.root)


def bench_phases():
    """One launch per operator class of the GPT-162M step (its tasks alone, see phase_subgraph), after one launch of
    the whole step, in this order: step, gemm, attention, cross_entropy, optimizer, other. A counter run of rocprofv3
    lists the dispatches in the same order; the summaries in profiles/ attribute the step's HBM bytes with them."""
    import numpy as np
    from kvm_amd.executor import Executor
    from kvm_amd.workloads import gpt
    w = gpt.build(gpt.GPTConfig())
    ex, lb = build_executor(w, trace=False)
    ex.relaunch(); ex.finish()
    ops = lb.tasks[:, 0]
    out = {'step': {'tasks': lb.ntasks}}
    ex.close()
    used = np.zeros(lb.ntasks, bool)
    for name in (*PHASE_OPS, 'other'):
        keep = np.isin(ops, PHASE_OPS[name]) if name != 'other' else ~used
        used |= keep
        sub = phase_subgraph(lb, keep)
        ex = Executor(num_vars=1, trace=False, timeout_s=60.0, path=0)
        for m in lb.metadata['buffers']:
            ex.add_buffer(m['name'], m['rows'], m['cols'], m['dtype'], init=w.init_override.get(m['name'], m['init']), root=lb.root)
        ex.submit(sub)
        res = ex.run()
        out[name] = {'tasks': int(keep.sum()), 'kernel_ms': round(res['kernel_ms'], 3)}
        log(f'  phase {name}: {int(keep.sum())} tasks, {res["kernel_ms"]:.3f} ms')
        ex.close()
    return out


def first_step_invariants(ex, lb, vocab):
    """Full-size sanity of the first training step (untimed): the loss of a randomly initialised model is close to
    ln V, and every weight gradient is finite and nonzero. Raises when not."""
    import numpy as np
    ex.relaunch()
    ex.finish()
    loss = float(ex.read('loss')[0])
    if not abs(loss - np.log(vocab)) <= 0.05 * np.log(vocab):
        raise RuntimeError(f'first-step loss {loss} is not near ln V = {np.log(vocab):.3f}')
    grads = [m['name'] for m in lb.metadata['buffers'] if m['name'].startswith('d.w')]
    for g in grads:
        x = ex.read(g)
        if not np.isfinite(x).all() or not np.abs(x).max() > 0:
            raise RuntimeError(f'gradient {g} is not finite and nonzero')
    return {'loss_step1': round(loss, 4), 'ln_vocab': round(float(np.log(vocab)), 4), 'grads_finite_nonzero': len(grads)}


def cpu_gpt_whole():
    """CPU reference time of the GPT-162M step: the oracle on the whole 12-layer step graph."""
    from kvm_amd.workloads import gpt
    t = _oracle_time(gpt.build(gpt.GPTConfig()), CPU_THREADS)
    return {'value': round(t * 1e3, 1), 'unit': 'ms/step', 'cores': CPU_THREADS, 'nproc': os.cpu_count(), 'kind': 'port',
            'sample': f'oracle (C++ restatement of the reference CPU VM + ops, {CPU_THREADS} worker threads) on the whole step graph '
                      f'(12 layers, forward + backward + AdamW), one step: {t:.1f} s'}


def cpu_gpt(layers=12, dtype='bf16', **kw):
    """CPU reference time of a GPT step from whole-graph oracle timings at full width and 1 and 2 layers (GPT-355M, whose
    whole 24-layer f32 graph would take minutes on the oracle)."""
    from kvm_amd.workloads import gpt
    make = (lambda L: gpt.build(gpt.GPTConfig(layers=L, **kw))) if dtype == 'bf16' else (lambda L: gpt.build(gpt.GPTConfig.gpt355m(layers=L, **kw)))
    est, t1, t2 = _layer_fit(make, layers, CPU_THREADS)
    return {'value': round(est * 1e3, 1), 'unit': 'ms/step', 'cores': CPU_THREADS, 'nproc': os.cpu_count(), 'kind': 'port',
            'sample': f'oracle (C++ restatement of the reference CPU VM + ops, {CPU_THREADS} worker threads) timed on whole full-width '
                      f'step graphs of 1 and 2 layers: {t1:.1f} s and {t2:.1f} s; {layers} layers = t1 + {layers - 1} (t2 - t1)'}


def bench_small(name, w, steps_in_graph, reps, warmup, cpu):
    """A graph that holds several training steps (C1, C2): time per step = launch time / steps in the graph; worker-busy
    fraction = summed task time / (workers x span) from the last launch's trace."""
    import numpy as np
    log(f'{name}: building')
    ex, lb = build_executor(w, trace=True)
    ex.set_trace(False)
    ms, kms, res = time_steps(ex, reps, warmup)
    ex.set_trace(True)
    ex.relaunch()
    res = ex.finish()
    tr = ex.trace()
    dur = (tr['end'] - tr['start']).astype(np.float64)
    span = float(tr['end'].max() - tr['start'].min())
    busy = float(dur.sum() / (res['grid'] * span))
    crit = critical_path(lb, tr)
    out = {'us_per_step': round(kms * 1e3 / steps_in_graph, 2), 'path': PATH_NAMES.get(ex.path()), 'launch_ms': round(kms, 4), 'steps_in_graph': steps_in_graph,
           'worker_busy_frac': round(busy, 4), 'tasks': lb.ntasks, 'edges': int(lb.succ.size), 'critical_path_traced': crit}
    log(f'  {name}: {out["us_per_step"]} us/step ({steps_in_graph} steps per launch, {lb.ntasks} tasks), workers busy {busy:.1%}; traced launch '
        f'{crit["span_us"]} us, critical path of its task times {crit["critical_path_us"]} us, the chain it ran: {crit["chain_tasks"]} tasks, '
        f'{crit["chain_running_us"]} us running, {crit["chain_waiting_us"]} us waiting')
    ex.close()
    if cpu:
        t = _oracle_time(w, CPU_THREADS)
        out['cpu_baseline'] = {'value': round(t * 1e6 / steps_in_graph, 1), 'unit': 'us/step', 'cores': CPU_THREADS, 'nproc': os.cpu_count(),
                               'kind': 'port', 'sample': f'oracle on the whole graph ({steps_in_graph} steps, {CPU_THREADS} threads): {t:.2f} s'}
    return out


def bench_gpt355m(steps, warmup, cpu):
    """GPT-355M shape, f32 storage and math (fp32 GEMM tiles), batch 4."""
    from kvm_amd.workloads import gpt
    c = gpt.GPTConfig.gpt355m()
    log('gpt-355m f32 training step: building')
    w = gpt.build(c)
    ex, lb = build_executor(w, trace=False)
    check = first_step_invariants(ex, lb, c.vocab)
    ms, kms, res = time_steps(ex, steps, warmup)
    flops = w.info['flops']['total']
    tflops = flops / (kms / 1e3) / 1e12
    out = {'ms_per_step': round(ms, 2), 'path': PATH_NAMES.get(ex.path()), 'kernel_ms': round(kms, 2), 'tflops': round(tflops, 2), 'fp32_frac': round(tflops / FP32_PEAK_TFLOPS, 4),
           'step_flops': flops, 'params': w.info['params'], 'tasks': lb.ntasks, 'first_step_check': check}
    log(f'  gpt-355m f32: {ms:.1f} ms/step, {tflops:.1f} TFLOP/s ({tflops / FP32_PEAK_TFLOPS:.1%} of the fp32 peak)')
    ex.close()
    if cpu:   # batch 1 graphs, times 4 (every phase of the step is linear in the batch at fixed T)
        cb = cpu_gpt(layers=24, dtype='f32', batch=1)
        cb['value'] = round(cb['value'] * 4, 1)
        cb['sample'] += ', at batch 1, x4 for batch 4'
        out['cpu_baseline'] = cb
    return out


def bench_sched():
    """Dependent-hop latency (a chain of noops) and fan-out/fan-in cost (wide noop phases)."""
    from kvm_amd.workloads import Builder, Workload
    b = Builder()
    prev = []
    for i in range(2000):
        prev = [b.task('noop', after=prev)]
    ex, lb = build_executor(Workload(b.spec()), path=0)
    _, ms, _ = time_steps(ex, 5, 2)
    hop_us = ms * 1e3 / 2000
    ex.close()
    b = Builder()
    prev = []
    for p in range(50):
        prev = [b.task('noop', after=prev) for _ in range(512)]
        prev = [b.task('noop', after=prev)]
    ex, lb = build_executor(Workload(b.spec()), path=0)
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
    for m in str(mib).split(','):
        executor.copy_probe(int(m) << 20)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--workload', default='all', choices=['all', 'gpt162m', 'decode', 'sched', 'tiny', 'mlp8', 'gpt355m', 'phases'])
    ap.add_argument('--decode-batch', default='1,8')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--copy-probe', default='', metavar='MIB[,MIB..]',
                    help='after the runs, plain device copies of these sizes (reference dispatches for the HBM byte counters)')
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
    _INIT_CACHE.clear()
    if a.workload in ('all', 'tiny'):
        from kvm_amd.workloads import gpt
        extra['tiny_gpt'] = bench_small('tiny gpt f32 (C1, 10 steps per graph)', gpt.build(gpt.GPTConfig.tiny()), 10, a.steps, a.warmup, cpu)
    if a.workload in ('all', 'mlp8'):
        from kvm_amd.workloads import mlp
        extra['mlp8'] = bench_small('8 MLPs f32 (C2, 50 steps per graph)', mlp.build(), 50, max(3, a.steps // 4), 1, cpu)
    if a.workload in ('all', 'gpt355m'):
        extra['gpt355m'] = bench_gpt355m(max(3, a.steps // 4), 1, cpu)
    if a.workload == 'phases':
        extra['phases'] = bench_phases()
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
    if 'roofline' in result and a.workload != 'phases':
        result['roofline']['traffic'] = hbm_traffic('gpt162m' if 'gpt162m' in extra else f'decode_b{extra["decode"][0]["batch"]}')
    result.update(extra)
    if a.copy_probe:
        copy_probe(a.copy_probe)
    print(json.dumps(result))


if __name__ == '__main__':
    main()
