"""Scheduler classes in stream mode on the GPU (reference: the class rings of the admitter path, include/mvm_sched.cuh
mvm_enqueue / mvm_scan / mvm_claim, where a class is a workload_id and bundles of several workloads are admitted while
the persistent kernel runs). Each queue group holds one ring per class; the class policy (caps, weights,
reservations, EDF, inheritance, the static split) works on the rings as on the launch-mode queues, and deadlines count
from the admission of the task's window. Results do not depend on the policy; the guarantees are checked from the
per-task trace (window slots are not reused in these tests, so every task keeps its trace record)."""
import time

import numpy as np
import pytest

import oracle
from gpu_check import compare_run
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.executor import (SCHED_DYNAMIC, SCHED_F_GUARANTEE, SCHED_F_INHERIT, SCHED_STATIC, TRACE_BOOST, TRACE_MISSED, Executor,
                              KvmError)

pytestmark = pytest.mark.gpu


def spin_bundle(n, us, cls, deadline_us=None, variables=(), pub=None, wait=None):
    """n independent spin tasks of class `cls`; optionally the first publishes `pub` or waits for version 1 of `wait`."""
    ts = []
    for k in range(n):
        t = {'id': f't{k}', 'op': 'spin', 'args': {'us': us}}
        if deadline_us is not None:
            t['deadline_us'] = deadline_us
        if k == 0 and pub:
            t['publishes'] = pub
        ts.append(t)
    spec = {'buffers': [{'name': 'x', 'rows': 4}], 'graphs': [{'name': 'g', 'tasks': ts}]}
    if variables:
        spec['variables'] = list(variables)
    b = bl.load(compiler.compile_spec(spec))
    b.tasks[:, 12] = cls
    if wait is not None:
        b.tasks[0, 8], b.tasks[0, 9] = wait, 1
    return b


def stream_executor(b, classes, mode=SCHED_DYNAMIC, flags=None, **kw):
    ex = Executor(num_vars=max(1, len(b.metadata['variables'])), **kw)
    for m in b.metadata['buffers']:
        ex.add_buffer(m['name'], m['rows'], m['cols'], m['dtype'], init=m['init'], root=b.root)
    for v in b.metadata['variables']:
        ex.set_version(v['id'], v['base_version'])
    ex.meta = b.metadata
    ex.set_classes(mode, classes)
    if flags is not None:
        ex.set_sched_flags(flags)
    return ex


def max_overlap(tr, mask):
    ev = sorted([(s, 1) for s in tr['start'][mask]] + [(e, -1) for e in tr['end'][mask]], key=lambda x: (x[0], x[1]))
    cur = best = 0
    for _, d in ev:
        cur += d
        best = max(best, cur)
    return best


def slots_of(wids, n, window_tasks):
    """Trace indices of the first n tasks of each window id (slot = (wid % window_cap) * window_tasks + i)."""
    return np.concatenate([np.arange(n) + w * window_tasks for w in wids])


def test_stream_cap_bounds_a_class_and_every_task_runs_once():
    """Eight bundles of 32 spin tasks, alternating classes, admitted while the kernel runs: class 0 capped at three
    running tasks (at every instant, from the trace and the class's own maximum), class 1 uncapped runs more at once;
    every task runs exactly once and is counted in its class."""
    nb, n = 8, 32
    bundles = [spin_bundle(n, 20, k % 2) for k in range(nb)]
    ex = stream_executor(bundles[0], [{'max_cta': 3}, {}], window_cap=nb, window_tasks=n, window_edges=4, timeout_s=10.0)
    print('stream classes: cap 3, 8 bundles', flush=True)
    ex.start()
    wids = [ex.submit(b) for b in bundles]
    res = ex.finish()
    assert res['err_code'] == 0 and res['done'] == nb * n
    tr = ex.trace()
    idx = slots_of(wids, n, n)
    assert (tr['exec_count'][idx] == 1).all()
    cls = np.repeat([k % 2 for k in range(nb)], n)
    t = tr[idx]
    peak0, peak1 = max_overlap(t, cls == 0), max_overlap(t, cls == 1)
    st = ex.class_stats(2)
    print('peaks', peak0, peak1, 'max_running', st['max_running'].tolist(), flush=True)
    assert 1 <= peak0 <= 3 and st['max_running'][0] <= 3
    assert peak1 > 3
    assert st['tasks'].tolist() == [nb * n // 2] * 2
    ex.close()


def test_stream_inheritance_runs_a_throttled_publisher_admitted_later():
    """A class-0 task waits for version 1 of v; the publisher comes in a later bundle of class 1, which may not run at all
    (max_cta 0): inheritance boosts class 1 and the waiter runs after it. Without inheritance the waiter parks for ever
    and the kernel ends with the stall TIMEOUT."""
    reader = spin_bundle(2, 10, 0, variables=['v'], wait=0)
    pub = spin_bundle(1, 30, 1, variables=['v'], pub='v')
    assert pub.tasks[0, 10] == 0 and pub.tasks[0, 11] == 1
    ex = stream_executor(reader, [{}, {'max_cta': 0}], flags=SCHED_F_GUARANTEE | SCHED_F_INHERIT, window_cap=4, window_tasks=4,
                         window_edges=4, timeout_s=10.0)
    print('stream classes: inheritance', flush=True)
    ex.start()
    w0 = ex.submit(reader)
    time.sleep(0.05)
    w1 = ex.submit(pub)
    res = ex.finish()
    assert res['err_code'] == 0 and res['done'] == 3
    tr = ex.trace()
    p, r = w1 * 4, w0 * 4
    assert tr['how'][p] & TRACE_BOOST
    assert tr['end'][p] <= tr['start'][r]
    assert ex.class_stats(2)['boost_starts'][1] == 1
    assert ex.versions(1)[0] == 1
    ex.close()
    ex = stream_executor(reader, [{}, {'max_cta': 0}], flags=SCHED_F_GUARANTEE, window_cap=4, window_tasks=4, window_edges=4,
                         timeout_s=0.5)
    ex.start()
    ex.submit(reader)
    ex.submit(pub)
    res = ex.finish(check=False)
    assert res['err_code'] == 15, res          # TIMEOUT
    ex.close()


def test_stream_deadlines_count_from_admission():
    """A bundle admitted 200 ms after the launch with 50 ms deadlines meets them (they count from its window's
    admission, not from the launch); a bundle whose 50 us tasks have 1 us deadlines misses every one."""
    first = spin_bundle(4, 10, 0)
    late = spin_bundle(16, 5, 0, deadline_us=50_000)
    tight = spin_bundle(8, 50, 1, deadline_us=1)
    ex = stream_executor(first, [{'urgent_us': 1000}, {}], window_cap=4, window_tasks=16, window_edges=4, timeout_s=10.0)
    print('stream classes: deadlines from admission', flush=True)
    ex.start()
    w0 = ex.submit(first)
    time.sleep(0.2)
    w1 = ex.submit(late)
    w2 = ex.submit(tight)
    res = ex.finish()
    assert res['err_code'] == 0 and res['done'] == 28
    st = ex.class_stats(2)
    assert st['missed'].tolist() == [0, 8], st
    tr = ex.trace()
    assert not (tr['how'][slots_of([w1], 16, 16)] & TRACE_MISSED).any()
    assert (tr['how'][slots_of([w2], 8, 16)] & TRACE_MISSED).all()
    assert w0 == 0
    ex.close()


def test_stream_static_split_keeps_classes_on_their_workers():
    """STATIC split 1:7 of 32 workers in stream mode: class 0 runs only on workers 0-3 (fewer than the queue groups of
    the shared mode, so its rings must be visible to those four), class 1 only on 4-31."""
    bundles = [spin_bundle(64, 5, k % 2) for k in range(6)]
    ex = stream_executor(bundles[0], [{'share': 1}, {'share': 7}], mode=SCHED_STATIC, window_cap=6, window_tasks=64, window_edges=4,
                         timeout_s=10.0, blocks=32)
    print('stream classes: static split', flush=True)
    ex.start()
    wids = [ex.submit(b) for b in bundles]
    res = ex.finish()
    assert res['err_code'] == 0 and res['done'] == 6 * 64
    tr = ex.trace()[slots_of(wids, 64, 64)]
    cls = np.repeat([k % 2 for k in range(6)], 64)
    assert tr['block'][cls == 0].max() < 4 and tr['block'][cls == 1].min() >= 4
    assert len(np.unique(tr['block'][cls == 1])) > 8
    ex.close()


def test_stream_classes_results_match_the_oracle():
    """Tiny GPT, 2 training steps, one bundle cut into windows of 256 tasks, its tasks split over three classes
    (task index mod 3; dependencies cross classes) with a cap, a reservation and unequal weights: results as the
    oracle's; a task of an unknown class is refused before anything is staged."""
    from kvm_amd.workloads import gpt
    w = gpt.build(gpt.GPTConfig.tiny(steps=2))
    b = bl.load(compiler.compile_spec(w.spec))
    t = b.tasks
    topo = all(int(s) > u for u in range(t.shape[0]) for s in b.succ[t[u, 1]:t[u, 1] + t[u, 2]])
    if not topo:
        pytest.skip('the compiled bundle is not in topological order')
    b.tasks[:, 12] = np.arange(b.ntasks) % 3
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in b.metadata['buffers']]
    ref = oracle.run(b, [x.copy() for x in init], threads=16)
    ex = Executor(num_vars=max(1, len(b.metadata['variables'])), window_cap=4, window_tasks=256, window_edges=4096, timeout_s=20.0)
    for m, x in zip(b.metadata['buffers'], init):
        ex.add_buffer(m['name'], m['rows'], m['cols'], m['dtype'], data=x)
    for v in b.metadata['variables']:
        ex.set_version(v['id'], v['base_version'])
    ex.meta = b.metadata
    ex.set_classes(SCHED_DYNAMIC, [{'max_cta': 8}, {'weight': 3, 'min_cta': 2}, {'weight': 1}])
    print(f'stream classes: tiny gpt, {b.ntasks} tasks over 3 classes', flush=True)
    ex.start()
    bad = spin_bundle(2, 1, 5)
    with pytest.raises(KvmError, match='workload_id'):
        ex.submit(bad)
    nw = ex.submit_stream(b, max_window_tasks=256)
    assert nw >= b.ntasks // 256
    res = ex.finish()
    assert res['err_code'] == 0 and res['done'] == b.ntasks
    st = ex.class_stats(3)
    assert st['tasks'].sum() == b.ntasks and st['max_running'][0] <= 8
    skip = tuple(m['name'] for m in b.metadata['buffers'] if m['name'].startswith(('bk.', 'd.bk.', 'm.bk.', 'v.bk.')))
    assert not compare_run(ex, b.metadata, ref, tol_f32=2e-4, skip=skip)
    ex.close()


def test_stream_task_affinity_keeps_a_chain_on_its_worker():
    """Affinity window 1 s in stream mode: each admitted chain of 8 dependent spin tasks runs on one worker."""
    ts = [{'id': f'k{k}', 'op': 'spin', 'args': {'us': 10}, **({'after': [f'k{k - 1}']} if k else {})} for k in range(8)]
    b = bl.load(compiler.compile_spec({'buffers': [{'name': 'x', 'rows': 4}], 'graphs': [{'name': 'g', 'tasks': ts}]}))
    ex = stream_executor(b, [{}], window_cap=4, window_tasks=8, window_edges=8, timeout_s=10.0)
    ex.set_affinity(1_000_000)
    print('stream classes: task affinity', flush=True)
    ex.start()
    wids = [ex.submit(b) for _ in range(4)]
    res = ex.finish()
    assert res['err_code'] == 0 and res['done'] == 32
    tr = ex.trace()
    blocks = [len(np.unique(tr['block'][w * 8:(w + 1) * 8])) for w in wids]
    print('workers per chain', blocks, flush=True)
    assert blocks == [1] * 4
    ex.close()
