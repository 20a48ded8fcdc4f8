"""GPU tests of the scheduler classes (kvm_set_classes; reference policy: include/mvm_sched.cuh mvm_pop, tiers of
reservation, EDF and weighted fair sharing, and the static split). Results do not depend on the class policy; the
policy's own guarantees are checked from the per-task trace: a cap bounds the class's concurrently running tasks at
every instant, weights split worker-time while both classes have ready work, a reservation keeps a low-weight class
served, the EDF tier starts deadline tasks first in deadline order, the static split keeps each class on its own
workers, and deadline misses are counted."""
import json

import numpy as np
import pytest

import oracle
from conftest import GOLDEN
from gpu_check import check_schedule, compare_run
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.executor import (SCHED_DYNAMIC, SCHED_STATIC, TRACE_MISSED, TRACE_RESV, TRACE_URGENT, UNLIMITED, Executor,
                              KvmError)

pytestmark = pytest.mark.gpu


def spin_spec(classes, buf_rows=4):
    """One graph per class: classes[c] = list of (spin us, deadline_us or None); every task a root."""
    graphs = []
    for c, tasks in enumerate(classes):
        ts = []
        for k, (us, dl) in enumerate(tasks):
            t = {'id': f't{k}', 'op': 'spin', 'args': {'us': us}}
            if dl is not None:
                t['deadline_us'] = dl
            ts.append(t)
        graphs.append({'name': f'c{c}', 'tasks': ts})
    return {'buffers': [{'name': 'x', 'rows': buf_rows}], 'graphs': graphs}


def run(spec, mode, classes, **kw):
    b = bl.load(compiler.compile_spec(spec))
    ex = Executor.from_bundle(b, **kw)
    ex.set_classes(mode, classes)
    ex.run()
    tr = check_schedule(ex, b)
    st = ex.class_stats(len(classes))
    cls = b.tasks[:, 12]
    return ex, b, tr, st, cls


def max_overlap(tr, mask):
    """Largest number of the masked tasks whose [start, end) intervals overlap at one instant."""
    ev = sorted([(s, 1) for s in tr['start'][mask]] + [(e, -1) for e in tr['end'][mask]], key=lambda x: (x[0], x[1]))
    cur = best = 0
    for _, d in ev:
        cur += d
        best = max(best, cur)
    return best


def busy_until(tr, mask, t_end):
    s, e = tr['start'][mask].astype(np.int64), tr['end'][mask].astype(np.int64)
    return np.clip(np.minimum(e, t_end) - s, 0, None).sum()


def test_results_do_not_depend_on_the_class_policy():
    """A small GPT training step (bf16) with one class and with the static split gives the same bits as the default
    scheduler; the two-graph golden case (training + inference, versioned weights) matches the oracle with two classes."""
    from kvm_amd.workloads import gpt
    c = gpt.GPTConfig(layers=2, d=128, heads=2, T=128, vocab=512, ffn=256, batch=2, steps=1, tasks_target=32)
    w = gpt.build(c)
    lb = bl.load(compiler.compile_spec(w.spec))
    init = [bl.materialize({**m, 'init': w.init_override.get(m['name'], m['init'])}) for m in lb.metadata['buffers']]
    outs = []
    for mode, classes in ((None, None), (SCHED_DYNAMIC, [{'weight': 3, 'max_cta': 40, 'min_cta': 4}]),
                          (SCHED_STATIC, [{'share': 1}])):
        print('gpt step, classes', mode, flush=True)
        ex = Executor.from_bundle(lb, buffers=init)
        if mode is not None:
            ex.set_classes(mode, classes)
        ex.run()
        check_schedule(ex, lb)
        outs.append({m['name']: ex.read_raw(m['name']).copy() for m in lb.metadata['buffers']})
        ex.close()
    for o in outs[1:]:
        for k in outs[0]:
            assert np.array_equal(outs[0][k], o[k]), k
    d = GOLDEN / 'live_training_inference'
    b = bl.load(compiler.compile_spec(json.loads((d / 'workload.json').read_text())))
    ref = oracle.run(b)
    print('golden live_training_inference, 2 classes', flush=True)
    ex = Executor.from_bundle(b)
    ex.set_classes(SCHED_DYNAMIC, [{'weight': 1}, {'weight': 5, 'urgent_us': 100}])
    ex.run()
    check_schedule(ex, b)
    assert compare_run(ex, b.metadata, ref) == []
    assert ex.class_stats(2)['tasks'].tolist() == [int((b.tasks[:, 12] == k).sum()) for k in range(2)]


def test_cap_bounds_running_tasks():
    print('cap 3 of 32 workers', flush=True)
    spec = spin_spec([[(20, None)] * 256, [(20, None)] * 256])
    ex, b, tr, st, cls = run(spec, SCHED_DYNAMIC, [{'weight': 1}, {'weight': 1, 'max_cta': 3}], blocks=32)
    assert max_overlap(tr, cls == 1) <= 3
    assert st['max_running'][1] == 3 and st['max_running'][0] > 3
    assert st['tasks'].tolist() == [256, 256]


def test_weights_split_worker_time():
    """Weights 1 : 3 over 32 workers; until the first class runs dry the busy time divides about 1 : 3."""
    print('weights 1:3', flush=True)
    spec = spin_spec([[(10, None)] * 1500, [(10, None)] * 1500])
    ex, b, tr, st, cls = run(spec, SCHED_DYNAMIC, [{'weight': 1}, {'weight': 3}], blocks=32)
    t_end = min(tr['end'][cls == 0].max(), tr['end'][cls == 1].max())
    b0, b1 = busy_until(tr, cls == 0, t_end), busy_until(tr, cls == 1, t_end)
    share = b1 / (b0 + b1)
    print('class 1 share', share)
    assert 0.65 <= share <= 0.85, share


def test_reservation_keeps_a_light_class_served():
    """Class 1 weighs 1000 times less, so fair sharing alone would almost starve it; min_cta 8 keeps about 8 of its
    tasks running while it has ready work."""
    print('reservation 8 of 32', flush=True)
    spec = spin_spec([[(10, None)] * 2000, [(10, None)] * 400])
    ex, b, tr, st, cls = run(spec, SCHED_DYNAMIC, [{'weight': 1000}, {'weight': 1, 'min_cta': 8}], blocks=32)
    t_end = tr['end'][cls == 1].max()
    assert t_end < tr['end'][cls == 0].max()          # the light class finished first
    b1 = busy_until(tr, cls == 1, t_end)
    t0 = tr['start'].min()
    assert b1 / (t_end - t0) >= 6.0, b1 / (t_end - t0)   # about 8 workers' worth
    assert st['resv_starts'][1] > 0 and (tr['how'][cls == 1] & TRACE_RESV).any()


def test_edf_tier_serves_deadlines_first_in_order():
    """8 workers; class 0 holds 400 tasks without deadlines, class 1 40 tasks, several per priority level, whose
    deadlines grow with the priority, all inside the EDF window. EDF compares the ready heads of the priority buckets
    (the reference rule: mvm_scan scores bucket heads, mvm_sched.cuh:155-190) of a worker's queue group (task t in
    group t % 8, one worker each here), so each worker runs its class-1 tasks first, earliest deadline first: the
    reverse of their priority order."""
    print('edf', flush=True)
    n1 = 40
    prios = [k % 20 for k in range(n1)]
    dls = [100_000 + 10_000 * p + k for k, p in enumerate(prios)]
    spec = spin_spec([[(20, None)] * 400, [(20, d) for d in dls]])
    for t, p in zip(spec['graphs'][1]['tasks'], prios):
        t['priority'] = p
    ex, b, tr, st, cls = run(spec, SCHED_DYNAMIC, [{'weight': 1}, {'weight': 1, 'urgent_us': 10_000_000}], blocks=8)
    assert st['urgent_starts'][1] == n1 and (tr['how'][cls == 1] & TRACE_URGENT).all()
    dl = np.full(len(cls), -1)
    dl[cls == 1] = dls
    for g in range(8):
        mine = np.arange(len(cls)) % 8 == g
        one = np.nonzero(mine & (cls == 1))[0]
        by_start = one[np.argsort(tr['start'][one])]
        assert (np.diff(dl[by_start]) > 0).all(), (g, dl[by_start], [prios[i - 400] for i in by_start])
        zero = mine & (cls == 0)
        assert tr['start'][one].max() < tr['start'][zero].min(), g


def test_missed_deadlines_are_counted():
    print('missed deadlines', flush=True)
    spec = spin_spec([[(50, 1)] * 16, [(5, 1_000_000)] * 16])
    ex, b, tr, st, cls = run(spec, SCHED_DYNAMIC, [{'weight': 1}, {'weight': 1}], blocks=4)
    assert st['missed'].tolist() == [16, 0]
    assert (tr['how'][cls == 0] & TRACE_MISSED).all() and not (tr['how'][cls == 1] & TRACE_MISSED).any()


def test_static_split_keeps_classes_on_their_workers():
    print('static split 1:3 of 32', flush=True)
    spec = spin_spec([[(5, None)] * 300, [(5, None)] * 300])
    ex, b, tr, st, cls = run(spec, SCHED_STATIC, [{'share': 1}, {'share': 3}], blocks=32)
    assert tr['block'][cls == 0].max() < 8 and tr['block'][cls == 1].min() >= 8
    assert len(np.unique(tr['block'][cls == 1])) > 8


def test_class_errors():
    spec = spin_spec([[(1, None)] * 4, [(1, None)] * 4])
    b = bl.load(compiler.compile_spec(spec))
    ex = Executor.from_bundle(b)
    with pytest.raises(KvmError, match='weight'):
        ex.set_classes(SCHED_DYNAMIC, [{'weight': 0}])
    with pytest.raises(KvmError, match='max_cta'):
        ex.set_classes(SCHED_DYNAMIC, [{'max_cta': 0}])
    ex.set_classes(SCHED_DYNAMIC, [{'weight': 1}])            # graph 1 has no class
    with pytest.raises(KvmError, match='workload_id'):
        ex.start()
    ex.close()
    ex = Executor.from_bundle(b, path=1)
    ex.set_classes(SCHED_DYNAMIC, [{}, {}])
    with pytest.raises(KvmError, match='dynamic path'):
        ex.start()
    ex.close()
    ex = Executor.from_bundle(b)
    ex.run()
    with pytest.raises(KvmError, match='before the first'):
        ex.set_classes(SCHED_DYNAMIC, [{}, {}])
    ex.close()


def test_cli_sched_flags(tmp_path):
    """kvm_exec --sched dynamic --classes 2 ...: the golden two-graph bundle still matches, with a report per class."""
    import subprocess
    from conftest import REPO
    exe = REPO / 'kvm_amd' / '_build' / 'kvm_exec'
    d = GOLDEN / 'live_training_inference'
    print('kvm_exec --sched dynamic', flush=True)
    r = subprocess.run([str(exe), '--golden', '--sched', 'dynamic', '--classes', '2', '--weights', '1,3', '--max', '4,2',
                        '--urgent-us', '0,100', str(d)], capture_output=True, text=True, timeout=120)
    lines = r.stdout.splitlines()
    assert r.returncode == 0 and lines[0].startswith('OK') and 'golden match' in lines[0], (r.stdout, r.stderr)
    assert lines[1].startswith('class 0: 6 tasks') and lines[2].startswith('class 1: 3 tasks'), lines
    r = subprocess.run([str(exe), '--sched', 'dynamic', '--classes', '1', str(d)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and 'workload_id' in r.stderr, (r.stdout, r.stderr)
