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
from kvm_amd.executor import (SCHED_DYNAMIC, SCHED_F_ARBITER, SCHED_F_GUARANTEE, SCHED_F_INHERIT, SCHED_STATIC, TRACE_BOOST,
                              TRACE_MISSED, TRACE_RESV, TRACE_URGENT, UNLIMITED, Executor, KvmError)

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
        ex.set_classes(SCHED_DYNAMIC, [{'max_cta': -1}])
    with pytest.raises(KvmError, match='bw_cta'):
        ex.set_classes(SCHED_DYNAMIC, [{'bw_cta': -1}])
    with pytest.raises(KvmError, match='unknown flags'):
        ex.set_sched_flags(8)
    with pytest.raises(KvmError, match='bw_limit'):
        ex.set_sched_flags(SCHED_F_ARBITER, 0)
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


# ---- priority inheritance across version waits and bandwidth caps (reference: include/mvm_sched.cuh:35-40, 486-496;
# include/mvm_sched.h:26-33, 45-46)

def versioned_spec(graphs, variables):
    """graphs: per class, a list of (spin us, publishes var or None, reads var or None)."""
    out = []
    for c, tasks in enumerate(graphs):
        ts = []
        for k, (us, pub, rd) in enumerate(tasks):
            t = {'id': f't{k}', 'op': 'spin', 'args': {'us': us}}
            if pub:
                t['publishes'] = pub
            if rd:
                t['reads'] = [{'var': rd, 'policy': 'at_least', 'version': 1}]
            ts.append(t)
        out.append({'name': f'c{c}', 'tasks': ts})
    return {'variables': variables, 'buffers': [{'name': 'x', 'rows': 4}], 'graphs': out}


def run_flags(spec, classes, flags, bw_limit=UNLIMITED, timeout_s=20.0):
    b = bl.load(compiler.compile_spec(spec))
    ex = Executor.from_bundle(b, timeout_s=timeout_s)
    ex.set_classes(SCHED_DYNAMIC, classes)
    ex.set_sched_flags(flags, bw_limit)
    return ex, b


def test_inheritance_runs_a_fully_throttled_publisher():
    """Class 1 may not run at all (max_cta 0) but publishes the version a class-0 task waits for: inheritance boosts it,
    its task starts under the boost and the graph completes; with inheritance off the waiter parks for ever and the run
    ends with the stall TIMEOUT (the reference's negative test, mvm_sched.cuh:40)."""
    spec = versioned_spec([[(20, None, 'v'), (20, None, None)], [(50, 'v', None)]], ['v'])
    classes = [{}, {'max_cta': 0}]
    ex, b = run_flags(spec, classes, SCHED_F_GUARANTEE | SCHED_F_INHERIT)
    ex.run()
    tr = check_schedule(ex, b)
    cls = b.tasks[:, 12]
    assert (tr['how'][cls == 1] & TRACE_BOOST).all()
    assert ex.class_stats(2)['boost_starts'][1] == 1
    assert ex.versions(1)[0] == 1
    ex.close()
    ex, b = run_flags(spec, classes, SCHED_F_GUARANTEE, timeout_s=0.5)
    ex.start()
    res = ex.finish(check=False)
    assert res['err_code'] == 15, res          # TIMEOUT: nothing finished while work was pending
    ex.close()


def test_inheritance_is_transitive():
    """Class 0 waits on v1, published by a class-1 task that itself waits on v2, published by class 2; classes 1 and 2
    are both throttled to nothing: both get boosted (the closure over parked waiters) and the chain completes in order."""
    spec = versioned_spec([[(10, None, 'v1')], [(30, 'v1', 'v2')], [(30, 'v2', None)]], ['v1', 'v2'])
    ex, b = run_flags(spec, [{}, {'max_cta': 0}, {'max_cta': 0}], SCHED_F_GUARANTEE | SCHED_F_INHERIT)
    ex.run()
    tr = check_schedule(ex, b)
    cls = b.tasks[:, 12]
    assert (tr['how'][cls >= 1] & TRACE_BOOST).all()
    t1, t2 = np.where(cls == 1)[0][0], np.where(cls == 2)[0][0]
    assert tr['end'][t2] <= tr['start'][t1]
    assert ex.versions(2).tolist() == [1, 1]
    ex.close()


def fill_spec(per_class, n=1 << 22):
    """Per class, `per_class[c]` independent fill tasks of n floats each (bandwidth-bound: 4n bytes) and two spins."""
    graphs = []
    for c, k in enumerate(per_class):
        ts = [{'id': f'f{i}', 'op': 'fill', 'args': {'x': f'b{c}', 'value': float(i), 'n': n}} for i in range(k)]
        ts += [{'id': f's{i}', 'op': 'spin', 'args': {'us': 30}} for i in range(2)]
        graphs.append({'name': f'c{c}', 'tasks': ts})
    return {'buffers': [{'name': f'b{c}', 'rows': n} for c in range(len(per_class))], 'graphs': graphs}


def test_bw_cta_bounds_a_class_bandwidth_bound_tasks():
    """bw_cta 2: at no instant do more than two of class 0's fill tasks run (its spin tasks are not bandwidth-bound and
    are not held back); uncapped, the same graph runs more of them at once (so the bound is the cap's doing)."""
    spec = fill_spec([24, 8])
    for cap in (2, UNLIMITED):
        ex, b = run_flags(spec, [{'bw_cta': cap}, {}], SCHED_F_GUARANTEE | SCHED_F_INHERIT)
        ex.run()
        tr = check_schedule(ex, b)
        cls, fills = b.tasks[:, 12], b.tasks[:, 0] == 9
        peak = max_overlap(tr, (cls == 0) & fills)
        print('bw_cta', cap, 'peak running fills', peak, flush=True)
        if cap == 2:
            assert 1 <= peak <= 2
        else:
            assert peak > 2
        ex.close()


def test_arbiter_bounds_bandwidth_bound_tasks_of_all_classes():
    """ARBITER with bw_limit 3: at most three fill tasks of the two classes together run at once."""
    spec = fill_spec([16, 16])
    ex, b = run_flags(spec, [{}, {}], SCHED_F_GUARANTEE | SCHED_F_INHERIT | SCHED_F_ARBITER, bw_limit=3)
    ex.run()
    tr = check_schedule(ex, b)
    peak = max_overlap(tr, b.tasks[:, 0] == 9)
    print('arbiter peak running fills', peak, flush=True)
    assert 1 <= peak <= 3
    ex.close()


def chain_spec(chains, length, us):
    """`chains` independent chains of `length` dependent spin tasks, one class."""
    ts = []
    for c in range(chains):
        for k in range(length):
            t = {'id': f'c{c}k{k}', 'op': 'spin', 'args': {'us': us}}
            if k:
                t['after'] = [f'c{c}k{k - 1}']
            ts.append(t)
    return {'buffers': [{'name': 'x', 'rows': 4}], 'graphs': [{'name': 'g', 'tasks': ts}]}


def test_task_affinity_keeps_a_chain_on_its_worker():
    """Affinity window 1 s (reference: MvmSchedParams.affinity_us): each task released by its predecessor is offered
    only to the worker that ran the predecessor, so every chain runs on one worker (its root's)."""
    spec = chain_spec(8, 10, 10)
    for aff in (1_000_000, 0):
        b = bl.load(compiler.compile_spec(spec))
        ex = Executor.from_bundle(b)
        ex.set_classes(SCHED_DYNAMIC, [{}])
        ex.set_affinity(aff)
        ex.run()
        tr = check_schedule(ex, b)
        blocks = [len(np.unique(tr['block'][c * 10:(c + 1) * 10])) for c in range(8)]
        print('affinity', aff, 'workers per chain', blocks, flush=True)
        if aff:
            assert blocks == [1] * 8
        ex.close()


def test_op_affinity_prefers_the_worker_that_last_ran_the_operator():
    """Task C (spin) waits for A (a 1 us spin) and B (a 64 MiB fill, which ends later and releases C). With op affinity
    C runs on A's worker, the last to finish a spin; with chain affinity only, on B's worker, which released it."""
    ts = [{'id': 'a', 'op': 'spin', 'args': {'us': 1}},
          {'id': 'b', 'op': 'fill', 'args': {'x': 'y', 'value': 1.0, 'n': 1 << 24}},
          {'id': 'c', 'op': 'spin', 'args': {'us': 1}, 'after': ['a', 'b']}]
    spec = {'buffers': [{'name': 'x', 'rows': 4}, {'name': 'y', 'rows': 1 << 24}], 'graphs': [{'name': 'g', 'tasks': ts}]}
    for opaff in (True, False):
        b = bl.load(compiler.compile_spec(spec))
        ex = Executor.from_bundle(b)
        ex.set_classes(SCHED_DYNAMIC, [{'opaff': opaff}])
        ex.set_affinity(1_000_000)
        ex.run()
        tr = check_schedule(ex, b)
        print('op affinity', opaff, 'blocks a b c', tr['block'][:3].tolist(), 'ends', tr['end'][:2].tolist(), flush=True)
        assert tr['end'][0] < tr['end'][1] and tr['block'][0] != tr['block'][1]
        assert tr['block'][2] == tr['block'][0 if opaff else 1]
        ex.close()


def test_affinity_errors():
    """A negative window and class flags other than op affinity are refused; a short window runs normally."""
    import ctypes
    from kvm_amd.executor import KvmClassParams, lib
    b = bl.load(compiler.compile_spec(spin_spec([[(1, None)]])))
    ex = Executor.from_bundle(b)
    with pytest.raises(KvmError, match='affinity_us'):
        ex.set_affinity(-1)
    p = (KvmClassParams * 1)()
    p[0] = KvmClassParams(1, 0, UNLIMITED, 0, 1, UNLIMITED, 1)
    with pytest.raises(KvmError, match='unknown flags'):
        ex._check(lib().kvm_set_classes(ex._h, SCHED_DYNAMIC, ctypes.byref(p), 1), 'set_classes')
    ex.set_classes(SCHED_DYNAMIC, [{'opaff': True}])
    ex.set_affinity(50)
    ex.run()
    ex.close()
