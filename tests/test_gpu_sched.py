"""GPU tests of the scheduler's policy and error paths: priority order among ready tasks (strict, and with aging),
randomised priorities on the golden graphs, and device error reporting (operator argument errors found on the device,
VERSION_GAP, stall TIMEOUT), each ending with a normal kernel exit."""
import numpy as np
import pytest

import oracle
from conftest import GOLDEN
from gpu_check import check_schedule, compare_run
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.executor import Executor
from cases import W

pytestmark = pytest.mark.gpu


def _run(w, check=True, **kw):
    b = bl.load(compiler.compile_spec(w.spec()))
    ex = Executor.from_bundle(b, **kw)
    ex.start()
    res = ex.finish(check=check)
    return ex, b, res


def test_strict_priority_order_on_one_worker():
    """One worker: after the root, its 48 children are ready together and must start in descending priority, ties in
    release (index) order (reference rule: larger priority first, FIFO within a bucket)."""
    rng = np.random.default_rng(5)
    pr = rng.integers(0, 32, 48)
    w = W(1)
    w.buf('x', 4)
    r = w.task('noop')
    for p in pr:
        w.tasks.append({'id': f'c{len(w.tasks)}', 'op': 'noop', 'args': {}, 'after': [r], 'priority': int(p)})
    print('strict priority, 1 worker', flush=True)
    ex, b, res = _run(w, blocks=1)
    assert res['done'] == 49
    tr = check_schedule(ex, b)
    order = np.argsort(tr['start'][1:], kind='stable')
    want = sorted(range(48), key=lambda i: (-pr[i], i))
    assert order.tolist() == want
    ex.close()


def test_aging_lets_an_old_low_priority_task_overtake():
    """One worker. The root releases L (priority 0) and S (priority 1, spins 200 us); S releases eight priority-1
    tasks. Strict priority runs all eight before L; with aging_us = 20 L has gained ~10 levels while S ran and
    runs first (score = priority * aging + age, reference: mvm_sched.cuh:155-220)."""
    def graph():
        w = W(1)
        w.buf('x', 4)
        r = w.task('noop')
        w.tasks.append({'id': 'L', 'op': 'noop', 'args': {}, 'after': [r], 'priority': 0})
        w.tasks.append({'id': 'S', 'op': 'spin', 'args': {'us': 200}, 'after': [r], 'priority': 1})
        for k in range(8):
            w.tasks.append({'id': f'H{k}', 'op': 'noop', 'args': {}, 'after': ['S'], 'priority': 1})
        return w
    print('aging, 1 worker', flush=True)
    for aging, first in ((0, False), (20, True)):
        ex, b, res = _run(graph(), blocks=1, aging_us=aging)
        tr = ex.trace()
        names = b.metadata['task_names']
        L = names.index('g/L')
        H = [i for i, n in enumerate(names) if n.startswith('g/H')]
        assert (tr['start'][L] < tr['start'][H].min()) == first, aging
        ex.close()


@pytest.mark.parametrize('case', ['gpt_ops', 'versions', 'live_training_inference', 'core'])
def test_golden_with_random_priorities(case):
    """Random priorities (all 32 buckets) on a golden graph, full grid: exactly-once, dependency order and results as in
    FIFO mode (the oracle honours the same priorities; results do not depend on the order)."""
    b = bl.load(GOLDEN / case)
    t = b.tasks.copy()
    t[:, 4] = np.random.default_rng(7).integers(0, 32, t.shape[0])
    b = bl.LoadedBundle(b.metadata, t, b.succ, b.args, b.root)
    print(f'random priorities {case}', flush=True)
    ref = oracle.run(b)
    ex = Executor.from_bundle(b)
    res = ex.run()
    assert res['done'] == b.ntasks
    check_schedule(ex, b)
    for v in b.metadata['variables']:
        assert ex.versions()[v['id']] == ref['versions'][v['name']]
    assert not compare_run(ex, b.metadata, ref)
    ex.close()


def test_token_out_of_range_is_a_device_error():
    """The host cannot see data: an id >= V is found by the embedding task on the device (op error 1005, task slot and
    row/id reported); the run stops and the kernel exits normally."""
    w = W(1)
    w.ints('ids', [1, 2, 99, 3]), w.buf('wte', 16, 8), w.zeros('out', 4, 8)
    w.task('embedding_fwd', ids='ids', wte='wte', wpe=None, out='out', r0=0, r1=4, T=4, d=8)
    print('token error', flush=True)
    ex, b, res = _run(w, check=False)
    assert res['err_code'] == 1005 and res['err_slot'] == 0
    assert (res['err_a'], res['err_b']) == (2, 99)
    ex.close()


def test_kv_length_overflow_is_a_device_error():
    w = W(1)
    hd, Tm = 16, 8
    w.buf('q', 1, hd), w.buf('kc', Tm, hd), w.buf('vc', Tm, hd), w.ints('lens', [Tm]), w.zeros('o', 1, hd)
    w.task('attn_decode', q='q', kc='kc', vc='vc', lens='lens', o='o', b=0, h=0, H=1, Hkv=1, hd=hd, Tmax=Tm, scale=0.25)
    print('kv length error', flush=True)
    ex, b, res = _run(w, check=False)
    assert res['err_code'] == 1006 and res['err_slot'] == 0
    ex.close()


def _edited(w, edit):
    b = bl.load(compiler.compile_spec(w.spec()))
    t = b.tasks.copy()
    edit(t)
    return bl.LoadedBundle(b.metadata, t, b.succ, b.args, b.root)


def test_version_gap_is_reported():
    """Two tasks in a chain both publish version 1 of one variable (the compiler numbers publications itself, so the
    second is edited from 2 to 1): the second CAS finds 1, not 0, and reports VERSION_GAP (7) with (found, wanted)."""
    w = W(1)
    w.buf('x', 4)
    w.vars = ['v']
    w.tasks.append({'id': 'a', 'op': 'noop', 'args': {}, 'publishes': 'v'})
    w.tasks.append({'id': 'b', 'op': 'noop', 'args': {}, 'after': ['a'], 'publishes': 'v'})

    def edit(t):
        assert t[1, 10] == 0 and t[1, 11] == 2
        t[1, 11] = 1
    b = _edited(w, edit)
    print('version gap', flush=True)
    ex = Executor.from_bundle(b)
    ex.start()
    res = ex.finish(check=False)
    assert res['err_code'] == 7 and res['err_slot'] == 1
    assert (res['err_a'], res['err_b']) == (1, 1)
    ex.close()


def test_unsatisfiable_wait_times_out():
    """A task waits for a version no task publishes: the stall timeout (0.2 s here) ends the run with TIMEOUT (15)
    and every worker leaves."""
    w = W(1)
    w.buf('x', 4)
    w.vars = ['v']
    w.task('noop'), w.task('noop')

    def edit(t):
        t[1, 8], t[1, 9] = 0, 3
    b = _edited(w, edit)
    print('stall timeout', flush=True)
    ex = Executor.from_bundle(b, timeout_s=0.2)
    ex.start()
    res = ex.finish(check=False)
    assert res['err_code'] == 15
    assert res['done'] == 1
    ex.close()


def test_grid_beyond_coresidency_is_refused():
    """A persistent executor needs every worker resident at once: more workgroups than the device holds is refused."""
    from kvm_amd.executor import KvmError
    with pytest.raises(KvmError, match='co-resident'):
        Executor(blocks=100000)
