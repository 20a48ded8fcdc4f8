"""GPU parity: every golden workload runs on the HIP executor and matches the CPU oracle (tolerances in gpu_check.py);
task counts, dependency order, exactly-once execution, versions and read snapshots are checked exactly."""
import numpy as np
import pytest

import oracle
from conftest import GOLDEN, REPO, golden_cases
from gpu_check import check_schedule, compare_run
from kvm_amd import bundle as bl
from kvm_amd.executor import Executor, seeded_fill_test

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('case', golden_cases())
def test_golden_workload_on_gpu(case):
    print(f'case {case}', flush=True)
    b = bl.load(GOLDEN / case)
    ref = oracle.run(b)
    ex = Executor.from_bundle(b)
    res = ex.run()
    assert res['done'] == res['admitted'] == b.ntasks
    tr = check_schedule(ex, b)
    vers = ex.versions()
    for v in b.metadata['variables']:
        assert vers[v['id']] == ref['versions'][v['name']]
    pubs = {(p['var'], p['version']): p['task'] for p in b.metadata['publishers']}
    for r in b.metadata['reads']:           # each read saw an admissible version
        slot = r['gate'] if r['gate'] is not None else r['task']
        if tr['ver0'][slot] < 0:            # version-0 read: no wait; the snapshot holds if the next publisher ran after it
            nxt = pubs.get((r['var'], r['version'] + 1))
            assert r['version'] == 0 and (r['policy'] != 'exact' or nxt is None or tr['start'][nxt] >= tr['end'][r['task']])
        elif r['policy'] == 'exact':
            assert tr['ver0'][slot] == r['version'] == tr['ver1'][slot]
        else:
            assert tr['ver0'][slot] >= r['version']
    bad = compare_run(ex, b.metadata, ref)
    assert not bad, bad
    ex.close()


def test_seeded_init_matches_reference_vectors():
    lines = (REPO / 'tests/golden/data/initgen_vectors.txt').read_text().split('\n')
    import struct
    for k in range(0, len(lines) - 1, 2):
        seed, draws, bh, ch, n = lines[k].split()
        f = lambda h: struct.unpack('<f', struct.pack('<I', int(h, 16)))[0]
        got = seeded_fill_test(int(seed), int(n), int(draws), f(bh), f(ch))
        assert got.view(np.uint32).tolist() == [int(h, 16) for h in lines[k + 1].split()]


def test_relaunch_is_repeatable():
    """Running the same graph again restarts versions and counters; a pure-function graph gives identical buffers."""
    b = bl.load(GOLDEN / 'gpt_ops')
    ex = Executor.from_bundle(b)
    ex.run()
    first = {m['name']: ex.read(m['name']) for m in b.metadata['buffers'] if m['name'] in ('mm0', 'o', 'dq', 'dk', 'mm32', 'lse')}
    ex.relaunch()
    ex.finish()
    for k, v in first.items():
        assert np.array_equal(ex.read(k), v), k
    ex.close()


@pytest.mark.parametrize('path', [0, 1])
def test_wide_fanout_and_fanin(path):
    """A root with 200 successors (the first 64 edges travel in the dispatch record, the rest come from the successor
    array), half of them also waiting on the version the root publishes (no no-wait edge bit), a task joining all
    200, and 100 more after it: every task runs once, after its predecessors, on both paths."""
    from kvm_amd import compiler
    from kvm_amd.workloads import Builder
    print(f'wide fan-out / fan-in, path {path}', flush=True)
    b = Builder(7)
    n = 200
    b.fill('c', 1 + n + 1 + 100, 1, 'i32')
    b.variables.append('v')
    root = b.task('counter_inc', publishes='v', x='c', i0=0, i1=1, delta=1)
    mids = [b.task('counter_inc', after=[root], reads=[{'var': 'v', 'policy': 'exact', 'version': 1}] if i % 2 else None,
                   x='c', i0=1 + i, i1=2 + i, delta=i + 1) for i in range(n)]
    last = b.task('counter_inc', after=mids, x='c', i0=n + 1, i1=n + 2, delta=5)
    for i in range(100):
        b.task('counter_inc', after=[last], x='c', i0=n + 2 + i, i1=n + 3 + i, delta=2)
    lb = bl.load(compiler.compile_spec(b.spec()))
    ex = Executor.from_bundle(lb, path=path)
    res = ex.run()
    assert res['done'] == res['admitted'] == lb.ntasks
    check_schedule(ex, lb)
    got = ex.read('c').reshape(-1)
    want = np.array([1] + [i + 1 for i in range(n)] + [5] + [2] * 100, np.int32)
    assert (got == want).all()
    ex.close()
