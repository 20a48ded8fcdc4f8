"""The static path's planner on the host (kvm_static_plan; reference design include/mvm_static.h): every task is placed
once, each worker's program respects the dependency DAG (successor edges plus the orderings version waits imply),
and replaying the programs with only the planned cross-worker waits finishes with every DAG edge honoured."""
import numpy as np
import pytest

from conftest import GOLDEN, golden_cases
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.executor import static_plan


def dag_edges(b):
    t = b.tasks
    edges = set()
    for u in range(t.shape[0]):
        for v in b.succ[t[u, 1]:t[u, 1] + t[u, 2]]:
            edges.add((u, int(v)))
    pubs = {}
    for i in range(t.shape[0]):
        if t[i, 10] >= 0:
            pubs.setdefault(int(t[i, 10]), []).append((int(t[i, 11]), i))
    for v in pubs.values():
        v.sort()
        edges |= {(v[j - 1][1], v[j][1]) for j in range(1, len(v))}
    for i in range(t.shape[0]):
        if t[i, 8] >= 0 and int(t[i, 8]) in pubs:
            cand = [p for ver, p in pubs[int(t[i, 8])] if ver <= t[i, 9]]
            if cand and cand[-1] != i:
                edges.add((cand[-1], i))
    return edges


def replay(b, P, workers):
    """Runs the programs with the planned waits only; returns the completion step of every task."""
    n = b.ntasks
    progs = [sorted([i for i in range(n) if P['worker'][i] == w], key=lambda i: P['pos'][i]) for w in range(workers)]
    woff = np.concatenate([[0], np.cumsum(P['nwaits'])])
    progress = [0] * workers                 # published watermark per worker
    nxt = [0] * workers
    done_at = [-1] * n
    step = 0
    while step < n:
        moved = False
        for w in range(workers):
            if nxt[w] == len(progs[w]):
                continue
            i = progs[w][nxt[w]]
            if all(progress[ww] >= need for ww, need in P['waits'][woff[i]:woff[i + 1]]):
                done_at[i] = step
                step += 1
                nxt[w] += 1
                if P['publishes'][i]:
                    progress[w] = nxt[w]
                moved = True
        assert moved, 'the planned waits deadlock'
    return done_at


def _check(b, workers):
    P = static_plan(b, workers)
    n = b.ntasks
    assert sorted((int(P['worker'][i]), int(P['pos'][i])) for i in range(n)) == sorted(
        (w, k) for w in range(workers) for k in range(int((P['worker'] == w).sum())))
    done = replay(b, P, workers)
    for u, v in dag_edges(b):
        assert done[u] < done[v], (u, v)
        if P['worker'][u] == P['worker'][v]:
            assert P['pos'][u] < P['pos'][v]
    assert P['makespan_us'] > 0 and P['work_us'] >= P['makespan_us'] * 0.999 / workers
    return P


@pytest.mark.parametrize('case', golden_cases())
@pytest.mark.parametrize('workers', [1, 3, 16])
def test_plan_of_golden_bundles(case, workers):
    _check(bl.load(GOLDEN / case), workers)


def test_plan_of_generated_graphs():
    from kvm_amd.workloads import gpt, mlp
    for w, workers in ((gpt.build(gpt.GPTConfig.tiny(steps=2)), 64), (mlp.build(mlp.MLPConfig(steps=2, widths=(64, 128, 768))), 256)):
        b = bl.load(compiler.compile_spec(w.spec))
        P = _check(b, workers)
        assert P['cross_edges'] <= P['edges'] and P['nwaits'].sum() <= P['cross_edges']


def test_plan_keeps_a_chain_on_one_worker():
    """A pure chain costs a cross-worker hop per edge elsewhere: the list scheduler keeps it on one worker, no waits."""
    from cases import W
    w = W(1)
    w.buf('x', 4)
    prev = []
    for _ in range(20):
        prev = [w.task('relu', after=prev, x='x', out='x', n=4)]
    b = bl.load(compiler.compile_spec(w.spec()))
    P = static_plan(b, 8)
    assert len(set(P['worker'].tolist())) == 1 and P['nwaits'].sum() == 0
