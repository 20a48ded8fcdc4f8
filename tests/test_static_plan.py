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


def expand(P, lo, hi, self_w):
    """The (worker, need) pairs of waits[lo:hi], set references expanded, the worker's own entries dropped (program
    order covers them, as the device skips them)."""
    out = []
    for ww, need in P['waits'][lo:hi]:
        if ww < 0:
            out += [tuple(x) for x in P['waits'][need:need + (-1 - ww)] if x[0] != self_w]
        elif ww != self_w:
            out.append((ww, need))
    return out


def replay(b, P, workers):
    """Runs the programs with the planned waits only; returns the completion step of every placed task (dissolved
    no-ops: -1)."""
    n = b.ntasks
    progs = [sorted([i for i in range(n) if P['worker'][i] == w], key=lambda i: P['pos'][i]) for w in range(workers)]
    placed = sum(len(p) for p in progs)
    woff = np.concatenate([[0], np.cumsum(P['nwaits'])])
    progress = [0] * workers                 # published watermark per worker
    nxt = [0] * workers
    done_at = [-1] * n
    step = 0
    while step < placed:
        moved = False
        for w in range(workers):
            if nxt[w] == len(progs[w]):
                continue
            i = progs[w][nxt[w]]
            if all(progress[ww] >= need for ww, need in expand(P, woff[i], woff[i + 1], w)):
                done_at[i] = step
                step += 1
                nxt[w] += 1
                if P['publishes'][i]:
                    progress[w] = nxt[w]
                moved = True
        assert moved, 'the planned waits deadlock'
    return done_at


def placed_edges(b, gone):
    """DAG edges between placed tasks, through chains of dissolved no-ops."""
    succ = {}
    for u, v in dag_edges(b):
        succ.setdefault(u, []).append(v)
    out = set()
    for u in range(b.ntasks):
        if gone[u]:
            continue
        stack, seen = list(succ.get(u, [])), set()
        while stack:
            v = stack.pop()
            if not gone[v]:
                out.add((u, v))
            elif v not in seen:
                seen.add(v)
                stack += succ.get(v, [])
    return out


def _check(b, workers, dissolve=False):
    P = static_plan(b, workers, dissolve)
    n = b.ntasks
    gone = P['worker'] < 0
    assert gone.sum() == P['dissolved'] and (dissolve or not gone.any())
    assert (b.tasks[gone, 0] == 0).all() and (P['pos'][gone] == -1).all()       # only no-ops dissolve
    assert sorted((int(P['worker'][i]), int(P['pos'][i])) for i in range(n) if not gone[i]) == sorted(
        (w, k) for w in range(workers) for k in range(int((P['worker'] == w).sum())))
    done = replay(b, P, workers)
    for u, v in placed_edges(b, gone):
        assert done[u] < done[v], (u, v)
        if P['worker'][u] == P['worker'][v]:
            assert P['pos'][u] < P['pos'][v]
    assert P['makespan_us'] > 0 and P['work_us'] >= P['makespan_us'] * 0.999 / workers
    return P


@pytest.mark.parametrize('case', golden_cases())
@pytest.mark.parametrize('workers', [1, 3, 16])
@pytest.mark.parametrize('dissolve', [False, True])
def test_plan_of_golden_bundles(case, workers, dissolve):
    _check(bl.load(GOLDEN / case), workers, dissolve)


@pytest.mark.parametrize('dissolve', [False, True])
def test_plan_of_generated_graphs(dissolve):
    from kvm_amd.workloads import gpt, mlp, qwen3
    for w, workers in ((gpt.build(gpt.GPTConfig.tiny(steps=2)), 64), (mlp.build(mlp.MLPConfig(steps=2, widths=(64, 128, 768))), 256),
                       (qwen3.build(qwen3.Qwen3Config.tiny(batch=2)), 32)):
        b = bl.load(compiler.compile_spec(w.spec))
        P = _check(b, workers, dissolve)
        assert P['nwaits'].sum() <= P['cross_edges']
        if dissolve:
            assert P['dissolved'] > 0


def test_dissolved_join_becomes_one_shared_wait_set():
    """A wide join between two phases: dissolved, the consumers reference one shared set whose entries name the
    producers' workers, and the replay still honours every producer -> consumer order."""
    from kvm_amd.workloads import Builder, Workload
    w = Builder(1)
    for k in range(8):
        w.fill(f'x{k}', 4)
    prod = [w.task('relu', x=f'x{k}', out=f'x{k}', n=4) for k in range(8)]
    j = w.join(prod, 8)
    [w.task('relu', after=j, x=f'x{k}', out=f'x{k}', n=4) for k in range(8)]
    b = bl.load(compiler.compile_spec(Workload(w.spec()).spec))
    assert (b.tasks[:, 0] == 0).sum() == 1
    P = _check(b, 8, dissolve=True)
    assert P['dissolved'] == 1
    refs = P['waits'][:int(P['nwaits'].sum())]
    assert (refs[:, 0] < 0).any() and len({int(x) for x in refs[refs[:, 0] < 0, 1]}) == 1
