"""The static path on the GPU (KVM_PATH_STATIC: host-planned per-worker programs, progress-watermark waits; reference
design include/mvm_static.h): the golden graphs and generated workloads give the same results as the oracle, every
task runs once after its predecessors, and a graph the plan cannot decide is refused."""
import numpy as np
import pytest

import oracle
from conftest import GOLDEN, golden_cases
from gpu_check import check_schedule, compare_run
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.executor import Executor, KvmError, PATH_AUTO, PATH_DYNAMIC, PATH_STATIC
from cases import W

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('case', golden_cases())
def test_golden_on_static_path(case):
    print(f'static {case}', flush=True)
    b = bl.load(GOLDEN / case)
    ref = oracle.run(b)
    ex = Executor.from_bundle(b, path=PATH_STATIC)
    res = ex.run()
    assert ex.path() == PATH_STATIC
    assert res['done'] == b.ntasks
    check_schedule(ex, b)
    vers = ex.versions()
    for v in b.metadata['variables']:
        assert vers[v['id']] == ref['versions'][v['name']]
    assert not compare_run(ex, b.metadata, ref)
    ex.relaunch()                            # a second launch of the same plan
    assert ex.finish()['done'] == b.ntasks
    ex.close()


def _run(w, path):
    lb = bl.load(compiler.compile_spec(w.spec))
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    ex = Executor.from_bundle(lb, buffers=init, path=path)
    ex.run()
    return lb, init, ex


def test_tiny_gpt_and_mlps_on_static_path():
    from kvm_amd.workloads import gpt, mlp
    for w, tol in ((gpt.build(gpt.GPTConfig.tiny(steps=3)), 2e-4), (mlp.build(mlp.MLPConfig(steps=2)), 2e-4)):
        print('static workload', flush=True)
        lb, init, ex = _run(w, PATH_STATIC)
        assert ex.path() == PATH_STATIC
        check_schedule(ex, lb)
        ref = oracle.run(lb, [x.copy() for x in init], threads=16)
        skip = tuple(m['name'] for m in lb.metadata['buffers'] if m['name'].startswith(('bk.', 'd.bk.', 'm.bk.', 'v.bk.')))
        assert not compare_run(ex, lb.metadata, ref, tol_f32=tol, skip=skip)
        ex.close()


def test_auto_path_picks_static_for_short_tasks_and_dynamic_for_long():
    from kvm_amd.workloads import mlp
    lb, _, ex = _run(mlp.build(mlp.MLPConfig(steps=1, widths=(64,))), PATH_AUTO)
    assert ex.path() == PATH_STATIC
    ex.close()
    w = W(1)
    w.buf('A', 2048, 2048), w.buf('B', 2048, 2048), w.zeros('C', 2048, 2048)
    for m0 in range(0, 2048, 128):
        w.task('matmul_tile', a='A', b='B', out='C', bias=None, res=None, pre=None, m0=m0, n0=0, M=2048, N=2048, K=2048, flags=32, alpha=1.0)
    b = bl.load(compiler.compile_spec(w.spec()))
    ex = Executor.from_bundle(b, path=PATH_AUTO)
    ex.run()
    assert ex.path() == PATH_DYNAMIC
    ex.close()


def test_undecidable_wait_is_refused_on_the_static_path():
    w = W(1)
    w.buf('x', 4)
    w.vars = ['v']
    w.task('noop'), w.task('noop')
    b = bl.load(compiler.compile_spec(w.spec()))
    t = b.tasks.copy()
    t[1, 8], t[1, 9] = 0, 3                  # waits for a version no task publishes
    b = bl.LoadedBundle(b.metadata, t, b.succ, b.args, b.root)
    ex = Executor.from_bundle(b, path=PATH_STATIC)
    with pytest.raises(KvmError, match='no task of the graph publishes'):
        ex.run()
    ex.close()


def test_untraced_launches_run_the_plan_with_dissolved_noops():
    """Untraced launches run the plan with the ordering no-ops dissolved into wait sets: the same results as the
    oracle and every task counted done; a traced launch of the same executor runs every task (trace complete)."""
    from kvm_amd.workloads import gpt, mlp, qwen3
    for w, tol in ((gpt.build(gpt.GPTConfig.tiny(steps=2)), 2e-4), (mlp.build(mlp.MLPConfig(steps=2)), 2e-4),
                   (qwen3.build(qwen3.Qwen3Config.tiny(batch=2)), None)):
        lb = bl.load(compiler.compile_spec(w.spec))
        assert (lb.tasks[:, 0] == 0).any()
        print(f'static dissolved: {lb.ntasks} tasks', flush=True)
        init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
        ref = oracle.run(lb, [x.copy() for x in init], threads=16)
        names = [m['name'] for m in lb.metadata['buffers']]
        skip = tuple(n for n in names if n.startswith(('bk.', 'd.bk.', 'm.bk.', 'v.bk.')))
        ex = Executor.from_bundle(lb, buffers=[x.copy() for x in init], path=PATH_STATIC)
        ex.set_trace(False)
        res = ex.run()
        assert ex.path() == PATH_STATIC and res['done'] == lb.ntasks and res['err_code'] == 0
        if tol is not None:
            assert not compare_run(ex, lb.metadata, ref, tol_f32=tol, skip=skip)
        else:   # decode: tokens and lengths exact, logits close (the dynamic-path tolerance of this graph is derived elsewhere)
            assert np.array_equal(ex.read('tok'), ref['buffers'][names.index('tok')])
            assert np.array_equal(ex.read('lens'), ref['buffers'][names.index('lens')])
        ex.close()
        # traced: every task in the trace, the schedule checked (a fresh executor: the graph mutates its buffers)
        ex = Executor.from_bundle(lb, buffers=[x.copy() for x in init], path=PATH_STATIC)
        ex.run()
        check_schedule(ex, lb)
        ex.close()


def test_trace_setting_before_the_first_launch_holds():
    """set_trace(False) on an executor created with a trace buffer, before its first launch: the launches run untraced
    (the graph upload at the first launch keeps the request), on the static path and on the dynamic one."""
    from kvm_amd.workloads import gpt
    for path in (PATH_STATIC, PATH_DYNAMIC):
        w = gpt.build(gpt.GPTConfig.tiny(steps=1))
        lb = bl.load(compiler.compile_spec(w.spec))
        ex = Executor.from_bundle(lb, path=path, trace=True)
        ex.set_trace(False)
        assert not ex.tracing()
        res = ex.run()
        assert res['err_code'] == 0 and res['done'] == lb.ntasks
        assert ex.path() == path and not ex.tracing()
        ex.set_trace(True)
        ex.relaunch()
        ex.finish()
        assert ex.tracing() and (ex.trace()['exec_count'] == 1).all()
        ex.close()
