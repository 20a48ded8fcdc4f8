"""Stream mode on the GPU (reference: the admitter, its windows and submit_stream, mvm_exec.cuh:820-1058,
mvm_exec.cu:742-889): bundles admitted while the persistent kernel runs, window slots reused once their window has
finished, cross-bundle version waits, one large bundle cut into windows, and the host-side failure paths
(TOO_BIG, BACKPRESSURE_TIMEOUT, CLOSED) with the device ending normally."""
import numpy as np
import pytest

import oracle
from gpu_check import compare_run
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.executor import Executor, KvmError
from cases import W

pytestmark = pytest.mark.gpu

K = 24          # bundles of the reuse test
N = 64          # elements per buffer


def _table(nb):
    """A spec with the shared buffer table: x0..x{nb-1} (seeded), c (seeded), and no tasks yet."""
    w = W(3)
    for k in range(nb):
        w.buf(f'x{k}', N)
    w.buf('c', N)
    return w


def _bundle(w0, tasks):
    w = W(3)
    w.bufs, w.vars = w0.bufs, w0.vars
    w.tasks = tasks
    return bl.load(compiler.compile_spec(w.spec()))


def _stream_executor(b, **kw):
    ex = Executor(num_vars=max(1, len(b.metadata['variables'])), **kw)
    for m in b.metadata['buffers']:
        ex.add_buffer(m['name'], m['rows'], m['cols'], m['dtype'], init=m['init'], root=b.root)
    for v in b.metadata['variables']:
        ex.set_version(v['id'], v['base_version'])
    ex.meta = b.metadata
    return ex


def _chain(k):
    """x_k <- relu(0.5 x_k) * 3 + c, as four dependent tasks."""
    x = f'x{k}'
    return [{'id': 'a', 'op': 'scale', 'args': {'x': x, 'out': x, 'alpha': 0.5, 'n': N}},
            {'id': 'b', 'op': 'relu', 'args': {'x': x, 'out': x, 'n': N}, 'after': ['a']},
            {'id': 'c', 'op': 'scale', 'args': {'x': x, 'out': x, 'alpha': 3.0, 'n': N}, 'after': ['b']},
            {'id': 'd', 'op': 'add', 'args': {'a': x, 'b': 'c', 'out': x, 'n': N}, 'after': ['c']}]


def _f32(v):
    return np.float32(v)


def test_many_bundles_through_few_window_slots():
    """24 bundles of 4 dependent tasks through 3 window slots: every bundle runs once, its slot reused after it
    finished; each buffer ends equal to the closed form of its own chain (f32 per operation, as the reference)."""
    w0 = _table(K)
    bundles = [_bundle(w0, _chain(k)) for k in range(K)]
    ex = _stream_executor(bundles[0], window_cap=3, window_tasks=8, window_edges=8, timeout_s=10.0)
    init = {f'x{k}': ex.read(f'x{k}').copy() for k in range(K)}
    c = ex.read('c').copy()
    print('stream: 24 bundles, 3 slots', flush=True)
    ex.start()
    wids = [ex.submit(b) for b in bundles]
    assert wids == list(range(K))
    ex.stream_close()
    res = ex.finish()
    assert res['err_code'] == 0 and res['done'] == 4 * K and res['admitted'] == 4 * K
    assert all(ex.window_done(i) for i in range(K))
    for k in range(K):
        x = init[f'x{k}'].astype(np.float32)
        want = (np.maximum(x * _f32(0.5), 0).astype(np.float32) * _f32(3.0)).astype(np.float32) + c
        assert np.array_equal(ex.read(f'x{k}'), want.astype(np.float32)), k
    ex.close()


def test_bundles_submitted_before_start_and_a_cross_bundle_version_wait():
    """Bundle R (submitted first, before start) waits for version 1 of `v`, which only bundle P (submitted after
    start) publishes: R parks until P's publication, then reads P's output."""
    w0 = _table(2)
    w0.vars = ['v']
    reader = _bundle(w0, [{'id': 'r', 'op': 'add', 'args': {'a': 'x1', 'b': 'c', 'out': 'x0', 'n': N}}])
    reader.tasks[0, 8], reader.tasks[0, 9] = 0, 1          # wait_var, wait_ver: v >= 1 (published by another bundle)
    pub = _bundle(w0, [{'id': 'p', 'op': 'scale', 'args': {'x': 'c', 'out': 'x1', 'alpha': 2.0, 'n': N}, 'publishes': 'v'}])
    assert pub.tasks[0, 10] == 0 and pub.tasks[0, 11] == 1
    ex = _stream_executor(pub, window_cap=2, window_tasks=4, window_edges=4, timeout_s=10.0)
    c = ex.read('c').copy()
    print('stream: cross-bundle wait', flush=True)
    assert ex.submit(reader) == 0
    ex.start()
    assert ex.submit(pub) == 1
    res = ex.finish()               # closes the stream
    assert res['err_code'] == 0 and res['done'] == 2
    assert np.array_equal(ex.read('x0'), (c * _f32(2.0)).astype(np.float32) + c)
    assert ex.versions(1)[0] == 1
    ex.close()


def test_one_large_bundle_in_windows_matches_the_oracle():
    """Tiny GPT, 2 training steps, as one topologically ordered bundle cut into windows of 256 tasks over 4 slots:
    a window whose predecessors sit in earlier windows is submitted once those finished. Results as the oracle's."""
    from kvm_amd.workloads import gpt
    w = gpt.build(gpt.GPTConfig.tiny(steps=2))
    b = bl.load(compiler.compile_spec(w.spec))
    t = b.tasks
    topo = all(int(s) > u for u in range(t.shape[0]) for s in b.succ[t[u, 1]:t[u, 1] + t[u, 2]])
    if not topo:
        pytest.skip('the compiled bundle is not in topological order')
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in b.metadata['buffers']]
    ref = oracle.run(b, [x.copy() for x in init], threads=16)
    ex = Executor(num_vars=max(1, len(b.metadata['variables'])), window_cap=4, window_tasks=256, window_edges=4096, timeout_s=20.0)
    for m, x in zip(b.metadata['buffers'], init):
        ex.add_buffer(m['name'], m['rows'], m['cols'], m['dtype'], data=x)
    for v in b.metadata['variables']:
        ex.set_version(v['id'], v['base_version'])
    ex.meta = b.metadata
    print(f'stream: tiny gpt, {b.ntasks} tasks in windows of 256', flush=True)
    ex.start()
    nw = ex.submit_stream(b, max_window_tasks=256)
    assert nw >= b.ntasks // 256
    res = ex.finish()
    assert res['err_code'] == 0 and res['done'] == b.ntasks
    skip = tuple(m['name'] for m in b.metadata['buffers'] if m['name'].startswith(('bk.', 'd.bk.', 'm.bk.', 'v.bk.')))
    assert not compare_run(ex, b.metadata, ref, tol_f32=2e-4, skip=skip)
    ex.close()


def test_host_failure_paths_and_a_normal_device_exit():
    """A bundle larger than a window is TOO_BIG; with both slots held by tasks waiting for a version nobody
    publishes, a third submit gives up after backpressure_ms (BACKPRESSURE_TIMEOUT); the device then reports the stall
    (TIMEOUT) and every worker leaves; a submit after close is CLOSED."""
    w0 = _table(1)
    w0.vars = ['v']
    big = _bundle(w0, [{'id': f't{i}', 'op': 'noop', 'args': {}} for i in range(5)])
    waiter = _bundle(w0, [{'id': 'r', 'op': 'relu', 'args': {'x': 'x0', 'out': 'x0', 'n': N}}])
    t = waiter.tasks
    t[0, 8], t[0, 9] = 0, 7
    ex = _stream_executor(waiter, window_cap=2, window_tasks=4, window_edges=4, timeout_s=1.0, backpressure_ms=200)
    print('stream: failure paths', flush=True)
    ex.start()
    with pytest.raises(KvmError, match='exceeds a window'):
        ex.submit(big)
    assert ex.submit(waiter) == 0 and ex.submit(waiter) == 1
    with pytest.raises(KvmError, match='no window slot became free'):
        ex.submit(waiter)
    ex.stream_close()
    with pytest.raises(KvmError):
        ex.submit(waiter)
    res = ex.finish(check=False)
    assert res['err_code'] == 15 and res['done'] == 0
    ex.close()
