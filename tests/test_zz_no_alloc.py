"""kvm_run_noalloc (the allocation-free entry point) against the allocating path (kvm_create / kvm_submit / kvm_start
/ kvm_finish) on the same bundles: same buffers bit for bit, same versions, exactly-once counts; two calls in a row,
the second on a smaller graph, then a graph larger than the scratch is refused before anything runs."""
import numpy as np
import pytest

from conftest import GOLDEN
from kvm_amd import bundle as bl
from kvm_amd import executor
from kvm_amd.executor import Executor
from cases import W

pytestmark = pytest.mark.gpu


def _caller_buffers(b):
    """Device buffers owned by the caller: an executor that only holds the buffer table (never started)."""
    ex = Executor(num_vars=max(1, len(b.metadata['variables'])), trace=False)
    for m in b.metadata['buffers']:
        ex.add_buffer(m['name'], m['rows'], m['cols'], m['dtype'], init=m['init'], root=b.root)
    ptrs = [executor.lib().kvm_buffer_device_ptr(ex._h, i) for i in range(len(b.metadata['buffers']))]
    return ex, ptrs


def test_noalloc_matches_allocating_path_twice():
    for case in ('gpt_ops', 'live_training_inference', 'versions'):   # gpt_ops is the largest: later calls are smaller
        print(f'noalloc {case}', flush=True)
        b = bl.load(GOLDEN / case)
        ref = Executor.from_bundle(b)
        rres = ref.run()
        mem, ptrs = _caller_buffers(b)
        base = [v['base_version'] for v in b.metadata['variables']]
        res, vers = executor.run_noalloc(b, ptrs, base)
        assert res['rc'] == 0, res
        assert res['err_code'] == 0 and res['done'] == res['admitted'] == b.ntasks == rres['done']
        want = ref.versions()
        assert vers[:len(base)] == [int(want[v['id']]) for v in b.metadata['variables']]
        for m in b.metadata['buffers']:
            g, r = mem.read_raw(m['name']), ref.read_raw(m['name'])
            assert np.array_equal(g.view(np.uint8), r.view(np.uint8)), (case, m['name'])
        ref.close()
        mem.close()


def test_noalloc_refuses_a_graph_beyond_its_scratch():
    w = W(1)
    w.buf('x', 4)
    for _ in range(50000):                 # 50,000 dispatch records of 768 B exceed the 32 MiB scratch
        w.task('noop')
    from kvm_amd import compiler
    b = bl.load(compiler.compile_spec(w.spec()))
    mem, ptrs = _caller_buffers(b)
    res, _ = executor.run_noalloc(b, ptrs, [0])
    assert res['rc'] == -2          # KVM_STATUS_TOO_BIG
    assert 'MiB' in res['err']
    mem.close()


def test_noalloc_refuses_a_grid_beyond_resident_capacity():
    """A persistent grid larger than the device can hold at once is refused before launch (workers that never start
    would leave their queues unserved), as kvm_create refuses it."""
    b = bl.load(GOLDEN / 'versions')
    mem, ptrs = _caller_buffers(b)
    res, _ = executor.run_noalloc(b, ptrs, [v['base_version'] for v in b.metadata['variables']], blocks=1 << 20)
    assert res['rc'] == -5 and 'co-resident capacity' in res['err'], res     # KVM_STATUS_INVALID
    mem.close()
