"""The bundle compiler restatement emits byte-identical bundles to the reference compiler's (fixtures in tests/golden)."""
import json

import numpy as np
import pytest

from conftest import GOLDEN, golden_cases
from kvm_amd import abi, compiler


@pytest.mark.parametrize('case', golden_cases())
def test_bundle_bytes_identical(case, tmp_path):
    d = GOLDEN / case
    b = compiler.compile_spec(json.loads((d / 'workload.json').read_text()))
    b.write(tmp_path)
    for f in ('tasks.bin', 'successors.bin', 'args.bin', 'metadata.json'):
        assert (tmp_path / f).read_bytes() == (d / f).read_bytes(), f


def test_abi_header_and_registry():
    abi.check_header()
    ops = abi.load_ops()
    assert ops['matmul_tile'].id == 34 and ops['matmul_tile'].arity == 13
    assert ops['gemv_bf16'].id == 134 and ops['attn_decode_part'].arity == 18
    assert ops['head_rmsnorm'].id >= abi.EXT_ID_MIN
    assert len({o.id for o in ops.values()}) == len(ops)


def _spec(tasks, variables=(), bufs=None):
    s = {'buffers': bufs or [{'name': 'a', 'rows': 4}], 'graphs': [{'name': 'g', 'tasks': tasks}]}
    if variables:
        s['variables'] = list(variables)
    return s


def test_cycle_rejected():
    with pytest.raises(compiler.CompileError):
        compiler.compile_spec(_spec([{'id': 'x', 'op': 'noop', 'after': ['y']}, {'id': 'y', 'op': 'noop', 'after': ['x']}]))


def test_unordered_publishers_rejected():
    t = [{'id': 'p1', 'op': 'noop', 'publishes': 'w'}, {'id': 'p2', 'op': 'noop', 'publishes': 'w'}]
    with pytest.raises(compiler.CompileError, match='unordered'):
        compiler.compile_spec(_spec(t, ['w']))


def test_gate_and_war_edge():
    t = [{'id': 'p1', 'op': 'noop', 'publishes': 'w'}, {'id': 'p2', 'op': 'noop', 'publishes': 'w', 'after': ['p1']},
         {'id': 'q', 'op': 'noop', 'publishes': 'z'},
         {'id': 'r', 'op': 'noop', 'reads': [{'var': 'w', 'policy': 'exact', 'version': 1}, {'var': 'z', 'policy': 'at_least', 'version': 1}]}]
    b = compiler.compile_spec(_spec(t, ['w', 'z']))
    names = b.names
    assert names[3].startswith('__gate/g/r/')          # the second waiting read gets a gate just before r
    tasks = np.frombuffer(b.tasks, np.int32).reshape(-1, 16)
    r = names.index('g/r')
    assert tasks[r, 8] == 0 and tasks[r, 9] == 1       # r waits on w >= 1 itself
    succ = np.frombuffer(b.successors, np.int32)
    assert names.index('g/p2') in succ[tasks[r, 1]:tasks[r, 1] + tasks[r, 2]]   # write-after-read edge r -> p2


def test_bad_args_rejected():
    with pytest.raises(compiler.CompileError):
        compiler.compile_spec(_spec([{'id': 'x', 'op': 'copy', 'args': {'src': 'a', 'dst': 'nope', 'n': 1}}]))
    with pytest.raises(compiler.CompileError):
        compiler.compile_spec(_spec([{'id': 'x', 'op': 'copy', 'args': {'src': 'a', 'n': 1}}]))


def test_every_registry_op_fits_the_task_argument_block():
    """A task's argument words are staged in a fixed LDS block of KVM_MAX_ARGS words; every registry operator's arity
    must fit (an argument past the block would be read from whatever follows it)."""
    import re
    from conftest import REPO
    cap = int(re.search(r'#define KVM_MAX_ARGS (\d+)', (REPO / 'kvm_amd/csrc/common.h').read_text()).group(1))
    for f in sorted((REPO / 'include').glob('*.def')):
        for m in re.finditer(r'X\((\w+),\s*(\d+),\s*"([^"]*)"', f.read_text()):
            assert len(m.group(3).split(',')) <= cap, (f.name, m.group(1))
