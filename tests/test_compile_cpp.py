"""The C++ bundle compiler (kvm_compile) writes the same bytes as the Python compiler and as the reference compiler's
fixtures, and refuses the same malformed workloads. No GPU needed."""
import json
import subprocess

import pytest

from conftest import GOLDEN, golden_cases
from kvm_amd import build, compiler
from kvm_amd.workloads import gpt, mlp, qwen3

FILES = ('tasks.bin', 'successors.bin', 'args.bin', 'metadata.json')


def kvm_compile(spec_path, out, base=None):
    exe = build.OUT / 'kvm_compile'
    assert exe.exists(), 'kvm_compile is not built (python -m kvm_amd.build)'
    cmd = [str(exe), str(spec_path), str(out)]
    if base:
        cmd += ['--base-versions', ','.join(f'{k}={v}' for k, v in base.items())]
    return subprocess.run(cmd, capture_output=True, text=True)


def same_as_python(spec, tmp_path, base=None):
    p = tmp_path / 'w.json'
    p.write_text(json.dumps(spec))
    r = kvm_compile(p, tmp_path / 'cpp', base)
    assert r.returncode == 0, r.stderr
    b = compiler.compile_spec(spec, base, data_dir=tmp_path)
    b.write(tmp_path / 'py')
    files = [x.init['path'] for x in b.buffers if x.init['kind'] == 'file']
    for f in list(FILES) + files:
        assert (tmp_path / 'cpp' / f).read_bytes() == (tmp_path / 'py' / f).read_bytes(), f


@pytest.mark.parametrize('case', golden_cases())
def test_golden_bytes(case, tmp_path):
    d = GOLDEN / case
    r = kvm_compile(d / 'workload.json', tmp_path)
    assert r.returncode == 0, r.stderr
    for f in FILES:
        assert (tmp_path / f).read_bytes() == (d / f).read_bytes(), f


@pytest.mark.parametrize('name', ['gpt_tiny', 'mlp', 'qwen3_tiny', 'qwen3_tiny_b2'])
def test_generated_workloads(name, tmp_path):
    spec = {'gpt_tiny': lambda: gpt.build(gpt.GPTConfig.tiny()).spec,
            'mlp': lambda: mlp.build(mlp.MLPConfig(widths=(64, 96), steps=2)).spec,
            'qwen3_tiny': lambda: qwen3.build(qwen3.Qwen3Config.tiny()).spec,
            'qwen3_tiny_b2': lambda: qwen3.build(qwen3.Qwen3Config.tiny(batch=2)).spec}[name]()
    same_as_python(spec, tmp_path)


def _spec(tasks, variables=(), bufs=None):
    s = {'buffers': bufs or [{'name': 'a', 'rows': 4}], 'graphs': [{'name': 'g', 'tasks': tasks}]}
    if variables:
        s['variables'] = list(variables)
    return s


VERSIONED = [{'id': 'p1', 'op': 'noop', 'publishes': 'w'},
             {'id': 'p2', 'op': 'noop', 'publishes': 'w', 'after': ['p1']},
             {'id': 'q', 'op': 'noop', 'publishes': 'z', 'priority': 3, 'deadline_us': 50},
             {'id': 'r', 'op': 'noop', 'reads': [{'var': 'w', 'policy': 'exact', 'version': 1},
                                                {'var': 'z', 'policy': 'at_least', 'version': 1}]},
             {'id': 's', 'op': 'noop', 'reads': [{'var': 'w', 'policy': 'at_least', 'version': 0}]}]


@pytest.mark.parametrize('base', [None, {'w': 0}, {'w': 4}, {'w': 2, 'z': 7}])
def test_versions_gates_base(base, tmp_path):
    t = [dict(x) for x in VERSIONED]
    if base and base.get('w'):        # reads shifted to the base so none is stale
        t[3] = dict(t[3], reads=[{'var': 'w', 'policy': 'exact', 'version': base['w'] + 1},
                                 {'var': 'z', 'policy': 'at_least', 'version': base.get('z', 0) + 1}])
    same_as_python(_spec(t, ['w', 'z']), tmp_path, base)


def test_inits_and_args(tmp_path):
    (tmp_path / 'data').mkdir()
    (tmp_path / 'data' / 'x.bin').write_bytes(bytes(range(8)))
    bufs = [{'name': 'a', 'rows': 2, 'cols': 3, 'init': {'kind': 'values', 'values': [0.1, -2, 3.5e-7, 1e20, 123456789, 0]}},
            {'name': 'b', 'rows': 4, 'dtype': 'bf16', 'init': {'kind': 'values', 'values': [0.1, 1.0009765625, -3.3, 1e-30]}},
            {'name': 'c', 'rows': 3, 'dtype': 'i32', 'init': {'kind': 'values', 'values': [1, -7, 2.0]}},
            {'name': 'd', 'rows': 5, 'cols': 7, 'init': {'kind': 'seeded', 'seed': 2**63 - 1, 'scale': 0.02}},
            {'name': 'e', 'rows': 5, 'init': {'kind': 'seeded', 'seed': 3, 'scale': 1.5, 'dist': 'uniform'}},
            {'name': 'f', 'rows': 2, 'dtype': 'bf16', 'init': {'kind': 'fill', 'value': 0.3}},
            {'name': 'g', 'rows': 2, 'init': {'kind': 'file', 'path': './data//x.bin'}},
            {'name': 'hé\U0001F600', 'rows': 1}, {'name': 'i', 'rows': 4, 'dtype': 'i32'}]
    t = [{'id': 'x', 'op': 'scale', 'args': {'x': 'a', 'out': 'a', 'n': 6, 'alpha': 1e-45}},
         {'id': 'y', 'op': 'scale', 'args': {'x': 'a', 'out': 'a', 'n': 6, 'alpha': -0.0}, 'after': ['x']}]
    same_as_python(_spec(t, bufs=bufs), tmp_path)


BAD = [
    _spec([{'id': 'x', 'op': 'noop', 'after': ['y']}, {'id': 'y', 'op': 'noop', 'after': ['x']}]),
    _spec([{'id': 'p1', 'op': 'noop', 'publishes': 'w'}, {'id': 'p2', 'op': 'noop', 'publishes': 'w'}], ['w']),
    _spec([{'id': 'x', 'op': 'nope'}]),
    _spec([{'id': 'x', 'op': 'noop', 'after': ['x']}]),
    _spec([{'id': 'x', 'op': 'noop'}, {'id': 'x', 'op': 'noop'}]),
    _spec([{'id': 'x', 'op': 'scale', 'args': {'x': 'a', 'out': 'a', 'n': 1.5, 'alpha': 1}}]),
    _spec([{'id': 'x', 'op': 'scale', 'args': {'x': 'a', 'out': 'zz', 'n': 1, 'alpha': 1}}]),
    _spec([{'id': 'x', 'op': 'scale', 'args': {'x': 'a', 'out': 'a', 'n': 1, 'alpha': 1e39}}]),
    _spec([{'id': 'x', 'op': 'scale', 'args': {'x': 'a', 'out': 'a', 'n': 1}}]),
    _spec([{'id': 'x', 'op': 'noop', 'reads': [{'var': 'w', 'policy': 'exact', 'version': 2}]}], ['w']),
    _spec([{'id': 'x', 'op': 'noop', 'publishes': 'w', 'reads': [{'var': 'w', 'policy': 'at_least', 'version': 1}]}], ['w']),
    _spec([{'id': 'x', 'op': 'noop'}], bufs=[{'name': 'a', 'rows': 0}]),
    _spec([{'id': 'x', 'op': 'noop'}], bufs=[{'name': 'a', 'rows': 2, 'init': {'kind': 'values', 'values': [1]}}]),
    _spec([{'id': 'x', 'op': 'noop'}], bufs=[{'name': 'a', 'rows': 2, 'init': {'kind': 'file', 'path': '../x'}}]),
    _spec([{'id': 'x', 'op': 'noop'}], bufs=[{'name': 'a', 'dtype': 'i32', 'init': {'kind': 'seeded', 'seed': 1, 'scale': 1}}]),
    _spec([{'id': 'x', 'op': 'noop'}], bufs=[{'name': 'a', 'dtype': 'i32', 'init': {'kind': 'fill', 'value': 2**31}}]),
    {'graphs': [], 'extra': 1},
]


@pytest.mark.parametrize('k', range(len(BAD)))
def test_refuses_what_python_refuses(k, tmp_path):
    spec = BAD[k]
    with pytest.raises(compiler.CompileError):
        compiler.compile_spec(spec)
    p = tmp_path / 'w.json'
    p.write_text(json.dumps(spec))
    r = kvm_compile(p, tmp_path / 'out')
    assert r.returncode == 2 and 'kvm_compile:' in r.stderr
    assert not (tmp_path / 'out').exists()


def test_file_init_checked_against_data_dir(tmp_path):
    (tmp_path / 'x.bin').write_bytes(bytes(12))
    spec = _spec([{'id': 'x', 'op': 'noop'}], bufs=[{'name': 'a', 'rows': 2, 'init': {'kind': 'file', 'path': 'x.bin'}}])
    with pytest.raises(compiler.CompileError, match='bytes'):
        compiler.compile_spec(spec, data_dir=tmp_path)
    with pytest.raises(compiler.CompileError, match='data_dir'):
        compiler.compile_spec(spec).write(tmp_path / 'o')
    p = tmp_path / 'w.json'
    p.write_text(json.dumps(spec))
    r = kvm_compile(p, tmp_path / 'o')
    assert r.returncode == 2 and 'bytes' in r.stderr
    (tmp_path / 'x.bin').write_bytes(bytes(8))
    assert kvm_compile(p, tmp_path / 'o').returncode == 0
    assert (tmp_path / 'o' / 'x.bin').read_bytes() == bytes(8)


def test_base_versions_undeclared(tmp_path):
    p = tmp_path / 'w.json'
    p.write_text(json.dumps(_spec([{'id': 'x', 'op': 'noop'}], ['w'])))
    assert kvm_compile(p, tmp_path / 'o', {'q': 1}).returncode == 2
