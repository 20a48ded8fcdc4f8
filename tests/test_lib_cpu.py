"""The C-ABI library builds, loads, exports every symbol include/kvm_exec.h declares, and its host-only validator
accepts the golden bundles and rejects malformed ones. No GPU needed."""
import ctypes
import json

import numpy as np
import pytest

from conftest import GOLDEN, golden_cases
from kvm_amd import bundle as bl
from kvm_amd import compiler, executor
from cases import W


def test_exports_every_declared_symbol():
    L = executor.lib()
    names = executor.declared_symbols()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), n


def test_registry_names():
    assert executor.op_name(34) == 'matmul_tile'
    assert executor.op_name(300) == 'head_rmsnorm'
    assert executor.op_name(999) is None


@pytest.mark.parametrize('case', golden_cases())
def test_validator_accepts_golden(case):
    assert executor.validate(bl.load(GOLDEN / case)) is None


def _bundle(w):
    return bl.load(compiler.compile_spec(w.spec()))


def test_validator_rejects_out_of_bounds_tile():
    w = W(1)
    w.buf('A', 8, 8), w.buf('B', 8, 8), w.zeros('C', 8, 8)
    w.task('matmul_tile', a='A', b='B', out='C', bias=None, res=None, pre=None, m0=0, n0=0, M=16, N=8, K=8, flags=0, alpha=1.0)
    assert 'too small' in executor.validate(_bundle(w))


def test_validator_rejects_dtype_and_cycle_and_arity():
    w = W(1)
    w.buf('x', 4), w.zeros('o', 4)
    w.ints('i', [1, 2, 3, 4])
    w.task('gelu_fwd', x='i', out='o', e0=0, e1=4)
    assert 'f32' in executor.validate(_bundle(w))
    b = _bundle(W(1).__class__(1)) if False else None
    w2 = W(1)
    w2.buf('x', 4)
    w2.task('relu', x='x', out='x', n=4)
    w2.task('relu', x='x', out='x', n=4)
    b = _bundle(w2)
    t = b.tasks.copy()
    t[0, 3] = 1                      # indegree no longer matches the edges
    assert 'indegree' in executor.validate(bl.LoadedBundle(b.metadata, t, b.succ, b.args))
    t = b.tasks.copy()
    t[0, 7] = 2                      # args_words != arity
    assert 'arity' in executor.validate(bl.LoadedBundle(b.metadata, t, b.succ, b.args))
    t = b.tasks.copy()
    t[0, 0] = 64                     # a registry op this executor does not run (comm pack)
    assert 'not run' in executor.validate(bl.LoadedBundle(b.metadata, t, b.succ, b.args))


def _chain(n=3):
    """n relu tasks t0 -> t1 -> ... in one bundle with one version variable (tasks edited per test)."""
    w = W(1)
    w.buf('x', 4)
    prev = []
    for _ in range(n):
        prev = [w.task('relu', after=prev, x='x', out='x', n=4)]
    b = _bundle(w)
    return b, b.tasks.copy()


def _with(b, t):
    return executor.validate(bl.LoadedBundle(b.metadata, t, b.succ, b.args))


def test_validator_rejects_priority_deadline_and_wait_ver():
    """Reference: mvm_exec.cu:154-157 (priority in [0, 32), deadline -1 or >= 0, wait_ver >= 0, pub_ver >= 1)."""
    b, t = _chain()
    t[1, 4] = 31
    assert _with(b, t) is None
    t[1, 4] = 32
    assert 'priority 32' in _with(b, t)
    t[1, 4] = -1
    assert 'priority' in _with(b, t)
    b, t = _chain()
    t[2, 5] = -2
    assert 'deadline' in _with(b, t)
    b, t = _chain()
    t[0, 8], t[0, 9] = 0, -1
    assert 'wait_ver' in _with(b, t)
    b, t = _chain()
    t[0, 10], t[0, 11] = 0, 0
    assert 'pub_ver' in _with(b, t)


def test_validator_rejects_version_wait_cycles():
    """A task that waits for a version only its own descendants (or itself) publish can never start (reference:
    mvm_exec.cu:179-205), also when the dependency runs through the version order (waiting for v2 needs v1 first).
    The same waits in the other direction, or for a variable no task of the bundle publishes, are accepted."""
    b, t = _chain(3)
    t[0, 8], t[0, 9] = 0, 1           # t0 waits for version 1 of variable 0 ...
    t[2, 10], t[2, 11] = 0, 1         # ... which t2, a descendant of t0, publishes
    assert 'version-wait cycle' in _with(b, t)
    t[0, 9] = 2                       # version 2 needs version 1 first: still a cycle
    assert 'version-wait cycle' in _with(b, t)
    t[2, 10], t[2, 11] = -1, 0        # no task of the bundle publishes the variable: decided outside
    assert _with(b, t) is None
    b, t = _chain(3)
    t[2, 8], t[2, 9] = 0, 1           # reversed: t2 waits for the version t0 publishes
    t[0, 10], t[0, 11] = 0, 1
    assert _with(b, t) is None
    b, t = _chain(3)
    t[1, 8], t[1, 9], t[1, 10], t[1, 11] = 0, 1, 0, 1
    assert 'publishes itself' in _with(b, t)
    b, t = _bundle_two_chains(), None
    t = b.tasks.copy()                # chains A (t0 -> t1 -> t2) and B (t3 -> t4 -> t5)
    t[0, 8], t[0, 9] = 0, 2           # A's head waits for v2
    t[3, 10], t[3, 11] = 0, 2         # B publishes v2 ...
    t[2, 10], t[2, 11] = 0, 1         # ... but v1 comes from A's tail: a cycle through the version order
    assert 'version-wait cycle' in _with(b, t)
    t[2, 10], t[2, 11] = -1, 0
    t[3, 10], t[3, 11] = 0, 1         # B publishes v1 then v2: satisfiable
    t[5, 10], t[5, 11] = 0, 2
    assert _with(b, t) is None


def _bundle_two_chains():
    w = W(1)
    w.buf('x', 4), w.buf('y', 4)
    for nm in ('x', 'y'):
        prev = []
        for _ in range(3):
            prev = [w.task('relu', after=prev, x=nm, out=nm, n=4)]
    return _bundle(w)


def test_validator_rejects_self_successor():
    b, t = _chain(2)
    s = b.succ.copy()
    s[0] = 0                          # t0 -> t0
    t[1, 3], t[0, 3] = 0, 1
    assert 'successor' in executor.validate(bl.LoadedBundle(b.metadata, t, s, b.args))
