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
