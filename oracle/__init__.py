"""CPU ORACLE (test infrastructure only; the product path never imports this package).

Python binding of oracle/oracle.cpp, the C++ restatement of the reference's deterministic CPU VM and reference operators.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker.
"""
from __future__ import annotations

import ctypes
import subprocess
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / '_build' / 'liboracle.so'
_lib = None


class OrcBuf(ctypes.Structure):
    _fields_ = [('p', ctypes.c_void_p), ('rows', ctypes.c_int32), ('cols', ctypes.c_int32), ('dtype', ctypes.c_int32)]


class OrcRead(ctypes.Structure):
    _fields_ = [('task', ctypes.c_int32), ('var', ctypes.c_int32), ('policy', ctypes.c_int32), ('version', ctypes.c_int32)]


def build() -> Path:
    subprocess.run(['make', '-s', '-C', str(HERE)], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = ctypes.CDLL(str(LIB))
        P = ctypes.c_void_p
        _lib.orc_run.argtypes = [P, ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int, P,
                                 ctypes.c_int, P, P, ctypes.c_int, P, ctypes.c_char_p, ctypes.c_int]
        _lib.orc_run.restype = ctypes.c_int
        _lib.orc_run_mt.argtypes = [P, ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int, P,
                                    ctypes.c_int, P, P, P, ctypes.c_int, ctypes.c_char_p, ctypes.c_int]
        _lib.orc_run_mt.restype = ctypes.c_int
        _lib.orc_seeded.argtypes = [P, ctypes.c_longlong, ctypes.c_ulonglong, ctypes.c_int, ctypes.c_float, ctypes.c_float]
        _lib.orc_seeded_bf16.argtypes = _lib.orc_seeded.argtypes
    return _lib


class OracleError(RuntimeError):
    pass


def run(bundle, buffers=None, limit=0, threads=1):
    """Run a bundle (directory, compiler.Bundle or bundle.LoadedBundle) on the CPU oracle.

    buffers: optional list of initial arrays (float32 for f32/bf16, int32 for i32); default = the metadata init.
    Returns dict(buffers=[arrays], versions={name: v}, order=[task indices], observed=[...per metadata read], seconds=s).
    limit > 0 stops after that many tasks (bounded CPU-baseline samples). threads > 1 runs ready tasks in parallel on
    that many worker threads (same results; `order` is then the completion order); limit applies to threads == 1 only.
    """
    from kvm_amd import bundle as bl
    b = bundle if isinstance(bundle, bl.LoadedBundle) else bl.load(bundle)
    meta = b.metadata
    if buffers is None:
        buffers = [bl.materialize(m, b.root) for m in meta['buffers']]
    buffers = [np.ascontiguousarray(x) for x in buffers]
    obufs = (OrcBuf * max(1, len(buffers)))()
    for i, (m, x) in enumerate(zip(meta['buffers'], buffers)):
        obufs[i] = OrcBuf(x.ctypes.data, m['rows'], m['cols'], m['dtype'])
    nvars = len(meta['variables'])
    versions = np.array([v['base_version'] for v in meta['variables']] or [0], np.int32)
    reads = meta['reads']
    rarr = (OrcRead * max(1, len(reads)))()
    for i, r in enumerate(reads):
        rarr[i] = OrcRead(r['task'], r['var'], 0 if r['policy'] == 'exact' else 1, r['version'])
    observed = np.zeros(max(1, len(reads)), np.int32)
    order = np.full(b.ntasks, -1, np.int32)
    dur = np.zeros(b.ntasks, np.float32)
    err = ctypes.create_string_buffer(512)
    tasks = np.ascontiguousarray(b.tasks, np.int32)
    succ = np.ascontiguousarray(b.succ, np.int32) if b.succ.size else np.zeros(1, np.int32)
    args = np.ascontiguousarray(b.args, np.int32) if b.args.size else np.zeros(1, np.int32)
    t0 = time.perf_counter()
    if threads > 1 and limit <= 0:
        rc = lib().orc_run_mt(tasks.ctypes.data, b.ntasks, succ.ctypes.data, int(b.succ.size), args.ctypes.data, int(b.args.size),
                              obufs, len(buffers), versions.ctypes.data, nvars, rarr, len(reads), observed.ctypes.data,
                              order.ctypes.data, dur.ctypes.data, threads, err, 512)
    else:
        rc = lib().orc_run(tasks.ctypes.data, b.ntasks, succ.ctypes.data, int(b.succ.size), args.ctypes.data, int(b.args.size),
                           obufs, len(buffers), versions.ctypes.data, nvars, rarr, len(reads), observed.ctypes.data,
                           order.ctypes.data, limit, dur.ctypes.data, err, 512)
    dt = time.perf_counter() - t0
    if rc:
        raise OracleError(err.value.decode())
    return {'buffers': buffers, 'versions': {v['name']: int(versions[v['id']]) for v in meta['variables']},
            'order': order, 'observed': observed[:len(reads)].tolist(), 'seconds': dt, 'task_us': dur}


def materialize(meta_buf, init=None, root=None):
    """Initial contents of a bundle buffer like kvm_amd.bundle.materialize, with the seeded generator in C (fast)."""
    from kvm_amd import bundle as bl
    init = init or meta_buf['init']
    if init['kind'] != 'seeded':
        return bl.materialize({**meta_buf, 'init': init}, root)
    return seeded(meta_buf['rows'] * meta_buf['cols'], init['seed'], init['draws'], init['bias'], init['coef'],
                  bf16=meta_buf['dtype'] == bl.DT_BF16)


def seeded(n, seed, draws, bias, coef, bf16=False):
    out = np.empty(n, np.float32)
    (lib().orc_seeded_bf16 if bf16 else lib().orc_seeded)(out.ctypes.data, n, seed % 2**64, draws, bias, coef)
    return out
