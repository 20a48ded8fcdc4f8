"""Python host side of the executor: a ctypes binding of libkvm_exec.so (include/kvm_exec.h).

Mirrors the reference's MvmExec interface (reference: mvm_exec.cu:492-1560): create, add buffers, set versions, submit
bundles, start, finish, read buffers, trace. The GPU path is the HIP library only: if it is not built, or no GPU is
present, the calls raise; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np

from . import bundle as bl

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / '_build' / 'libkvm_exec.so'
HEADER = HERE.parent / 'include' / 'kvm_exec.h'
_lib = None

KVM_INIT_ZERO, KVM_INIT_FILL, KVM_INIT_VALUES, KVM_INIT_SEEDED = 0, 1, 2, 3
ERRORS = {0: 'OK', 1: 'BAD_OP', 2: 'BAD_ARITY', 3: 'BAD_BUF_INDEX', 4: 'BAD_BUF', 5: 'BOUNDS', 6: 'BAD_VAR', 7: 'VERSION_GAP',
          8: 'WAIT_VIOLATION', 9: 'DOUBLE_EXEC', 11: 'BAD_TASK', 15: 'TIMEOUT', 16: 'QUEUE_OVERFLOW', 17: 'BAD_CONFIG',
          1001: 'OP_BUF', 1002: 'OP_DTYPE', 1003: 'OP_RANGE', 1004: 'OP_SHAPE', 1005: 'OP_TOKEN', 1006: 'OP_KVLEN'}


class KvmConfig(ctypes.Structure):
    _fields_ = [('blocks', ctypes.c_int), ('trace_on', ctypes.c_int), ('num_vars', ctypes.c_int), ('timeout_us', ctypes.c_ulonglong),
                ('device', ctypes.c_int), ('aging_us', ctypes.c_int), ('path', ctypes.c_int), ('window_cap', ctypes.c_int),
                ('window_tasks', ctypes.c_int), ('window_edges', ctypes.c_int), ('backpressure_ms', ctypes.c_int)]


PATH_DYNAMIC, PATH_STATIC, PATH_AUTO = 0, 1, 2


class KvmInit(ctypes.Structure):
    _fields_ = [('kind', ctypes.c_int), ('value', ctypes.c_float), ('values', ctypes.c_void_p), ('seed', ctypes.c_ulonglong),
                ('draws', ctypes.c_int), ('bias', ctypes.c_float), ('coef', ctypes.c_float)]


class KvmTrace(ctypes.Structure):
    _fields_ = [('start', ctypes.c_ulonglong), ('end', ctypes.c_ulonglong), ('block', ctypes.c_int), ('xcc', ctypes.c_int),
                ('ver0', ctypes.c_int), ('ver1', ctypes.c_int), ('exec_count', ctypes.c_int), ('how', ctypes.c_int)]


class KvmResult(ctypes.Structure):
    _fields_ = [('err_code', ctypes.c_int), ('err_slot', ctypes.c_int), ('err_a', ctypes.c_int), ('err_b', ctypes.c_int),
                ('done', ctypes.c_int), ('admitted', ctypes.c_int), ('grid', ctypes.c_int), ('kernel_ms', ctypes.c_float)]


TRACE_DTYPE = np.dtype([('start', '<u8'), ('end', '<u8'), ('block', '<i4'), ('xcc', '<i4'), ('ver0', '<i4'), ('ver1', '<i4'),
                        ('exec_count', '<i4'), ('how', '<i4')])
TRACE_MISSED, TRACE_RESV, TRACE_BOOST, TRACE_URGENT = 1, 2, 4, 8
SCHED_F_GUARANTEE, SCHED_F_INHERIT, SCHED_F_ARBITER = 1, 2, 4
CLASS_OPAFF = 2                 # KvmClassParams.flags: op affinity (kvm_set_affinity sets the window)
SCHED_GLOBAL, SCHED_STATIC, SCHED_DYNAMIC = 0, 1, 2
UNLIMITED = 0x7fffffff


class KvmClassParams(ctypes.Structure):
    _fields_ = [('weight', ctypes.c_int), ('min_cta', ctypes.c_int), ('max_cta', ctypes.c_int), ('urgent_us', ctypes.c_int),
                ('share', ctypes.c_int), ('bw_cta', ctypes.c_int), ('flags', ctypes.c_int)]


CLASS_STATS_DTYPE = np.dtype([('tasks', '<u8'), ('busy_ticks', '<u8'), ('resv_starts', '<u8'), ('urgent_starts', '<u8'),
                              ('missed', '<u8'), ('max_running', '<i4'), ('pad', '<i4'), ('boost_starts', '<u8')])


def declared_symbols() -> list[str]:
    """Every function include/kvm_exec.h declares."""
    return re.findall(r'^\s*[\w\s\*]+?\b(kvm_\w+)\s*\(', HEADER.read_text(), re.M)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f'{LIB_PATH} is not built: run __graft_entry__.build() (or python kvm_amd/build.py)')
        L = ctypes.CDLL(str(LIB_PATH))
        P, I, U = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        sig = {
            'kvm_config_default': (None, [P]), 'kvm_create': (P, [P]), 'kvm_destroy': (None, [P]),
            'kvm_last_error': (ctypes.c_char_p, [P]), 'kvm_add_buffer': (I, [P, I, I, I, P]), 'kvm_nbufs': (I, [P]),
            'kvm_buffer_dtype': (I, [P, I]), 'kvm_buffer_device_ptr': (P, [P, I]), 'kvm_write_buffer': (I, [P, I, P, U]),
            'kvm_read_buffer': (I, [P, I, P, U]), 'kvm_read_raw': (I, [P, I, P, U]), 'kvm_set_version': (I, [P, I, I]),
            'kvm_submit': (I, [P, P, I, P, I, P, I]), 'kvm_start': (I, [P]), 'kvm_finish': (I, [P, P]), 'kvm_relaunch': (I, [P]),
            'kvm_run_timed': (I, [P, I, P]), 'kvm_run_timed_split': (I, [P, I, P, P]), 'kvm_versions': (I, [P, P, I]), 'kvm_trace': (I, [P, P, I]), 'kvm_ntasks': (I, [P]), 'kvm_set_trace': (I, [P, I]), 'kvm_get_trace': (I, [P]),
            'kvm_op_name': (ctypes.c_char_p, [I]),
            'kvm_validate': (I, [P, I, P, I, P, I, P, I, I, ctypes.c_char_p, I]),
            'kvm_seeded_fill_test': (I, [ctypes.c_ulonglong, ctypes.c_longlong, I, ctypes.c_float, ctypes.c_float, P]),
            'kvm_copy_probe': (I, [ctypes.c_longlong]),
            'kvm_path': (I, [P]), 'kvm_close': (I, [P]), 'kvm_window_done': (I, [P, ctypes.c_longlong]), 'kvm_live_versions': (I, [P, P, I]),
            'kvm_submit_stream': (I, [P, P, I, P, I, P, I, I, I]),
            'kvm_static_plan': (I, [P, I, P, I, P, I, I, I, P, P, P, P, P, I, P, ctypes.c_char_p, I]),
            'kvm_set_classes': (I, [P, I, P, I]), 'kvm_class_stats': (I, [P, P, I]), 'kvm_set_sched_flags': (I, [P, I, I]), 'kvm_set_affinity': (I, [P, I]),
            'kvm_run_noalloc': (I, [P, I, P, I, P, I, P, I, P, I, I, ctypes.c_ulonglong, P, P, ctypes.c_char_p, I]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _lib = L
    return _lib


class KvmError(RuntimeError):
    pass


class Executor:
    """One persistent-kernel executor on one GPU. Typical use::

        ex = Executor.from_bundle(bundle_dir)   # buffers + versions from the metadata, bundle submitted
        res = ex.run()                          # start + finish
        x = ex.read('logits')
    """

    def __init__(self, num_vars: int = 64, trace: bool = True, timeout_s: float = 20.0, blocks: int = 0, device: int = 0,
                 aging_us: int = 0, path: int = 0, window_cap: int = 0, window_tasks: int = 0, window_edges: int = 0,
                 backpressure_ms: int = 60000):
        """window_cap > 0: stream mode (include/kvm_exec.h): start() launches the kernel, submit() admits bundles while
        it runs (window slots of window_tasks tasks / window_edges edges), stream_close() ends the stream."""
        L = lib()
        cfg = KvmConfig()
        L.kvm_config_default(ctypes.byref(cfg))
        cfg.num_vars, cfg.trace_on, cfg.timeout_us, cfg.blocks, cfg.device = max(1, num_vars), int(trace), int(timeout_s * 1e6), blocks, device
        cfg.aging_us, cfg.path = aging_us, path
        cfg.window_cap, cfg.window_tasks, cfg.window_edges, cfg.backpressure_ms = window_cap, window_tasks, window_edges, backpressure_ms
        self._h = L.kvm_create(ctypes.byref(cfg))
        if not self._h:
            raise KvmError(f'kvm_create: {L.kvm_last_error(None).decode()}')
        self.names, self.shapes, self.dtypes = [], [], []
        self.trace_on = trace
        self.meta = None

    def close(self):
        if self._h:
            lib().kvm_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        if rc < 0:
            raise KvmError(f'{what}: {lib().kvm_last_error(self._h).decode()}')
        return rc

    # ------------------------------------------------------------------ buffers
    def add_buffer(self, name, rows, cols, dtype, init: dict | None = None, data: np.ndarray | None = None, root=None) -> int:
        ini = KvmInit()
        keep = None
        if data is not None:
            keep = _as_storage(np.asarray(data), dtype)
            ini.kind, ini.values = KVM_INIT_VALUES, keep.ctypes.data
        elif init is None:
            ini.kind = KVM_INIT_ZERO
        elif init['kind'] == 'fill':
            ini.kind, ini.value = KVM_INIT_FILL, float(init['value'])
        elif init['kind'] == 'seeded':
            ini.kind, ini.seed, ini.draws, ini.bias, ini.coef = KVM_INIT_SEEDED, init['seed'] % 2**64, init['draws'], init['bias'], init['coef']
        else:
            keep = _as_storage(bl.materialize({'rows': rows, 'cols': cols, 'dtype': dtype, 'init': init}, root), dtype)
            ini.kind, ini.values = KVM_INIT_VALUES, keep.ctypes.data
        idx = self._check(lib().kvm_add_buffer(self._h, rows, cols, dtype, ctypes.byref(ini)), f'add_buffer {name}')
        self.names.append(name)
        self.shapes.append((rows, cols))
        self.dtypes.append(dtype)
        return idx

    def index(self, name) -> int:
        return self.names.index(name) if isinstance(name, str) else int(name)

    def read(self, name) -> np.ndarray:
        """f32 (bf16 widened) or int32 contents, flat."""
        i = self.index(name)
        r, c = self.shapes[i]
        if self.dtypes[i] == bl.DT_I32:
            out = np.empty(r * c, np.int32)
            self._check(lib().kvm_read_raw(self._h, i, out.ctypes.data, out.nbytes), 'read')
            return out
        out = np.empty(r * c, np.float32)
        self._check(lib().kvm_read_buffer(self._h, i, out.ctypes.data, out.size), 'read')
        return out

    def read_raw(self, name) -> np.ndarray:
        i = self.index(name)
        r, c = self.shapes[i]
        out = np.empty(r * c, {0: np.float32, 1: np.int32, 2: np.uint16}[self.dtypes[i]])
        self._check(lib().kvm_read_raw(self._h, i, out.ctypes.data, out.nbytes), 'read_raw')
        return out

    def write(self, name, data: np.ndarray):
        i = self.index(name)
        arr = _as_storage(np.asarray(data), self.dtypes[i])
        self._check(lib().kvm_write_buffer(self._h, i, arr.ctypes.data, arr.nbytes), 'write')

    def device_ptr(self, name) -> int:
        return lib().kvm_buffer_device_ptr(self._h, self.index(name))

    # ------------------------------------------------------------------ graph
    def set_version(self, var: int, v: int):
        self._check(lib().kvm_set_version(self._h, var, v), 'set_version')

    @staticmethod
    def _arrays(b: bl.LoadedBundle):
        t = np.ascontiguousarray(b.tasks, np.int32)
        s = np.ascontiguousarray(b.succ, np.int32) if b.succ.size else np.zeros(1, np.int32)
        a = np.ascontiguousarray(b.args, np.int32) if b.args.size else np.zeros(1, np.int32)
        return t, s, a

    def submit(self, b: bl.LoadedBundle) -> int:
        """kvm_submit. Stream mode: the bundle's window id."""
        t, s, a = self._arrays(b)
        rc = lib().kvm_submit(self._h, t.ctypes.data, t.shape[0], s.ctypes.data, int(b.succ.size), a.ctypes.data, int(b.args.size))
        self._check(rc, 'submit')
        return rc

    def submit_stream(self, b: bl.LoadedBundle, max_window_tasks: int = 0, timeout_ms: int = 60000) -> int:
        """kvm_submit_stream: one bundle larger than a window, in consecutive windows. Returns the number of windows."""
        t, s, a = self._arrays(b)
        rc = lib().kvm_submit_stream(self._h, t.ctypes.data, t.shape[0], s.ctypes.data, int(b.succ.size), a.ctypes.data, int(b.args.size),
                                     max_window_tasks, timeout_ms)
        self._check(rc, 'submit_stream')
        return rc

    def stream_close(self):
        """kvm_close: no bundle follows; the kernel ends once the admitted tasks have finished."""
        self._check(lib().kvm_close(self._h), 'close')

    def live_versions(self, n: int) -> np.ndarray:
        """Stream mode: the version variables as published so far (readable while the kernel runs)."""
        out = np.zeros(n, np.int32)
        self._check(lib().kvm_live_versions(self._h, out.ctypes.data, n), 'live_versions')
        return out

    def window_done(self, wid: int) -> bool:
        rc = lib().kvm_window_done(self._h, wid)
        self._check(rc, 'window_done')
        return rc == 1

    @classmethod
    def from_bundle(cls, src, buffers: list | None = None, **kw) -> 'Executor':
        """Executor with the bundle's buffer table (metadata init, or `buffers` arrays) and base versions; bundle submitted."""
        b = src if isinstance(src, bl.LoadedBundle) else bl.load(src)
        ex = cls(num_vars=len(b.metadata['variables']), **kw)
        for i, m in enumerate(b.metadata['buffers']):
            ex.add_buffer(m['name'], m['rows'], m['cols'], m['dtype'], init=m['init'], data=None if buffers is None else buffers[i], root=b.root)
        for v in b.metadata['variables']:
            ex.set_version(v['id'], v['base_version'])
        ex.submit(b)
        ex.meta = b.metadata
        return ex

    def set_classes(self, mode: int, classes: list):
        """Scheduler classes (include/kvm_exec.h, kvm_set_classes): classes[c] is a dict with weight, min_cta, max_cta,
        urgent_us, share, bw_cta, opaff (defaults 1, 0, UNLIMITED, 0, 1, UNLIMITED, False); a task's class is its
        workload_id. Before the first start."""
        arr = (KvmClassParams * max(1, len(classes)))()
        for c, d in enumerate(classes):
            arr[c] = KvmClassParams(d.get('weight', 1), d.get('min_cta', 0), d.get('max_cta', UNLIMITED), d.get('urgent_us', 0), d.get('share', 1),
                                    d.get('bw_cta', UNLIMITED), CLASS_OPAFF if d.get('opaff') else 0)
        self._check(lib().kvm_set_classes(self._h, mode, arr, len(classes)), 'set_classes')

    def set_sched_flags(self, flags: int, bw_limit: int = UNLIMITED):
        """Policy switches of the dynamic class scheduler (SCHED_F_*; default GUARANTEE | INHERIT) and the global cap on
        running bandwidth-bound tasks (ARBITER). Before the first start."""
        self._check(lib().kvm_set_sched_flags(self._h, flags, bw_limit), 'set_sched_flags')

    def set_affinity(self, affinity_us: int):
        """Task affinity window of the class scheduler (kvm_set_affinity): a released task is offered only to its
        preferred worker for affinity_us. Before the first start."""
        self._check(lib().kvm_set_affinity(self._h, affinity_us), 'set_affinity')

    def class_stats(self, n: int) -> np.ndarray:
        """Per-class counters of the last launch (CLASS_STATS_DTYPE; busy_ticks at 100 MHz)."""
        out = np.zeros(n, CLASS_STATS_DTYPE)
        m = self._check(lib().kvm_class_stats(self._h, out.ctypes.data, n), 'class_stats')
        return out[:m]

    def path(self) -> int:
        """PATH_DYNAMIC or PATH_STATIC: the path launches use (decided at the first start)."""
        return lib().kvm_path(self._h)

    def set_trace(self, on: bool):
        """Per-task tracing on / off for the following launches (needs an executor created with trace=True)."""
        self._check(lib().kvm_set_trace(self._h, int(on)), 'set_trace')

    def tracing(self) -> bool:
        """Whether the next launch traces (the last set_trace, else the creation's trace flag)."""
        return lib().kvm_get_trace(self._h) == 1

    def start(self):
        self._check(lib().kvm_start(self._h), 'start')

    def relaunch(self):
        self._check(lib().kvm_relaunch(self._h), 'relaunch')

    def finish(self, check: bool = True) -> dict:
        r = KvmResult()
        rc = lib().kvm_finish(self._h, ctypes.byref(r))
        res = {'err_code': r.err_code, 'err': ERRORS.get(r.err_code, str(r.err_code)), 'err_slot': r.err_slot, 'err_a': r.err_a,
               'err_b': r.err_b, 'done': r.done, 'admitted': r.admitted, 'grid': r.grid, 'kernel_ms': r.kernel_ms}
        if check and (rc < 0 or r.err_code):
            raise KvmError(f'run failed: {res} {lib().kvm_last_error(self._h).decode()}')
        return res

    def run(self, check: bool = True) -> dict:
        self.start()
        return self.finish(check)

    def run_timed(self, n: int) -> float:
        ms = ctypes.c_float()
        self._check(lib().kvm_run_timed(self._h, n, ctypes.byref(ms)), 'run_timed')
        return ms.value

    def run_timed_split(self, n: int) -> tuple[float, float]:
        """(total ms, persistent-kernel-only ms) of n back-to-back runs."""
        tot, exe = ctypes.c_float(), ctypes.c_float()
        self._check(lib().kvm_run_timed_split(self._h, n, ctypes.byref(tot), ctypes.byref(exe)), 'run_timed_split')
        return tot.value, exe.value

    def versions(self, n: int | None = None) -> np.ndarray:
        n = n if n is not None else max(1, len(self.meta['variables']) if self.meta else 1)
        out = np.zeros(n, np.int32)
        self._check(lib().kvm_versions(self._h, out.ctypes.data, n), 'versions')
        return out

    def trace(self) -> np.ndarray:
        n = lib().kvm_ntasks(self._h)
        out = np.zeros(n, TRACE_DTYPE)
        self._check(lib().kvm_trace(self._h, out.ctypes.data, n), 'trace')
        return out


def _as_storage(x: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == bl.DT_I32:
        return np.ascontiguousarray(x, np.int32)
    if dtype == bl.DT_BF16:
        if x.dtype == np.uint16:
            return np.ascontiguousarray(x)
        return bl.bf16_bits(np.asarray(x, np.float32))
    return np.ascontiguousarray(x, np.float32)


class MvmBuf(ctypes.Structure):
    _fields_ = [('p', ctypes.c_void_p), ('rows', ctypes.c_int32), ('cols', ctypes.c_int32), ('ld', ctypes.c_int32),
                ('dtype', ctypes.c_int32), ('reserved', ctypes.c_int32 * 2)]


def validate(b: bl.LoadedBundle) -> str | None:
    """Host-only bundle validation (the checks kvm_submit runs); None when valid, else the reason. Needs no GPU."""
    meta = b.metadata
    bufs = (MvmBuf * max(1, len(meta['buffers'])))()
    for i, m in enumerate(meta['buffers']):
        bufs[i] = MvmBuf(None, m['rows'], m['cols'], m['cols'], m['dtype'])
    t = np.ascontiguousarray(b.tasks, np.int32)
    s = np.ascontiguousarray(b.succ, np.int32) if b.succ.size else np.zeros(1, np.int32)
    a = np.ascontiguousarray(b.args, np.int32) if b.args.size else np.zeros(1, np.int32)
    err = ctypes.create_string_buffer(512)
    rc = lib().kvm_validate(t.ctypes.data, t.shape[0], s.ctypes.data, int(b.succ.size), a.ctypes.data, int(b.args.size), bufs,
                            len(meta['buffers']), max(1, len(meta['variables'])), err, 512)
    return None if rc == 0 else err.value.decode()


def op_name(op_id: int) -> str | None:
    r = lib().kvm_op_name(op_id)
    return r.decode() if r else None


def seeded_fill_test(seed, n, draws, bias, coef) -> np.ndarray:
    out = np.zeros(n, np.float32)
    if lib().kvm_seeded_fill_test(seed % 2**64, n, draws, bias, coef, out.ctypes.data) < 0:
        raise KvmError(lib().kvm_last_error(None).decode())
    return out


def copy_probe(nbytes: int) -> None:
    """One plain device copy of nbytes (kvm_copy_probe): the reference dispatch for HBM byte counters."""
    if lib().kvm_copy_probe(int(nbytes)) < 0:
        raise RuntimeError(lib().kvm_last_error(None).decode())


def run_noalloc(b: bl.LoadedBundle, buffer_ptrs: list[int], versions: list[int], blocks: int = 0, timeout_s: float = 20.0):
    """kvm_run_noalloc: runs bundle `b` on caller-owned device buffers (device addresses in metadata buffer order) with
    no device allocation. Returns (result dict, final versions)."""
    meta = b.metadata
    bufs = (MvmBuf * max(1, len(meta['buffers'])))()
    for i, (m, p) in enumerate(zip(meta['buffers'], buffer_ptrs)):
        bufs[i] = MvmBuf(p, m['rows'], m['cols'], m['cols'], m['dtype'])
    t = np.ascontiguousarray(b.tasks, np.int32)
    s = np.ascontiguousarray(b.succ, np.int32) if b.succ.size else np.zeros(1, np.int32)
    a = np.ascontiguousarray(b.args, np.int32) if b.args.size else np.zeros(1, np.int32)
    ver = np.array(list(versions) or [0], np.int32)
    r = KvmResult()
    err = ctypes.create_string_buffer(512)
    rc = lib().kvm_run_noalloc(t.ctypes.data, t.shape[0], s.ctypes.data, int(b.succ.size), a.ctypes.data, int(b.args.size), bufs,
                               len(meta['buffers']), ver.ctypes.data, ver.size, blocks, int(timeout_s * 1e6), None,
                               ctypes.byref(r), err, 512)
    res = {'rc': rc, 'err': err.value.decode(), 'err_code': r.err_code, 'err_slot': r.err_slot, 'done': r.done,
           'admitted': r.admitted, 'grid': r.grid}
    return res, ver.tolist()


def static_plan(b: bl.LoadedBundle, workers: int, dissolve: bool = False) -> dict:
    """kvm_static_plan: the static path's plan of bundle b for `workers` workers, computed on the host (no GPU).
    dissolve: the plan of untraced launches (ordering no-ops dissolved into wait sets; see include/kvm_exec.h)."""
    n = b.ntasks
    t = np.ascontiguousarray(b.tasks, np.int32)
    s = np.ascontiguousarray(b.succ, np.int32) if b.succ.size else np.zeros(1, np.int32)
    a = np.ascontiguousarray(b.args, np.int32) if b.args.size else np.zeros(1, np.int32)
    out = {k: np.zeros(n, np.int32) for k in ('worker', 'pos', 'nwaits', 'publishes')}
    stats = np.zeros(5, np.float64)
    cap = int(b.succ.size) + 2 * n + 1
    err = ctypes.create_string_buffer(512)
    while True:
        waits = np.zeros(2 * cap, np.int32)
        rc = lib().kvm_static_plan(t.ctypes.data, n, s.ctypes.data, int(b.succ.size), a.ctypes.data, int(b.args.size), workers,
                                   1 if dissolve else 0, out['worker'].ctypes.data, out['pos'].ctypes.data, out['nwaits'].ctypes.data,
                                   out['publishes'].ctypes.data, waits.ctypes.data, cap, stats.ctypes.data, err, 512)
        if rc < 0 and b'wait_cap' in err.value:
            cap *= 4
            continue
        break
    if rc < 0:
        raise KvmError(err.value.decode())
    out.update(makespan_us=float(stats[0]), work_us=float(stats[1]), cross_edges=int(stats[2]), edges=int(stats[3]),
               dissolved=int(stats[4]))
    w = waits.reshape(-1, 2)
    nt = int(out['nwaits'].sum())
    refs = w[:nt][w[:nt, 0] < 0]
    end = max([nt] + [int(st) + (-1 - int(c)) for c, st in refs])
    out['waits'] = w[:end].copy()
    return out
