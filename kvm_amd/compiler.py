"""Workload JSON -> task bundle (ABI v2): this project's restatement of the reference's bundle compiler.

The output format is the reference's (reference: runtime/compile_workload.py:624-713): ``tasks.bin`` (64-byte
descriptors), ``successors.bin`` (int32 CSR, successor lists ascending), ``args.bin`` (int32 argument words, f32 as IEEE
bits) and ``metadata.json``. For the same workload the bytes are identical to the reference compiler's; the tests pin
that against bundles the reference compiler wrote (tests/golden).

Semantics kept from the reference:
  * every ``publishes`` task numbers the variable's next version in declaration order (compile_workload.py:452-465);
  * each read waits for its version; reads beyond a task's first waiting read get a ``noop`` gate task inserted just
    before the task (compile_workload.py:497-522);
  * an ``exact`` read of version N adds a write-after-read edge to the publisher of N+1 (compile_workload.py:470-485);
  * the first publisher of a variable with base version > 0 waits for the live head (compile_workload.py:486-494);
  * the graph must be acyclic and every variable's publishers totally ordered (compile_workload.py:581-598).
Operand extent checks are enforced by the executor at run time (error codes), not here.
"""
from __future__ import annotations

import json
import math
import shutil
import struct
from array import array
from dataclasses import dataclass, field
from pathlib import Path

from . import abi
from .initgen import params as seeded_params

I32_MIN, I32_MAX = -2**31, 2**31 - 1
F32_MAX = 3.4028234663852886e38
DTYPES = {'f32': 0, 'i32': 1, 'bf16': 2}
_F = struct.Struct('<f')
_I = struct.Struct('<i')


class CompileError(ValueError):
    pass


def _need(ok, msg):
    if not ok:
        raise CompileError(msg)


def f32(x: float) -> float:
    return _F.unpack(_F.pack(x))[0]


def bf16(x: float) -> float:
    """float32 value rounded to bfloat16, nearest even; inf/nan kept."""
    if x != x or math.isinf(x):
        return x
    u = struct.unpack('<I', _F.pack(x))[0]
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return struct.unpack('<f', struct.pack('<I', u))[0]


@dataclass
class Buffer:
    name: str
    index: int
    rows: int
    cols: int
    dtype: str
    init: dict

    @property
    def numel(self):
        return self.rows * self.cols


@dataclass
class Variable:
    name: str
    id: int
    base: int
    final: int


@dataclass
class Read:
    var: str
    policy: str
    version: int
    wait_ver: int
    waits: bool
    implicit: bool = False
    gate: int | None = None        # final index of the gate task carrying the wait


@dataclass
class Task:
    name: str
    graph: int
    op: abi.Op
    words: list
    priority: int = 0
    deadline_us: int = -1
    after: list = field(default_factory=list)
    publishes: str | None = None
    decl_reads: list = field(default_factory=list)
    reads: list = field(default_factory=list)
    wait: tuple | None = None
    pub: tuple | None = None
    gate: bool = False


@dataclass
class Bundle:
    metadata: dict
    tasks: bytes
    successors: bytes
    args: bytes
    names: list
    buffers: list
    variables: list
    data_dir: Path | None = None

    def write(self, out_dir) -> Path:
        """Writes the bundle directory; `file` initial values are copied in under their relative path
        (reference: runtime/compile_workload.py:693-713)."""
        d = Path(out_dir)
        files = [b for b in self.buffers if b.init['kind'] == 'file']
        _need(not files or self.data_dir is not None, f'buffers {[b.name for b in files][:4]} use file init: compile with a data_dir')
        d.mkdir(parents=True, exist_ok=True)
        for b in files:
            src, dst = self.data_dir / b.init['path'], d / b.init['path']
            if src.resolve() != dst.resolve():
                dst.parent.mkdir(parents=True, exist_ok=True)
                shutil.copyfile(src, dst)
        (d / 'tasks.bin').write_bytes(self.tasks)
        (d / 'successors.bin').write_bytes(self.successors)
        (d / 'args.bin').write_bytes(self.args)
        with open(d / 'metadata.json', 'w') as f:
            json.dump(self.metadata, f, indent=2)
            f.write('\n')
        return d


# ------------------------------------------------------------------------------------------------ parsing
def _num_f32(x, where):
    _need(isinstance(x, (int, float)) and not isinstance(x, bool), f'{where}: expected a number, got {x!r}')
    v = float(x)
    _need(math.isfinite(v) and abs(v) <= F32_MAX, f'{where}: {x!r} is not a finite float32')
    return f32(v)


def _num_i32(x, where):
    _need(isinstance(x, int) or (isinstance(x, float) and x.is_integer()), f'{where}: integer expected, got {x!r}')
    _need(I32_MIN <= x <= I32_MAX, f'{where}: {x} overflows int32')
    return int(x)


def _init(where, init, n, dtype, data_dir=None):
    _need(isinstance(init, dict) and 'kind' in init, f'{where}: init needs a kind')
    conv = {'f32': _num_f32, 'i32': _num_i32, 'bf16': lambda x, w: bf16(_num_f32(x, w))}[dtype]
    k = init['kind']
    if k == 'fill':
        return {'kind': 'fill', 'value': conv(init['value'], where)}
    if k == 'values':
        vals = init['values']
        _need(isinstance(vals, list) and len(vals) == n, f'{where}: init.values needs {n} numbers')
        return {'kind': 'values', 'values': [conv(x, where) for x in vals]}
    if k == 'seeded':
        _need(dtype == 'f32', f'{where}: seeded init needs dtype f32')
        seed, dist = init['seed'], init.get('dist', 'normal')
        _need(isinstance(seed, int) and 0 <= seed < 2**63, f'{where}: seed must be in [0, 2^63)')
        scale = _num_f32(init['scale'], where)
        _need(scale >= 0, f'{where}: scale must be >= 0')
        draws, bias, coef = seeded_params(dist, scale)
        return {'kind': 'seeded', 'seed': seed, 'scale': scale, 'dist': dist, 'draws': draws, 'bias': bias, 'coef': coef}
    if k == 'file':
        p = init['path']
        _need(isinstance(p, str) and p and not Path(p).is_absolute() and '..' not in Path(p).parts and '\\' not in p,
              f'{where}: bad init.path')
        if data_dir is not None:      # validated when the data directory is known (compile_workload.py:237-241)
            f = Path(data_dir) / p
            _need(f.is_file(), f'{where}: init file {str(f)!r} not found')
            want = (2 if dtype == 'bf16' else 4) * n
            _need(f.stat().st_size == want, f'{where}: init file {p!r} has {f.stat().st_size} bytes, expected {want}')
        return {'kind': 'file', 'path': Path(p).as_posix()}
    raise CompileError(f'{where}: unknown init kind {k!r}')


def _args(where, op, raw, buffers):
    _need(isinstance(raw, dict), f'{where}: args must be an object')
    names = [a.name for a in op.args]
    _need(set(raw) == set(names), f'{where}: op {op.name} takes {names}, got {sorted(raw)}')
    words = []
    for a in op.args:
        v = raw[a.name]
        if a.type == 'buf':
            if v is None:
                _need(a.optional, f'{where}: {a.name} is a required buffer')
                words.append(abi.ABSENT_BUF)
            else:
                _need(isinstance(v, str) and v in buffers, f'{where}: {a.name}: unknown buffer {v!r}')
                words.append(buffers[v].index)
        elif a.type == 'i32':
            _need(isinstance(v, int) and not isinstance(v, bool) and I32_MIN <= v <= I32_MAX, f'{where}: {a.name}: int32 expected')
            words.append(v)
        else:
            _need(isinstance(v, (int, float)) and not isinstance(v, bool), f'{where}: {a.name}: number expected')
            try:
                packed = _F.pack(v)
            except OverflowError:
                raise CompileError(f'{where}: {a.name}: {v!r} overflows float32') from None
            w = _I.unpack(packed)[0]
            _need((w >> 23) & 0xFF != 0xFF, f'{where}: {a.name}: non-finite value')
            words.append(w)
    return words


# ------------------------------------------------------------------------------------------------ graph
def _csr(preds):
    n = len(preds)
    outs = [[] for _ in range(n)]
    for i, ps in enumerate(preds):
        for p in ps:
            outs[p].append(i)
    off = array('i', [0])
    succ = array('i')
    for o in outs:
        succ.extend(o)
        off.append(len(succ))
    indeg = array('i', (len(p) for p in preds))
    return off, succ, indeg


def _topo(off, succ, indeg):
    rem = array('i', indeg)
    order = [i for i in range(len(indeg)) if rem[i] == 0]
    h = 0
    while h < len(order):
        i = order[h]
        h += 1
        for k in range(off[i], off[i + 1]):
            j = succ[k]
            rem[j] -= 1
            if rem[j] == 0:
                order.append(j)
    if len(order) != len(indeg):
        return None
    pos = [0] * len(indeg)
    for p, i in enumerate(order):
        pos[i] = p
    return pos


def _reaches(off, succ, pos, a, b):
    if a == b:
        return True
    if pos[a] > pos[b]:
        return False
    stack, seen = [a], {a}
    while stack:
        i = stack.pop()
        for k in range(off[i], off[i + 1]):
            j = succ[k]
            if j == b:
                return True
            if j not in seen and pos[j] < pos[b]:
                seen.add(j)
                stack.append(j)
    return False


# ------------------------------------------------------------------------------------------------ compile
def compile_spec(spec: dict, base_versions: dict | None = None, ops: dict | None = None, data_dir=None) -> Bundle:
    """`data_dir`: where `file` initial values are read from (checked here, copied by Bundle.write); None leaves them
    unchecked, and writing such a bundle is then refused."""
    ops = ops or abi.load_ops()
    _need(isinstance(spec, dict) and 'graphs' in spec and set(spec) <= {'variables', 'buffers', 'graphs'},
          'workload: keys are variables, buffers, graphs (graphs required)')
    base_versions = dict(base_versions or {})
    vnames = spec.get('variables', [])
    _need(len(set(vnames)) == len(vnames), 'duplicate variable names')
    _need(not set(base_versions) - set(vnames), 'base_versions names undeclared variables')
    variables = {n: Variable(n, i, base_versions.get(n, 0), base_versions.get(n, 0)) for i, n in enumerate(vnames)}

    buffers = {}
    for i, d in enumerate(spec.get('buffers', [])):
        name = d['name']
        _need(name not in buffers, f'duplicate buffer {name!r}')
        rows, cols, dt = d.get('rows', 1), d.get('cols', 1), d.get('dtype', 'f32')
        _need(isinstance(rows, int) and isinstance(cols, int) and rows >= 1 and cols >= 1 and rows * cols <= I32_MAX,
              f'buffer {name!r}: bad shape')
        _need(dt in DTYPES, f'buffer {name!r}: bad dtype {dt!r}')
        init = _init(f'buffer {name!r}', d.get('init', {'kind': 'fill', 'value': 0}), rows * cols, dt, data_dir)
        buffers[name] = Buffer(name, len(buffers), rows, cols, dt, init)

    decls = []
    for gi, g in enumerate(spec['graphs']):
        gname = g['name']
        _need(isinstance(gname, str) and gname and '/' not in gname, f'graphs[{gi}]: bad name')
        base = len(decls)
        index = {}
        for ti, t in enumerate(g['tasks']):
            _need(t['id'] not in index, f'graph {gname!r}: duplicate task id {t["id"]!r}')
            index[t['id']] = base + ti
        for t in g['tasks']:
            where = f"{gname}/{t['id']}"
            op = ops.get(t['op'])
            _need(op is not None, f'{where}: unknown op {t["op"]!r}')
            words = _args(where, op, t.get('args', {}), buffers)
            try:
                deps = [index[x] for x in t.get('after', ())]
            except KeyError as e:
                raise CompileError(f'{where}: after names unknown task {e.args[0]!r}') from None
            _need(len(set(deps)) == len(deps) and len(decls) not in deps, f'{where}: bad after list')
            pub = t.get('publishes')
            _need(pub is None or pub in variables, f'{where}: publishes undeclared variable {pub!r}')
            reads = []
            for r in t.get('reads', ()):
                _need(r['var'] in variables and r['policy'] in ('exact', 'at_least') and isinstance(r['version'], int)
                      and r['version'] >= 0, f'{where}: bad read {r!r}')
                _need(all(x[0] != r['var'] for x in reads), f'{where}: reads {r["var"]!r} twice')
                reads.append((r['var'], r['policy'], r['version']))
            decls.append(Task(where, gi, op, words, t.get('priority', 0), t.get('deadline_us', -1), deps, pub, reads))

    # versions
    pubs = {v: [] for v in variables}
    for i, t in enumerate(decls):
        if t.publishes:
            v = variables[t.publishes]
            v.final += 1
            pubs[t.publishes].append(i)
            t.pub = (v.name, v.final)
    by_ver = {v: {variables[v].base + k + 1: i for k, i in enumerate(ix)} for v, ix in pubs.items()}
    exact_edges = []
    for i, t in enumerate(decls):
        for var, pol, n in t.decl_reads:
            v = variables[var]
            if pol == 'exact':
                _need(n >= v.base, f'{t.name}: exact read of {var!r} at {n} is stale (base {v.base})')
            if n > v.base:
                _need(n in by_ver[var], f'{t.name}: read of {var!r} at {n} can never be satisfied')
            nxt = by_ver[var].get(n + 1)
            if pol == 'exact' and nxt is not None and nxt != i:
                exact_edges.append((i, nxt))
            t.reads.append(Read(var, pol, n, n, n > 0))
    for var, ix in pubs.items():
        b = variables[var].base
        if ix and b > 0:
            t = decls[ix[0]]
            own = next((r for r in t.reads if r.var == var), None)
            if own:
                own.wait_ver = max(own.wait_ver, b)
            else:
                t.reads.append(Read(var, 'at_least', b, b, True, implicit=True))

    # gates and edges
    noop = ops['noop']
    tasks, final, gates_of = [], [0] * len(decls), {}
    for i, t in enumerate(decls):
        waiting = [r for r in t.reads if r.waits]
        for k, r in enumerate(waiting[1:], 1):
            g = Task(f'__gate/{t.name}/{k}', t.graph, noop, [], t.priority, t.deadline_us, gate=True)
            g.wait = (r.var, r.wait_ver)
            r.gate = len(tasks)
            gates_of.setdefault(i, []).append(len(tasks))
            tasks.append(g)
        final[i] = len(tasks)
        if waiting:
            t.wait = (waiting[0].var, waiting[0].wait_ver)
        tasks.append(t)
    preds = [[] for _ in tasks]
    for i, t in enumerate(decls):
        preds[final[i]] = gates_of.get(i, []) + [final[j] for j in t.after]
    for r, nx in exact_edges:
        if final[r] not in preds[final[nx]]:
            preds[final[nx]].append(final[r])
    off, succ, indeg = _csr(preds)
    pos = _topo(off, succ, indeg)
    _need(pos is not None, 'dependency cycle (possibly through an exact read\'s write-after-read edge)')
    for var, ix in pubs.items():
        for a, b in zip(ix, ix[1:]):
            _need(_reaches(off, succ, pos, final[a], final[b]), f'unordered publishers of {var!r}: {decls[a].name}, {decls[b].name}')
    for i, t in enumerate(decls):
        for r in t.reads:
            if r.wait_ver > variables[r.var].base:
                p = by_ver[r.var][r.wait_ver]
                _need(not _reaches(off, succ, pos, final[i], final[p]), f'{t.name}: waits for a publisher ordered after it (deadlock)')

    # pack
    used = {t.op.name for t in tasks}
    vid = {n: v.id for n, v in variables.items()}
    desc, words = bytearray(), array('i')
    for i, t in enumerate(tasks):
        wv, wn = (vid[t.wait[0]], t.wait[1]) if t.wait else (abi.NO_VAR, 0)
        pv, pn = (vid[t.pub[0]], t.pub[1]) if t.pub else (abi.NO_VAR, 0)
        desc += abi.DESC.pack(t.op.id, off[i], off[i + 1] - off[i], indeg[i], t.priority, t.deadline_us, len(words),
                              len(t.words), wv, wn, pv, pn, t.graph, 0, 0, 0)
        words.extend(t.words)
    meta = {
        'abi_version': abi.ABI_VERSION, 'task_count': len(tasks), 'edge_count': len(succ), 'args_words': len(words),
        'task_names': [t.name for t in tasks],
        'initial_ready': [i for i in range(len(tasks)) if indeg[i] == 0],
        'operator_ids': {n: o.id for n, o in ops.items() if o.id < abi.EXT_ID_MIN or n in used},
        'buffers': [{'name': b.name, 'index': b.index, 'rows': b.rows, 'cols': b.cols, 'dtype': DTYPES[b.dtype], 'init': b.init}
                    for b in buffers.values()],
        'variables': [{'name': v.name, 'id': v.id, 'base_version': v.base} for v in variables.values()],
        'publishers': [{'task': i, 'name': t.name, 'var': vid[t.pub[0]], 'version': t.pub[1]} for i, t in enumerate(tasks) if t.pub],
        'reads': [{'task': i, 'name': t.name, 'var': vid[r.var], 'policy': r.policy, 'version': r.version,
                   'observed': r.version if r.policy == 'exact' else None, 'gate': r.gate}
                  for i, t in enumerate(tasks) if not t.gate for r in t.reads if not r.implicit],
        'final_versions': {v.name: v.final for v in variables.values()},
    }
    return Bundle(meta, bytes(desc), succ.tobytes(), words.tobytes(), [t.name for t in tasks], list(buffers.values()),
                  list(variables.values()), Path(data_dir) if data_dir is not None else None)


def main(argv=None):
    import argparse
    p = argparse.ArgumentParser(description='compile a workload JSON into a task bundle directory')
    p.add_argument('workload')
    p.add_argument('out_dir')
    p.add_argument('--base-versions', action='append', default=[], help='var=N,... (repeatable)')
    p.add_argument('--data-dir', help='where `file` initial values live (default: the workload file directory)')
    a = p.parse_args(argv)
    base = {}
    for item in filter(None, ','.join(a.base_versions).split(',')):
        k, _, v = item.partition('=')
        base[k] = int(v)
    data_dir = Path(a.data_dir) if a.data_dir else Path(a.workload).resolve().parent
    compile_spec(json.loads(Path(a.workload).read_text()), base, data_dir=data_dir).write(a.out_dir)


if __name__ == '__main__':
    main()
