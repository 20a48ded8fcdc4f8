"""Demo directories for the manifest runner `kvm_run` (reference: demo/mvm_run.cu; the frontend's demo writer and its
CPU runner, frontend/mvmfe/demo.py and mvmfe.run_manifest).

A demo directory holds MANIFEST.json and the compiled bundles of its admissions (or, for an admission with a
`compile` entry, the workload file the runner compiles on demand). `Demo` writes one from workload
specs (compiled with kvm_amd.compiler); `serial_order` and `replay` restate the runner's semantics on the CPU: the
admissions in the first order their conditions allow, each bundle shifted to its base versions and mapped onto the
manifest's buffer and variable tables, run on the oracle against shared buffers. Tests compare a GPU run of
`kvm_run` with `replay`; the oracle is test infrastructure, so `replay` imports it lazily and only there.
"""
from __future__ import annotations

import copy
import json
from pathlib import Path

import numpy as np

from . import abi
from . import bundle as bl
from . import compiler

DTYPE_NAMES = {bl.DT_F32: 'f32', bl.DT_I32: 'i32', bl.DT_BF16: 'bf16'}


class Demo:
    """Builds a demo directory: workloads, buffers (declared by their owner workload's bundle), admissions."""

    def __init__(self, root):
        self.root = Path(root)
        self.root.mkdir(parents=True, exist_ok=True)
        self.workloads, self.buffers, self.admissions, self.classes = {}, {}, [], {}

    def workload(self, name, variables=(), cls='default', priority=0):
        self.workloads[name] = {'file': f'{name}.json', 'tasks': 1, 'edges': 0, 'priority': priority, 'class': cls,
                                'variables': list(variables)}

    def bundle(self, workload, subdir, spec, base_versions=None) -> bl.LoadedBundle:
        """Compiles `spec` (base versions as given) into root/subdir; the workload's sizes grow to cover it."""
        b = compiler.compile_spec(spec, base_versions)
        b.write(self.root / subdir)
        (self.root / self.workloads[workload]['file']).write_text(json.dumps(spec))
        lb = bl.load(self.root / subdir)
        w = self.workloads[workload]
        w['tasks'], w['edges'] = max(w['tasks'], lb.ntasks), max(w['edges'], int(lb.succ.size))
        return lb

    def buffer(self, name, rows, cols, dtype, owner):
        self.buffers[name] = {'rows': rows, 'cols': cols, 'dtype': dtype, 'owner': owner}

    def workload_file(self, rel, spec):
        """Writes a workload JSON for an admission compiled on demand (its `compile` entry)."""
        p = self.root / rel
        p.parent.mkdir(parents=True, exist_ok=True)
        p.write_text(json.dumps(spec))

    def admission(self, name, workload, bundle_dir=None, after=(), when=(), at_us=None, base_versions=None, publishes=None,
                  compile=None):
        """compile: (workload file, data dir) relative to the root, compiled by the runner when no bundle applies."""
        a = {'name': name, 'workload': workload}
        if bundle_dir:
            a['bundle_dir'] = bundle_dir
        if compile:
            a['compile'] = {'workload': compile[0], 'data_dir': compile[1]}
        if after:
            a['after_bundles'] = list(after)
        if when:
            a['when'] = [dict(var=v, min=lo, **({} if hi is None else {'max': hi})) for v, lo, hi in when]
        if at_us is not None:
            a['at_us'] = at_us
        if base_versions:
            a['base_versions'] = dict(base_versions)
        if publishes:
            a['publishes'] = dict(publishes)
        self.admissions.append(a)

    def write(self) -> Path:
        m = {'manifest_version': 1, 'workloads': self.workloads, 'buffers': self.buffers, 'admissions': self.admissions}
        if self.classes:
            m['classes'] = self.classes
        (self.root / 'MANIFEST.json').write_text(json.dumps(m, indent=1))
        return self.root


def load(root) -> dict:
    return json.loads((Path(root) / 'MANIFEST.json').read_text())


def variables(m: dict) -> list:
    """The manifest's version variables in declaration order (workloads in order, each one's list in order)."""
    out = []
    for w in m['workloads'].values():
        for v in w.get('variables', []):
            if v not in out:
                out.append(v)
    return out


def serial_order(m: dict) -> list:
    """The runner's serial simulation: one admission at a time, the first in manifest order whose conditions hold;
    a publishing admission moves its variables from its base to the published version."""
    vs = variables(m)
    live = {v: 0 for v in vs}
    done, order = set(), []
    while len(order) < len(m['admissions']):
        pick = None
        for a in m['admissions']:
            if a['name'] in done:
                continue
            ok = all(d in done for d in a.get('after_bundles', []))
            ok = ok and all(c['min'] <= live[c['var']] <= c.get('max', 1 << 62) for c in a.get('when', []))
            ok = ok and all(live[v] == a['base_versions'][v] for v in a.get('publishes', {}))
            if ok:
                pick = a
                break
        if pick is None:
            raise ValueError(f'the manifest cannot complete after {order}')
        done.add(pick['name'])
        order.append(pick['name'])
        live.update(pick.get('publishes', {}))
    return order


def _rebase(b: bl.LoadedBundle, to: dict) -> bl.LoadedBundle:
    """Version shift of the variables the bundle publishes to the target base versions."""
    b = copy.deepcopy(b)
    names = {v['id']: v['name'] for v in b.metadata['variables']}
    base = {v['name']: v['base_version'] for v in b.metadata['variables']}
    t = b.tasks
    for vid, name in names.items():
        if not (t[:, 10] == vid).any() or name not in to or to[name] == base[name]:
            continue
        d = to[name] - base[name]
        t[t[:, 10] == vid, 11] += d
        t[t[:, 8] == vid, 9] += d
        for v in b.metadata['variables']:
            if v['id'] == vid:
                v['base_version'] = to[name]
    return b


def _remap(b: bl.LoadedBundle, buf_names: list, var_names: list) -> bl.LoadedBundle:
    """Local buffer and variable ids onto the manifest's tables."""
    b = copy.deepcopy(b)
    bmap = {m['index'] if 'index' in m else i: buf_names.index(m['name']) for i, m in enumerate(b.metadata['buffers'])}
    vmap = {v['id']: var_names.index(v['name']) for v in b.metadata['variables']}
    ops = abi.ops_by_id()
    for t in b.tasks:
        op = ops[int(t[0])]
        for k, arg in enumerate(op.args):
            if arg.type == 'buf' and b.args[t[6] + k] >= 0:
                b.args[t[6] + k] = bmap[int(b.args[t[6] + k])]
        for j in (8, 10):
            if t[j] >= 0:
                t[j] = vmap[int(t[j])]
    return b


def replay(root, init: dict | None = None) -> dict:
    """Runs the manifest serially on the CPU oracle. init: name -> initial array (default: each buffer's owner bundle
    metadata init). Returns dict(buffers={name: array}, versions={var: v}, order=[admission names])."""
    import oracle
    root = Path(root)
    m = load(root)
    vs = variables(m)
    names = list(m['buffers'])
    adm = {a['name']: a for a in m['admissions']}
    bundles, last = {}, {}
    for a in m['admissions']:
        d = a.get('bundle_dir')
        if d and (root / d / 'metadata.json').exists():
            b = bl.load(root / d)
        elif a['workload'] in last:
            b = last[a['workload']]
        else:       # compiled on demand for the admission's base versions
            c = a['compile']
            b = bl.load(compiler.compile_spec(json.loads((root / c['workload']).read_text()), a.get('base_versions'),
                                              data_dir=root / c.get('data_dir', '.')))
        if a.get('publishes'):
            b = _rebase(b, a['base_versions'])
        last[a['workload']] = b
        bundles[a['name']] = b
    bufs = {}
    for n, d in m['buffers'].items():
        if init and n in init:
            bufs[n] = np.array(init[n], copy=True)
            continue
        owner = next(a for a in m['admissions'] if a['workload'] == d['owner'])
        meta = next(x for x in bundles[owner['name']].metadata['buffers'] if x['name'] == n)
        bufs[n] = bl.materialize(meta, bundles[owner['name']].root)
    live = {v: 0 for v in vs}
    order = serial_order(m)
    for name in order:
        b = _remap(bundles[name], names, vs)
        meta = {'buffers': [{'name': n, 'rows': d['rows'], 'cols': d['cols'],
                             'dtype': {'f32': bl.DT_F32, 'i32': bl.DT_I32, 'bf16': bl.DT_BF16}[d['dtype']]} for n, d in m['buffers'].items()],
                'variables': [{'name': v, 'id': i, 'base_version': live[v]} for i, v in enumerate(vs)], 'reads': []}
        g = bl.LoadedBundle(meta, b.tasks, b.succ, b.args, b.root)
        out = oracle.run(g, [bufs[n] for n in names])
        bufs = dict(zip(names, out['buffers']))
        live.update({v: int(out['versions'][v]) for v in vs if v in out['versions']})
        live.update(adm[name].get('publishes', {}))
    return {'buffers': bufs, 'versions': live, 'order': order}
