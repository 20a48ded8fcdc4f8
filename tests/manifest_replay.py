"""The CPU replay of a manifest, the checker the manifest-runner tests compare `kvm_run` with (reference semantics:
demo/mvm_run.cu and its CPU counterpart frontend/mvmfe/run_manifest.py).

`serial_order` is the runner's dry run: admissions one at a time, the first in manifest order whose gate is open
(after_bundles finished, every `when` window holding, every published variable at the admission's base version);
a completed admission advances each variable it publishes BY its `publishes` value (frontend/mvmfe/demo.py:136,
demo/mvm_run.cu:262). `replay` runs the admissions in that order on the oracle against one shared set of buffers,
each bundle moved to its admission's base versions and bound to the manifest's buffer and variable tables.
"""
from __future__ import annotations

import copy
import json
from pathlib import Path

import numpy as np

from kvm_amd import abi
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.manifest import load, variables

_DT = {'f32': bl.DT_F32, 'i32': bl.DT_I32, 'bf16': bl.DT_BF16}


def _gate_open(a, live, finished):
    if any(d not in finished for d in a.get('after_bundles', [])):
        return False
    if any(not (c['min'] <= live[c['var']] <= c.get('max', 1 << 62)) for c in a.get('when', [])):
        return False
    return all(live[v] == a['base_versions'][v] for v in a.get('publishes', {}))


def serial_order(m: dict) -> list:
    live = {v: 0 for v in variables(m)}
    finished, order = set(), []
    while len(order) < len(m['admissions']):
        nxt = next((a for a in m['admissions'] if a['name'] not in finished and _gate_open(a, live, finished)), None)
        if nxt is None:
            raise ValueError(f'the version flow is stuck after {order}')
        finished.add(nxt['name'])
        order.append(nxt['name'])
        for v, inc in nxt.get('publishes', {}).items():
            live[v] += inc
    return order


def _move_versions(b: bl.LoadedBundle, target: dict) -> bl.LoadedBundle:
    """Shifts the waits and publications of every variable the bundle publishes to the target base version."""
    b = copy.deepcopy(b)
    for v in b.metadata['variables']:
        vid, name = v['id'], v['name']
        pub = b.tasks[:, 10] == vid
        if not pub.any() or name not in target or target[name] == v['base_version']:
            continue
        d = target[name] - v['base_version']
        b.tasks[pub, 11] += d
        b.tasks[b.tasks[:, 8] == vid, 9] += d
        v['base_version'] = target[name]
    return b


def _bind(b: bl.LoadedBundle, buf_names: list, var_names: list) -> bl.LoadedBundle:
    b = copy.deepcopy(b)
    bmap = {e.get('index', i): buf_names.index(e['name']) for i, e in enumerate(b.metadata['buffers'])}
    vmap = {v['id']: var_names.index(v['name']) for v in b.metadata['variables']}
    ops = abi.ops_by_id()
    for t in b.tasks:
        for k, arg in enumerate(ops[int(t[0])].args):
            w = t[6] + k
            if arg.type == 'buf' and b.args[w] >= 0:
                b.args[w] = bmap[int(b.args[w])]
        for j in (8, 10):
            if t[j] >= 0:
                t[j] = vmap[int(t[j])]
    return b


def replay(root, init: dict | None = None) -> dict:
    """init: buffer name -> initial array (default: the owner bundle's declared init). Returns
    dict(buffers={name: array}, versions={var: version}, order=[admission names])."""
    import oracle
    root = Path(root)
    m = load(root)
    vs = variables(m)
    names = list(m['buffers'])
    adm = {a['name']: a for a in m['admissions']}
    bundles, previous = {}, {}
    for a in m['admissions']:
        d = a.get('bundle_dir')
        if d and (root / d / 'metadata.json').exists():
            b = bl.load(root / d)
        elif a['workload'] in previous:
            b = previous[a['workload']]
        else:
            c = a['compile']
            b = bl.load(compiler.compile_spec(json.loads((root / c['workload']).read_text()), a.get('base_versions'),
                                              data_dir=root / c.get('data_dir', '.')))
        if a.get('publishes'):
            b = _move_versions(b, a['base_versions'])
        previous[a['workload']] = b
        bundles[a['name']] = b
    bufs = {}
    for n, d in m['buffers'].items():
        if init and n in init:
            bufs[n] = np.array(init[n], copy=True)
            continue
        owner = next(a for a in m['admissions'] if a['workload'] == d['owner'])
        decl = next(x for x in bundles[owner['name']].metadata['buffers'] if x['name'] == n)
        bufs[n] = bl.materialize(decl, bundles[owner['name']].root)
    live = {v: 0 for v in vs}
    order = serial_order(m)
    table = [{'name': n, 'rows': d['rows'], 'cols': d['cols'], 'dtype': _DT[d['dtype']]} for n, d in m['buffers'].items()]
    for name in order:
        b = _bind(bundles[name], names, vs)
        meta = {'buffers': table, 'variables': [{'name': v, 'id': i, 'base_version': live[v]} for i, v in enumerate(vs)], 'reads': []}
        out = oracle.run(bl.LoadedBundle(meta, b.tasks, b.succ, b.args, b.root), [bufs[n] for n in names])
        bufs = dict(zip(names, out['buffers']))
        for v, inc in adm[name].get('publishes', {}).items():
            assert int(out['versions'][v]) == live[v] + inc, (name, v, out['versions'][v], live[v], inc)
            live[v] += inc
    return {'buffers': bufs, 'versions': live, 'order': order}
