"""Demo directories for the manifest runner `kvm_run` (reference: demo/mvm_run.cu; the frontend's demo writer,
frontend/mvmfe/demo.py).

A demo directory holds MANIFEST.json and the compiled bundles of its admissions (or, for an admission with a
`compile` entry, the workload file the runner compiles on demand). `Demo` writes one from workload specs (compiled
with kvm_amd.compiler). An admission's `publishes` maps a variable to the number of versions its bundle advances it
by: the live version after it completes is its base version plus that (frontend/mvmfe/demo.py:136).
"""
from __future__ import annotations

import json
from pathlib import Path

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
