"""Workload generators: task graphs (workload JSON in the reference's schema) for the benchmark configurations.

The reference's frontend has no generator for these exact configurations (tied-embedding GPT with learned positions,
Qwen3-shape decode), so they are built here from the registry operators. A generator returns a `Workload`: the
workload JSON dict plus executor-side buffer initialisers (`init_override`) for bf16 buffers, which the bundle format
can only declare as fill/values/file (the reference compiler refuses `seeded` for bf16).
"""
from __future__ import annotations

import zlib
from dataclasses import dataclass, field


@dataclass
class Workload:
    spec: dict
    init_override: dict = field(default_factory=dict)     # buffer name -> init dict (seeded bf16)
    info: dict = field(default_factory=dict)              # workload facts (bytes/flops per step, task counts)


def split(n: int, parts: int):
    """[lo, hi) ranges covering [0, n) in `parts` near-equal pieces (no empty piece)."""
    parts = max(1, min(parts, n))
    q, r = divmod(n, parts)
    out, lo = [], 0
    for i in range(parts):
        hi = lo + q + (1 if i < r else 0)
        out.append((lo, hi))
        lo = hi
    return out


def seed_of(seed: int, name: str) -> int:
    """Per-buffer seed, crc32 of 'seed/name' (the reference frontend's convention, frontend/mvmfe/train.py:122-124)."""
    return zlib.crc32(f'{seed}/{name}'.encode()) & 0x7FFFFFFF


class Builder:
    """Accumulates buffers and tasks of one graph. Tasks get sequential ids; `after` takes task ids."""

    def __init__(self, seed: int = 0):
        self.buffers, self.tasks, self.variables = [], [], []
        self.init_override = {}
        self.seed = seed
        self._n = 0
        self._names = set()

    def buf(self, name, rows, cols=1, dtype='f32', init=None):
        assert name not in self._names, name
        self._names.add(name)
        d = {'name': name, 'rows': rows, 'cols': cols, 'dtype': dtype}
        if init is not None:
            d['init'] = init
        self.buffers.append(d)
        return name

    def normal(self, name, rows, cols=1, dtype='f32', scale=0.02, seed_name=None):
        """Seeded N(0, scale) (Irwin-Hall(4), the reference's `normal`); bf16 buffers get it as an executor override.
        `seed_name`: draw the values of that buffer instead (a bf16 buffer then holds the other one's values rounded)."""
        init = {'kind': 'seeded', 'seed': seed_of(self.seed, seed_name or name), 'scale': scale, 'dist': 'normal'}
        if dtype == 'bf16':
            from ..initgen import params
            draws, bias, coef = params('normal', scale)
            self.init_override[name] = {**init, 'draws': draws, 'bias': bias, 'coef': coef}
            return self.buf(name, rows, cols, dtype, {'kind': 'fill', 'value': 0})
        return self.buf(name, rows, cols, dtype, init)

    def fill(self, name, rows, cols=1, dtype='f32', value=0.0):
        return self.buf(name, rows, cols, dtype, {'kind': 'fill', 'value': value})

    def values(self, name, vals, rows, cols=1, dtype='i32'):
        return self.buf(name, rows, cols, dtype, {'kind': 'values', 'values': list(vals)})

    def task(self, op, after=(), publishes=None, reads=None, **args):
        tid = f't{self._n}'
        self._n += 1
        t = {'id': tid, 'op': op, 'args': args}
        after = list(after)
        if after:
            t['after'] = after
        if publishes:
            t['publishes'] = publishes
        if reads:
            t['reads'] = reads
        self.tasks.append(t)
        return tid

    def join(self, preds, succ_count_hint=0):
        """A dependency point after all of `preds`: the preds themselves when few, else one noop they all feed
        (keeps the edge count linear for wide-to-wide phase boundaries)."""
        preds = list(preds)
        if len(preds) <= 2 or succ_count_hint <= 2:
            return preds
        return [self.task('noop', after=preds)]

    def spec(self, graph='g'):
        s = {'buffers': self.buffers, 'graphs': [{'name': graph, 'tasks': self.tasks}]}
        if self.variables:
            s['variables'] = self.variables
        return s
