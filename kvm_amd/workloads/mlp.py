"""eight independent MLPs trained together in one task graph (one persistent launch).

Each MLP i is 784 -> w_i -> w_i -> 10 with ReLU, w_i in {64, 96, 128, 192, 256, 384, 512, 768}, batch 256, f32,
softmax cross-entropy and AdamW, `steps` training steps unrolled into the graph. Inputs are seeded N(0, 1), labels
uniform in [0, 10), weights seeded N(0, 1/sqrt(fan_in)), biases 0. The reference ships no generator for this
configuration (its small-MLP panel, bench/exec_vs_torch/gen_mlp.py, trains other shapes), so it is built here from
registry operators, per MLP and step:

  z1 = x W1^T + b1 (matmul_tile, bias epilogue) -> a1 = relu(z1) (act_fwd) -> z2 = a1 W2^T + b2 -> a2 = relu(z2) ->
  logits = a2 W3^T + b3 -> softmax_ce_fused (loss rows + dlogits) -> softmax_ce_reduce -> backward: dW3 = dlogits^T a2,
  db3 = colsum, da2 = dlogits W3 -> dz2 = relu'(z2) da2 (act_bwd) -> dW2, db2, da1 -> dz1 -> dW1, db1 -> AdamW on every
  parameter chunk (one step counter per MLP, no gradient clipping).

The MLPs share nothing, so their task chains interleave freely: many small heterogeneous GEMM tiles, the scheduler-
stress case. Dependencies come from the same rectangle tracker as the GPT generator.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, asdict

from . import Workload, split
from .gpt import GPTBuilder, GPTConfig, Deps, row_chunks

WIDTHS = (64, 96, 128, 192, 256, 384, 512, 768)


@dataclass
class MLPConfig:
    widths: tuple = WIDTHS
    d_in: int = 784
    classes: int = 10
    batch: int = 256
    steps: int = 50
    lr: float = 1e-3
    b1: float = 0.9
    b2: float = 0.95
    wd: float = 0.1
    eps: float = 1e-8
    seed: int = 4242
    row_tasks: int = 8           # row-parallel split of the elementwise / loss phases per MLP
    opt_chunk: int = 12288       # elements per AdamW task (measured with row_tasks 8: 341 us/step; 4 / 49152: 384)


def param_count(c: MLPConfig) -> int:
    return sum(w * c.d_in + w + w * w + w + c.classes * w + c.classes for w in c.widths)


def step_flops(c: MLPConfig) -> float:
    """GEMM FLOPs of one training step of all MLPs (forward + both backward products)."""
    return sum(6.0 * c.batch * (c.d_in * w + w * w + w * c.classes) for w in c.widths)


class MLPBuilder(GPTBuilder):
    def __init__(self, c: MLPConfig):
        super().__init__(GPTConfig(layers=0, d=8, heads=1, T=1, vocab=8, ffn=8, batch=1, dtype='f32', seed=c.seed,
                                   tasks_target=c.row_tasks))
        self.m = c
        self.READ_JOIN_OVER = 1 << 30     # measured: 425 us/step with exact joins only, 440 with whole-buffer joins

    def build(self) -> Workload:
        c, b = self.m, self.b
        B, D, K = c.batch, c.d_in, c.classes
        nets = []
        for i, w in enumerate(c.widths):
            p = f'm{i}.'
            x = self.buf(p + 'x', B, D, 'f32', {'kind': 'seeded', 'seed': self._seed(p + 'x'), 'scale': 1.0, 'dist': 'normal'})
            labels = [(1103515245 * (j + 977 * i) + 12345) % (1 << 31) % K for j in range(B)]
            self.shapes[p + 'y'] = (B, 1)
            b.values(p + 'y', labels, B, 1, 'i32')
            self.buf(p + 'step', 1, 1, 'i32', {'kind': 'fill', 'value': 0})
            layers = []
            for l, (fi, fo) in enumerate(((D, w), (w, w), (w, K))):
                W = self._param(f'{p}W{l}', fo, fi, 1.0 / math.sqrt(fi))
                bb = self._param(f'{p}b{l}', 1, fo, 0.0)
                layers.append((W, bb, fi, fo))
            for nm, cols in (('z0', w), ('a0', w), ('z1', w), ('a1', w), ('logits', K), ('dlogits', K), ('da1', w), ('dz1', w),
                             ('da0', w), ('dz0', w)):
                self.buf(p + nm, B, cols)
            self.buf(p + 'rowloss', B), self.buf(p + 'lse', B), self.buf(p + 'loss', 2)
            nets.append((p, w, x, layers))
        self.dep = Deps(self.shapes)
        for s in range(c.steps):
            for net in nets:            # step s of every MLP, then step s + 1: the chains interleave in task order too
                self.step(*net)
        info = {'config': asdict(c), 'params': param_count(c), 'flops_per_step': step_flops(c), 'steps': c.steps}
        return Workload(b.spec('train'), b.init_override, info)

    def _seed(self, name):
        from . import seed_of
        return seed_of(self.m.seed, name)

    def _param(self, name, rows, cols, scale):
        if scale > 0:
            self.buf(name, rows, cols, 'f32', {'kind': 'seeded', 'seed': self._seed(name), 'scale': scale, 'dist': 'normal'})
        else:
            self.buf(name, rows, cols, 'f32', {'kind': 'fill', 'value': 0.0})
        for pre in ('d.', 'm.', 'v.'):
            self.buf(pre + name, rows, cols)
        self.params.append((name, 'd.' + name, 'm.' + name, 'v.' + name, None, scale > 0))
        return name

    def relu(self, z, a, cols):
        B = self.m.batch
        for r0, r1 in self.rows(B):
            self.task('act_fwd', [(z, (r0, r1))], [(a, (r0, r1))], x=z, out=a, kind=0, e0=r0 * cols, e1=r1 * cols)

    def relu_bwd(self, z, da, dz, cols):
        B = self.m.batch
        for r0, r1 in self.rows(B):
            self.task('act_bwd', [(z, (r0, r1)), (da, (r0, r1))], [(dz, (r0, r1))], x=z, dy=da, dx=dz, kind=0, e0=r0 * cols,
                      e1=r1 * cols, acc=0)

    def step(self, p, w, x, layers):
        c = self.m
        B, K = c.batch, c.classes
        (W0, b0, _, _), (W1, b1, _, _), (W2, b2, _, _) = layers
        self.task('counter_inc', [], [(p + 'step', ())], x=p + 'step', i0=0, i1=1, delta=1)
        # forward
        self.gemm(x, W0, p + 'z0', B, w, c.d_in, flags=2, bias=b0)
        self.relu(p + 'z0', p + 'a0', w)
        self.gemm(p + 'a0', W1, p + 'z1', B, w, w, flags=2, bias=b1)
        self.relu(p + 'z1', p + 'a1', w)
        self.gemm(p + 'a1', W2, p + 'logits', B, K, w, flags=2, bias=b2)
        for r0, r1 in self.rows(B):
            self.task('softmax_ce_fused', [(p + 'logits', (r0, r1)), (p + 'y', (r0, r1))],
                      [(p + 'rowloss', (r0, r1)), (p + 'lse', (r0, r1)), (p + 'dlogits', (r0, r1))],
                      logits=p + 'logits', tgt=p + 'y', rowloss=p + 'rowloss', lse=p + 'lse', dlogits=p + 'dlogits', r0=r0, r1=r1, V=K,
                      ignore=-1, N=B, scale=1.0)
        self.task('softmax_ce_reduce', [(p + 'rowloss', ()), (p + 'y', ())], [(p + 'loss', ())], rowloss=p + 'rowloss', tgt=p + 'y',
                  loss=p + 'loss', N=B, ignore=-1)
        # backward
        self.gemm(p + 'dlogits', p + 'a1', 'd.' + W2, K, w, B, flags=1)
        self.colsum(p + 'dlogits', 'd.' + b2, B, K)
        self.gemm(p + 'dlogits', W2, p + 'da1', B, w, K, flags=0)
        self.relu_bwd(p + 'z1', p + 'da1', p + 'dz1', w)
        self.gemm(p + 'dz1', p + 'a0', 'd.' + W1, w, w, B, flags=1)
        self.colsum(p + 'dz1', 'd.' + b1, B, w)
        self.gemm(p + 'dz1', W1, p + 'da0', B, w, w, flags=0)
        self.relu_bwd(p + 'z0', p + 'da0', p + 'dz0', w)
        self.gemm(p + 'dz0', x, 'd.' + W0, w, c.d_in, B, flags=1)
        self.colsum(p + 'dz0', 'd.' + b0, B, w)
        # AdamW (no clipping), this MLP's parameters only
        for (W, bb, _, _) in layers:
            for name, dec in ((W, True), (bb, False)):
                R, C = self.shapes[name]
                for e0, e1 in row_chunks(R, C, c.opt_chunk):
                    rows = (e0 // C, (e1 - 1) // C + 1)
                    self.task('adamw', [('d.' + name, rows), (p + 'step', ())], [(name, rows), ('m.' + name, rows), ('v.' + name, rows)],
                              p=name, g='d.' + name, m='m.' + name, v='v.' + name, gscale=None, step=p + 'step', e0=e0, e1=e1, lr=c.lr,
                              b1=c.b1, b2=c.b2, eps=c.eps, wd=c.wd if dec else 0.0)


def build(c: MLPConfig | None = None) -> Workload:
    return MLPBuilder(c or MLPConfig()).build()
