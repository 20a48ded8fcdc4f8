"""GPT training step(s) as a task graph: BASELINE configs 1 (tiny GPT, f32, 10 steps), 3 (GPT-162M, bf16 storage) and
4 (GPT-355M, f32). The reference's frontend emits untied / RoPE models only (frontend/mvmfe/nn.py:13-31); these
configurations (tied embeddings, learned positions) are built here from registry operators:

  embedding_fwd (wte + wpe) -> L x [layernorm -> q, k, v GEMMs -> causal attention -> projection (+ residual) ->
  layernorm -> fc1 (+ GELU, pre-activation kept) -> fc2 (+ residual)] -> layernorm -> tied head GEMM (wte^T) ->
  fused softmax cross-entropy -> the backward of all of it (dgelu fused into the fc1 input-gradient GEMM epilogue,
  layernorm backward accumulating into the residual gradient in place, embedding_bwd accumulating the tied head's
  wte gradient and the position-table gradient) -> global grad norm -> AdamW (fp32 master weights) -> bf16 copies.

Dependencies are data dependencies: every task declares the rectangles (rows x columns) of the buffers it reads and
writes, and a task follows exactly the earlier tasks whose writes it reads (read-after-write) or whose reads/writes
it overwrites (write-after-read / write-after-write). Layers and phases therefore overlap wherever the data allows
(a GEMM row block starts as soon as its input rows exist), with no barrier tasks.

bf16 mode ("bf16s"): activations and activation gradients are bf16 storage; GEMMs are matmul_mma_bf16 (128x256 bf16
MFMA tiles, fp32 accumulation) on bf16 copies of the fp32 master weights; weight gradients, LN statistics, losses and
optimizer state are fp32. f32 mode: everything fp32, GEMMs are matmul_tile (exact fp32 on this executor).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, asdict

from . import Builder, Workload, split

RB = 128   # row-block granularity of the dependency index
CHUNK = 49152    # elements per optimizer task (measured: 49152 balances the step's AdamW tail best of 32K-256K)


@dataclass
class GPTConfig:
    layers: int = 12
    d: int = 768
    heads: int = 12
    T: int = 1024
    vocab: int = 50304
    ffn: int = 3072
    batch: int = 4
    dtype: str = 'bf16'          # 'bf16' (bf16 storage, fp32 master weights) or 'f32'
    steps: int = 1               # training steps unrolled into one graph
    lr: float = 1e-3
    b1: float = 0.9
    b2: float = 0.95
    wd: float = 0.1
    eps: float = 1e-8
    clip: float = 1.0
    seed: int = 1234
    init_scale: float = 0.02
    tasks_target: int = 192      # task count target for row-parallel / flat phases (192 measured fastest of 96-512)
    opt_chunk: int = 0           # elements per optimizer task (0: CHUNK)

    @staticmethod
    def gpt162m(**kw):
        return GPTConfig(**kw)

    @staticmethod
    def gpt355m(**kw):
        base = dict(layers=24, d=1024, heads=16, ffn=4096, dtype='f32')
        base.update(kw)
        return GPTConfig(**base)

    @staticmethod
    def tiny(**kw):
        """2 layers, d 128, 4 heads, context 64, vocab 256, batch 8, f32, 10 steps."""
        # 64 row tasks and 8,192-element optimizer tasks: 659 us/step, against 711 with 32 / 49,152 (measured)
        base = dict(layers=2, d=128, heads=4, T=64, vocab=256, ffn=512, batch=8, dtype='f32', steps=10, tasks_target=64,
                    opt_chunk=8192)
        base.update(kw)
        return GPTConfig(**base)


def param_count(c: GPTConfig) -> int:
    d, f = c.d, c.ffn
    per = 4 * d * d + 4 * d + 2 * d * f + f + d + 4 * d
    return c.layers * per + c.vocab * d + c.T * d + 2 * d


def matmul_params(c: GPTConfig) -> int:
    return c.layers * (4 * c.d * c.d + 2 * c.d * c.ffn) + c.vocab * c.d


def step_flops(c: GPTConfig) -> dict:
    """GEMM and causal-attention FLOPs of one training step (forward + backward)."""
    N = c.batch * c.T
    gemm = 6 * matmul_params(c) * N
    hd = c.d // c.heads
    # causal: T*(T+1)/2 score entries per (b, h); fwd QK^T and PV: 2 GEMMs; bwd: 5 GEMM-sized products
    pairs = c.batch * c.heads * c.T * (c.T + 1) / 2
    attn_fwd = 2 * 2 * pairs * hd * c.layers
    attn_bwd = 5 * 2 * pairs * hd * c.layers
    return {'gemm': gemm, 'attn': attn_fwd + attn_bwd, 'total': gemm + attn_fwd + attn_bwd}


def row_chunks(R, C, chunk=None):
    """Flat [e0, e1) ranges of about `chunk` (default CHUNK) elements covering an R x C matrix, on whole rows: tasks of
    different chunks never share a row, so the dependency tracker keeps them independent."""
    return [(r0 * C, r1 * C) for r0, r1 in split(R, -(-(R * C) // (chunk or CHUNK)))]


class Deps:
    """Rectangle-based dependency tracker over buffers (rows bucketed by RB)."""

    def __init__(self, shapes):
        self.shapes = shapes            # name -> (rows, cols)
        self.acc = {}                   # name -> {bucket: [(r0, r1, c0, c1, task, is_write)]}
        self.writers = {}               # name -> every task that wrote it (for whole-buffer joins)
        self.gen = {}                   # name -> number of recorded writes

    def _rect(self, name, r0=0, r1=None, c0=0, c1=None):
        R, C = self.shapes[name]
        return (r0, R if r1 is None else r1, c0, C if c1 is None else c1)

    def deps(self, reads, writes):
        out = set()
        for kind, items in ((False, reads), (True, writes)):
            for name, rect in items:
                r0, r1, c0, c1 = rect
                bk = self.acc.get(name, {})
                for b in range(r0 // RB, (r1 - 1) // RB + 1):
                    for (a0, a1, d0, d1, t, w) in bk.get(b, ()):
                        if (w or kind) and a0 < r1 and r0 < a1 and d0 < c1 and c0 < d1:
                            out.add(t)
        return out

    def record(self, task, reads, writes):
        """Accesses are kept per row bucket, clipped to the bucket's rows. A write subtracts its rectangle from every
        older access it overlaps (up to four remainder pieces stay): later tasks touching the overlap are ordered after
        the writer, which is ordered after those accesses, so only the uncovered remainders still need edges of their
        own. Without the subtraction, reads that chunked writes only partly cover (a GEMM tile's weight columns against
        an optimizer's row chunks) would pile up over training steps, and every later write would depend on them all."""
        for name, _ in writes:
            self.writers.setdefault(name, []).append(task)
            self.gen[name] = self.gen.get(name, 0) + 1
        for kind, items in ((False, reads), (True, writes)):
            for name, rect in items:
                r0, r1, c0, c1 = rect
                bk = self.acc.setdefault(name, {})
                for b in range(r0 // RB, (r1 - 1) // RB + 1):
                    lst = bk.setdefault(b, [])
                    q0, q1 = max(r0, b * RB), min(r1, (b + 1) * RB)
                    if kind:
                        keep = []
                        for x in lst:
                            a0, a1, d0, d1 = x[:4]
                            if not (a0 < q1 and q0 < a1 and d0 < c1 and c0 < d1):
                                keep.append(x)
                                continue
                            t, w = x[4], x[5]
                            if a0 < q0:
                                keep.append((a0, q0, d0, d1, t, w))
                            if q1 < a1:
                                keep.append((q1, a1, d0, d1, t, w))
                            m0, m1 = max(a0, q0), min(a1, q1)
                            if d0 < c0:
                                keep.append((m0, m1, d0, c0, t, w))
                            if c1 < d1:
                                keep.append((m0, m1, c1, d1, t, w))
                        lst[:] = keep
                    lst.append((q0, q1, c0, c1, task, kind))


class GPTBuilder:
    def __init__(self, c: GPTConfig):
        self.c = c
        self.b = Builder(c.seed)
        self.shapes = {}
        self.dep = None
        self.bf = c.dtype == 'bf16'
        self.act = 'bf16' if self.bf else 'f32'
        if self.bf:
            self.READ_JOIN_OVER = 1 << 30
        self.params = []      # (master, grad, m, v, shadow or None, wd)
        self.joins = {}       # predecessor set -> join task
        self.bjoins = {}      # buffer -> (write generation, join task over all its writers)

    # ---- buffers
    def buf(self, name, rows, cols=1, dtype='f32', init=None):
        self.shapes[name] = (rows, cols)
        return self.b.buf(name, rows, cols, dtype, init)

    def normal(self, name, rows, cols=1):
        self.shapes[name] = (rows, cols)
        return self.b.normal(name, rows, cols, 'f32', scale=self.c.init_scale)

    def param(self, name, rows, cols=1, kind='matrix'):
        """fp32 master + grad + AdamW moments (+ bf16 shadow for GEMM weights in bf16 mode)."""
        if kind == 'matrix':
            self.normal(name, rows, cols)
        else:
            self.buf(name, rows, cols, 'f32', {'kind': 'fill', 'value': 1.0 if kind == 'gain' else 0.0})
        self.buf(f'd.{name}', rows, cols)
        self.buf(f'm.{name}', rows, cols)
        self.buf(f'v.{name}', rows, cols)
        shadow = None
        if self.bf and kind == 'matrix':   # starts as the master rounded to bf16; each AdamW task refreshes its rows
            self.shapes[f'{name}.bf'] = (rows, cols)
            shadow = self.b.normal(f'{name}.bf', rows, cols, 'bf16', scale=self.c.init_scale, seed_name=name)
        self.params.append((name, f'd.{name}', f'm.{name}', f'v.{name}', shadow, kind == 'matrix'))
        return name

    def w(self, name):
        """The buffer GEMMs read for a weight."""
        return f'{name}.bf' if self.bf else name

    # ---- tasks with data dependencies
    # A task with more predecessors than JOIN_OVER waits on a shared noop join of exactly those instead (edges stay
    # linear). A read depending on more writers than READ_JOIN_OVER waits on the whole buffer's completion join (a
    # barrier over every sequence). Measured on one MI355X: GPT-162M (bf16) 10.22-10.25 ms with joins over 24 and no
    # buffer joins, 10.42 with 48 / 16, 12.3-12.6 with joins over 8 or 16 (join tasks on the critical path);
    # GPT-355M (f32) 232.6 ms with buffer joins over 16, 266-280 without. The bf16 graphs take no buffer joins.
    JOIN_OVER = 24
    READ_JOIN_OVER = 16

    def buffer_join(self, name):
        g = self.dep.gen.get(name, 0)
        hit = self.bjoins.get(name)
        if hit and hit[0] == g:
            return hit[1]
        j = self.b.task('noop', after=sorted(set(self.dep.writers[name]), key=lambda t: int(t[1:])))
        self.bjoins[name] = (g, j)
        return j

    def task(self, op, reads, writes, extra_after=(), **args):
        R = [(n, self.dep._rect(n, *r)) for n, r in reads]
        W = [(n, self.dep._rect(n, *r)) for n, r in writes]
        deps = set(extra_after) | self.dep.deps([], W)
        for item in R:
            d = self.dep.deps([item], [])
            deps |= {self.buffer_join(item[0])} if len(d) > self.READ_JOIN_OVER else d
        deps = frozenset(deps)
        if len(deps) > self.JOIN_OVER:
            j = self.joins.get(deps)
            if j is None:
                j = self.joins[deps] = self.b.task('noop', after=sorted(deps, key=lambda t: int(t[1:])))
            deps = [j]
        t = self.b.task(op, after=sorted(deps, key=lambda t: int(t[1:])), **args)
        self.dep.record(t, R, W)
        return t

    # bf16 GEMMs with at least this many 256x256 output tiles use them (op 304). Off: with the 128x256 tile inlined
    # into the executor kernel, 128x256 tiles run the GPT-162M step in 8.93 ms against 9.08 with 256x256 tiles from 256.
    TILES_256 = 1 << 30
    TILES_ALONE = 128  # a GEMM running alone with fewer 128x256 tiles than this uses 128x128 tiles
    TILES_MMA = 16     # else at least this many 128x256 tiles: op 122; else 128x128 tiles (op 114), more of them
    F32_TILES_128 = 64   # f32 GEMMs with at least this many 128x128 output tiles use them (op 34), else 64x64 tiles
    F32_TILES_256 = 256  # f32 GEMMs with at least this many 256x128 output tiles use them (op 34, flag 64; GPT-355M 98.5 -> 97.9 ms)

    def gemm(self, A, B, out, M, N, K, flags=0, bias=None, res=None, pre=None, alpha=1.0, alone=False):
        """C = alpha * op(A) op(B) (+ epilogue), tiled; returns the task ids. `alone`: nothing else runs beside this
        GEMM (a forward projection after a layer's attention or MLP input), so its tiles should fill the chip by
        themselves: 128x128 tiles when 128x256 ones would leave most CUs idle."""
        bf, ta, tb = self.bf, flags & 1, flags & 2
        if bf and alone and -(-M // 128) * -(-N // 256) < self.TILES_ALONE:
            op, TM, TN, fl = 'matmul_tile_bf16', 128, 128, flags | 32
        elif bf and -(-M // 256) * -(-N // 256) >= self.TILES_256:
            op, TM, TN, fl = 'matmul_mma_bf16_256', 256, 256, flags
        elif bf and -(-M // 128) * -(-N // 256) >= self.TILES_MMA:
            op, TM, TN, fl = 'matmul_mma_bf16', 128, 256, flags
        elif bf:   # fewer than 256 tiles of 128x256: 128x128 tiles keep more of the chip busy
            op, TM, TN, fl = 'matmul_tile_bf16', 128, 128, flags | 32
        elif M >= 256 and N >= 128 and -(-M // 256) * -(-N // 128) >= self.F32_TILES_256:
            op, TM, TN, fl = 'matmul_tile', 256, 128, flags | 64
        elif M >= 128 and N >= 128 and -(-M // 128) * -(-N // 128) >= self.F32_TILES_128:
            op, TM, TN, fl = 'matmul_tile', 128, 128, flags | 32
        else:
            op, TM, TN, fl = 'matmul_tile', 64, 64, flags
        ts = []
        for m0 in range(0, M, TM):
            m1 = min(M, m0 + TM)
            for n0 in range(0, N, TN):
                n1 = min(N, n0 + TN)
                reads = [(A, (0, K, m0, m1) if ta else (m0, m1, 0, K)), (B, (n0, n1, 0, K) if tb else (0, K, n0, n1))]
                if bias:
                    reads.append((bias, (0, 1, n0, n1)))
                if res:
                    reads.append((res, (m0, m1, n0, n1)))
                writes = [(out, (m0, m1, n0, n1))]
                if pre is not None and fl & 512:
                    reads.append((pre, (m0, m1, n0, n1)))
                elif pre is not None:
                    writes.append((pre, (m0, m1, n0, n1)))
                if fl & 4:
                    reads.append((out, (m0, m1, n0, n1)))
                ts.append(self.task(op, reads, writes, a=A, b=B, out=out, bias=bias, res=res, pre=pre, m0=m0, n0=n0, M=M, N=N, K=K,
                                    flags=fl, alpha=alpha))
        return ts

    def gemm_delta(self, A, B, out, M, N, K, flags, o, delta, T, H):
        """The dO GEMM as op 308 tiles (128 x 256, plain epilogue): each also writes delta = rowsum(o * dO) for the four
        64-column heads it covers, in place of separate delta tasks. Returns False when the shapes do not allow it."""
        if not (self.bf and M % 128 == 0 and N % 256 == 0 and N == H * 64 and T % 128 == 0 and flags & ~3 == 0
                and -(-M // 256) * -(-N // 256) < self.TILES_256 and (M // 128) * (N // 256) >= self.TILES_MMA):
            return False
        ta, tb = flags & 1, flags & 2
        for m0 in range(0, M, 128):
            m1 = m0 + 128
            bi, t0 = m0 // T, m0 % T
            for n0 in range(0, N, 256):
                n1 = n0 + 256
                reads = [(A, (0, K, m0, m1) if ta else (m0, m1, 0, K)), (B, (n0, n1, 0, K) if tb else (0, K, n0, n1)), (o, (m0, m1, n0, n1))]
                writes = [(out, (m0, m1, n0, n1))] + [(delta, ((bi * H + h) * T + t0, (bi * H + h) * T + t0 + 128))
                                                       for h in range(n0 // 64, n1 // 64)]
                self.task('matmul_mma_bf16_delta', reads, writes, a=A, b=B, out=out, bias=None, res=None, pre=None, m0=m0, n0=n0, M=M, N=N,
                          K=K, flags=flags, alpha=1.0, o=o, delta=delta, T=T, H=H, hd=64)
        return True

    SPLITK_S, SPLITK_TM = 8, 256   # the head input gradient's K splits and tile rows
    CE_TASKS = 512       # cross-entropy tasks: rows of the logits split finer than tasks_target, so the rows of the last
                         # logits tiles to finish are spread over many workers (GPT-162M 8.935 -> 8.90 ms against 192)
    SPLITK_MIN = 16384   # K from which a GEMM with few output tiles is split along K (the tied head's input gradient)

    def gemm_splitk(self, A, B, out, M, N, K, flags, S, TM=128):
        """out = op(A) op(B) as S independent K ranges (split-K tiles, op 302; TM 256: 256x256 tiles) into an f32
        partial buffer of S row blocks, then an in-order sum of the blocks into `out` (op 303, row chunks). The K
        ranges are whole 32-deep slabs."""
        ta, tb = flags & 1, flags & 2
        part = f'{out}.kpart'
        if part not in self.shapes:
            self.buf(part, S * M, N)
        slabs = K // 32
        assert slabs * 32 == K, 'split-K needs K % 32 == 0'
        bounds = [32 * (slabs * s // S) for s in range(S + 1)]
        for s in range(S):
            k0, k1 = bounds[s], bounds[s + 1]
            for m0 in range(0, M, TM):
                m1 = min(M, m0 + TM)
                for n0 in range(0, N, 256):
                    n1 = min(N, n0 + 256)
                    reads = [(A, (k0, k1, m0, m1) if ta else (m0, m1, k0, k1)), (B, (n0, n1, k0, k1) if tb else (k0, k1, n0, n1))]
                    self.task('matmul_mma_bf16_kr', reads, [(part, (s * M + m0, s * M + m1, n0, n1))], a=A, b=B, out=part, bias=None,
                              res=None, pre=None, m0=m0, n0=n0, M=M, N=N, K=k1 - k0, flags=flags | (64 if TM == 256 else 0), alpha=1.0,
                              k0=k0, om0=s * M)
        for r0, r1 in self.rows(M):
            self.task('splitk_reduce', [(part, (s * M + r0, s * M + r1, 0, N)) for s in range(S)], [(out, (r0, r1, 0, N))],
                      part=part, out=out, M=M, N=N, S=S, r0=r0, r1=r1)

    def rows(self, n, target=None):
        return split(n, min(n, target or self.c.tasks_target))

    # ---- model
    def build(self) -> Workload:
        c, b = self.c, self.b
        N, d, H, T, V, F = c.batch * c.T, c.d, c.heads, c.T, c.vocab, c.ffn
        hd = d // H
        act = self.act
        # ---- parameters
        self.param('wte', V, d)
        self.param('wpe', T, d)
        for l in range(c.layers):
            for nm in ('wq', 'wk', 'wv', 'wo'):
                self.param(f'{nm}.{l}', d, d)
                self.param(f'b{nm[1]}.{l}', 1, d, 'bias')
            self.param(f'ln1g.{l}', 1, d, 'gain'), self.param(f'ln1b.{l}', 1, d, 'bias')
            self.param(f'ln2g.{l}', 1, d, 'gain'), self.param(f'ln2b.{l}', 1, d, 'bias')
            self.param(f'w1.{l}', F, d), self.param(f'b1.{l}', 1, F, 'bias')
            self.param(f'w2.{l}', d, F), self.param(f'b2.{l}', 1, d, 'bias')
        self.param('lnfg', 1, d, 'gain'), self.param('lnfb', 1, d, 'bias')
        # ---- data and activations
        ids = [(7919 * i + 13 * (i // T)) % V for i in range(N)]
        self.shapes['ids'] = (N, 1)
        b.values('ids', ids, N, 1, 'i32')
        self.shapes['tgt'] = (N, 1)
        b.values('tgt', [ids[(i + 1) % N] if (i + 1) % T else ids[i - T + 1] for i in range(N)], N, 1, 'i32')
        self.buf('step', 1, 1, 'i32', {'kind': 'fill', 'value': 0})
        for l in range(c.layers + 1):
            self.buf(f'x.{l}', N, d, act)                     # residual stream entering layer l (l = L: final)
        for l in range(c.layers):
            for nm in ('h1', 'q', 'k', 'v', 'o', 'xm', 'h2'):
                self.buf(f'{nm}.{l}', N, d, act)
            self.buf(f'u.{l}', N, F, act)                      # fc1 pre-activation
            self.buf(f'a.{l}', N, F, act)                      # gelu(u)
            for nm in ('mu1', 'rs1', 'mu2', 'rs2'):
                self.buf(f'{nm}.{l}', N)
            self.buf(f'lse.{l}', c.batch * H * T)
            self.buf(f'delta.{l}', c.batch * H * T)
        self.buf('hf', N, d, act), self.buf('muf', N), self.buf('rsf', N)
        self.buf('logits', N, V, act), self.buf('dlogits', N, V, act)
        self.buf('rowloss', N), self.buf('celse', N), self.buf('loss', 2)
        # gradient activations, one set per layer (no write-after-read chains between layers)
        for l in range(c.layers + 1):
            self.buf(f'dx.{l}', N, d, act)                     # gradient of the residual stream after layer l's LN1 bwd
            self.buf(f'dm.{l}', N, d, act)                     # gradient w.r.t. xm (after LN2 bwd)
            self.buf(f'dh.{l}', N, d, act)
        for l in range(c.layers):
            for nm in ('do', 'dq', 'dk', 'dv'):
                self.buf(f'{nm}.{l}', N, d, act)
            self.buf(f'du.{l}', N, F, act)
        if self.bf:
            self.buf('dx0f', N, d)                              # f32 copy for embedding_bwd
        self.dep = Deps(self.shapes)
        for s in range(c.steps):
            self.step(s)
        info = {'config': asdict(c), 'params': param_count(c), 'flops': step_flops(c)}
        return Workload(b.spec('train'), b.init_override, info)

    def step(self, s):
        c = self.c
        N, d, H, T, V, F = c.batch * c.T, c.d, c.heads, c.T, c.vocab, c.ffn
        hd = d // H
        L = c.layers
        scale = 1.0 / math.sqrt(hd)
        self.task('counter_inc', [], [('step', ())], x='step', i0=0, i1=1, delta=1)
        # ---- forward
        for r0, r1 in self.rows(N):
            self.task('embedding_fwd', [('ids', (r0, r1)), ('wte', ()), ('wpe', ())], [('x.0', (r0, r1))],
                      ids='ids', wte='wte', wpe='wpe', out='x.0', r0=r0, r1=r1, T=T, d=d)
        for l in range(L):
            x, h1 = f'x.{l}', f'h1.{l}'
            self.layernorm(x, f'ln1g.{l}', f'ln1b.{l}', h1, f'mu1.{l}', f'rs1.{l}')
            for nm in ('q', 'k', 'v'):
                self.gemm(h1, self.w(f'w{nm}.{l}'), f'{nm}.{l}', N, d, d, flags=2, bias=f'b{nm}.{l}')
            for bb in range(c.batch):
                for h in range(H):
                    for q0 in range(0, T, 128):
                        q1 = min(T, q0 + 128)
                        rd = [(f'q.{l}', (bb * T + q0, bb * T + q1, h * hd, (h + 1) * hd)),
                              (f'k.{l}', (bb * T, bb * T + q1, h * hd, (h + 1) * hd)), (f'v.{l}', (bb * T, bb * T + q1, h * hd, (h + 1) * hd))]
                        wr = [(f'o.{l}', (bb * T + q0, bb * T + q1, h * hd, (h + 1) * hd)),
                              (f'lse.{l}', ((bb * H + h) * T + q0, (bb * H + h) * T + q1))]
                        self.task('attn_fwd', rd, wr, q=f'q.{l}', k=f'k.{l}', v=f'v.{l}', o=f'o.{l}', lse=f'lse.{l}', b=bb, h=h, q0=q0,
                                  T=T, H=H, Hkv=H, hd=hd, scale=scale)
            self.gemm(f'o.{l}', self.w(f'wo.{l}'), f'xm.{l}', N, d, d, flags=2, bias=f'bo.{l}', res=x, alone=True)
            self.layernorm(f'xm.{l}', f'ln2g.{l}', f'ln2b.{l}', f'h2.{l}', f'mu2.{l}', f'rs2.{l}')
            self.gemm(f'h2.{l}', self.w(f'w1.{l}'), f'a.{l}', N, F, d, flags=2 | 8, bias=f'b1.{l}', pre=f'u.{l}')
            self.gemm(f'a.{l}', self.w(f'w2.{l}'), f'x.{l + 1}', N, d, F, flags=2, bias=f'b2.{l}', res=f'xm.{l}', alone=True)
        self.layernorm(f'x.{L}', 'lnfg', 'lnfb', 'hf', 'muf', 'rsf')
        self.gemm('hf', self.w('wte'), 'logits', N, V, d, flags=2)
        for r0, r1 in self.rows(N, self.CE_TASKS):
            self.task('softmax_ce_fused', [('logits', (r0, r1)), ('tgt', (r0, r1))],
                      [('rowloss', (r0, r1)), ('celse', (r0, r1)), ('dlogits', (r0, r1))],
                      logits='logits', tgt='tgt', rowloss='rowloss', lse='celse', dlogits='dlogits', r0=r0, r1=r1, V=V, ignore=-1, N=N,
                      scale=1.0)
        self.task('softmax_ce_reduce', [('rowloss', ()), ('tgt', ())], [('loss', ())], rowloss='rowloss', tgt='tgt', loss='loss', N=N,
                  ignore=-1)
        # ---- backward. Residual gradient buffers: dx.{L} (final LN), then per layer l: dm.l (w.r.t. xm) and dx.l (w.r.t. x.l);
        # each LN backward adds into a copy-free buffer: LN2 bwd writes dm.l = dx.{l+1} + LN'(dh) via acc on a buffer
        # first filled by the residual path (the GEMM below writes it with res=), LN1 bwd likewise into dx.l.
        if self.bf and V >= self.SPLITK_MIN and V % 32 == 0:                                 # d hf: K = V is long, M x d has few tiles
            self.gemm_splitk('dlogits', self.w('wte'), f'dh.{L}', N, d, V, flags=0, S=self.SPLITK_S, TM=self.SPLITK_TM)
        else:
            self.gemm('dlogits', self.w('wte'), f'dh.{L}', N, d, V, flags=0)
        self.gemm('dlogits', 'hf', 'd.wte', V, d, N, flags=1)                              # tied head: wte grad (overwrite)
        self.layernorm_bwd(f'x.{L}', f'dh.{L}', 'lnfg', 'muf', 'rsf', f'dx.{L}', 'd.lnfg', 'd.lnfb', acc=0)
        for l in reversed(range(L)):
            dxo, dm, dx = f'dx.{l + 1}', f'dm.{l}', f'dx.{l}'
            # fc2: x_{l+1} = a @ w2^T + b2 + xm
            self.gemm(dxo, self.w(f'w2.{l}'), f'du.{l}', N, F, d, flags=512, pre=f'u.{l}')   # du = (dx @ w2) * gelu'(u)
            self.gemm(dxo, f'a.{l}', f'd.w2.{l}', d, F, N, flags=1)
            self.colsum(dxo, f'd.b2.{l}', N, d)
            # fc1: a = gelu(h2 @ w1^T + b1); dh2 lands in dm (then LN2 backward turns it into d xm, in place below)
            self.gemm(f'du.{l}', self.w(f'w1.{l}'), f'dh.{l}', N, d, F, flags=0)
            self.gemm(f'du.{l}', f'h2.{l}', f'd.w1.{l}', F, d, N, flags=1)
            self.colsum(f'du.{l}', f'd.b1.{l}', N, F)
            self.layernorm_bwd(f'xm.{l}', f'dh.{l}', f'ln2g.{l}', f'mu2.{l}', f'rs2.{l}', dm, f'd.ln2g.{l}', f'd.ln2b.{l}', acc=1,
                               res=dxo)                                                     # + the residual path
            # projection: xm = o @ wo^T + bo + x
            fused_delta = self.gemm_delta(dm, self.w(f'wo.{l}'), f'do.{l}', N, d, d, 0, f'o.{l}', f'delta.{l}', T, H)
            if not fused_delta:
                self.gemm(dm, self.w(f'wo.{l}'), f'do.{l}', N, d, d, flags=0)
            self.gemm(dm, f'o.{l}', f'd.wo.{l}', d, d, N, flags=1)
            self.colsum(dm, f'd.bo.{l}', N, d)
            self.attention_bwd(l, delta_done=fused_delta)
            # q, k, v: dh1 = dq wq + dk wk + dv wv (per tile: overwrite, then accumulate twice); LN1 input grad into dx.l
            dh1 = f'dh.{l}'
            self.gemm(f'dq.{l}', self.w(f'wq.{l}'), dh1, N, d, d, flags=0)
            self.gemm(f'dk.{l}', self.w(f'wk.{l}'), dh1, N, d, d, flags=4)
            self.gemm(f'dv.{l}', self.w(f'wv.{l}'), dh1, N, d, d, flags=4)
            for nm in ('q', 'k', 'v'):
                self.gemm(f'd{nm}.{l}', f'h1.{l}', f'd.w{nm}.{l}', d, d, N, flags=1)
                self.colsum(f'd{nm}.{l}', f'd.b{nm}.{l}', N, d)
            self.layernorm_bwd(f'x.{l}', dh1, f'ln1g.{l}', f'mu1.{l}', f'rs1.{l}', dx, f'd.ln1g.{l}', f'd.ln1b.{l}', acc=1, res=dm)
        dx0 = 'dx.0'
        if self.bf:                                  # embedding_bwd takes an f32 gradient
            for r0, r1 in self.rows(N):
                self.task('round_bf16', [('dx.0', (r0, r1))], [('dx0f', (r0, r1))], x='dx.0', out='dx0f', e0=r0 * d, e1=r1 * d)
            dx0 = 'dx0f'
        for v0, v1 in self.rows(V, c.tasks_target):
            self.task('embedding_bwd', [('ids', ()), (dx0, ())], [('d.wte', (v0, v1))], ids='ids', dout=dx0, dtab='d.wte', N=N, mod=0,
                      v0=v0, v1=v1, d=d, acc=1)
        for v0, v1 in self.rows(T, c.tasks_target):
            self.task('embedding_bwd', [(dx0, ())], [('d.wpe', (v0, v1))], ids=None, dout=dx0, dtab='d.wpe', N=N, mod=T, v0=v0, v1=v1,
                      d=d, acc=0)
        self.optimizer()

    def layernorm(self, x, g, bta, out, mu, rs):
        c = self.c
        N, d = c.batch * c.T, c.d
        for r0, r1 in self.rows(N):
            self.task('layernorm_fwd', [(x, (r0, r1)), (g, ()), (bta, ())], [(out, (r0, r1)), (mu, (r0, r1)), (rs, (r0, r1))],
                      x=x, gamma=g, beta=bta, out=out, mean=mu, rstd=rs, r0=r0, r1=r1, d=d, eps=1e-5)

    def layernorm_bwd(self, x, dy, g, mu, rs, dx, dg, db, acc, res=None):
        """res: dx = res + the input gradient (op 309, the residual path) instead of accumulating into dx."""
        c = self.c
        N, d = c.batch * c.T, c.d
        for c0, c1 in split(d, max(1, d // 64)):
            self.task('norm_bwd_params', [(x, (0, N, c0, c1)), (dy, (0, N, c0, c1)), (mu, ()), (rs, ())],
                      [(dg, (0, 1, c0, c1)), (db, (0, 1, c0, c1))], x=x, dy=dy, mean=mu, rstd=rs, dgamma=dg, dbeta=db, R=N, d=d, c0=c0,
                      c1=c1, acc=0)
        for r0, r1 in self.rows(N):
            reads = [(x, (r0, r1)), (dy, (r0, r1)), (g, ()), (mu, (r0, r1)), (rs, (r0, r1))]
            if res is not None:
                reads.append((res, (r0, r1)))
                self.task('layernorm_bwd_dx_res', reads, [(dx, (r0, r1))], x=x, dy=dy, gamma=g, mean=mu, rstd=rs, dx=dx, res=res, r0=r0,
                          r1=r1, d=d)
                continue
            if acc:
                reads.append((dx, (r0, r1)))
            self.task('layernorm_bwd_dx', reads, [(dx, (r0, r1))], x=x, dy=dy, gamma=g, mean=mu, rstd=rs, dx=dx, r0=r0, r1=r1, d=d, acc=acc)

    def colsum(self, x, out, R, C):
        for c0, c1 in split(C, max(1, C // 64)):
            self.task('colsum', [(x, (0, R, c0, c1))], [(out, (0, 1, c0, c1))], x=x, out=out, R=R, c0=c0, c1=c1, acc=0)

    def attention_bwd(self, l, delta_done=False):
        c = self.c
        N, d, H, T = c.batch * c.T, c.d, c.heads, c.T
        hd = d // H
        scale = 1.0 / math.sqrt(hd)
        o, q, k, v, lse, delta = f'o.{l}', f'q.{l}', f'k.{l}', f'v.{l}', f'lse.{l}', f'delta.{l}'
        for r0, r1 in ([] if delta_done else self.rows(N)):
            # delta is [B*H*T] at (b*H + h)*T + t: rows [r0, r1) write one range per (batch, head), so delta tasks of
            # different row blocks stay independent
            dr = []
            for bi in range(r0 // T, (r1 - 1) // T + 1):
                t0, t1 = max(r0, bi * T) - bi * T, min(r1, (bi + 1) * T) - bi * T
                dr += [(delta, ((bi * H + h) * T + t0, (bi * H + h) * T + t1)) for h in range(H)]
            self.task('attn_bwd_delta', [(o, (r0, r1)), (f'do.{l}', (r0, r1))], dr, o=o, do=f'do.{l}', delta=delta, r0=r0, r1=r1, T=T, H=H, hd=hd)
        for bb in range(c.batch):
            for h in range(H):
                cs = (h * hd, (h + 1) * hd)
                lr = ((bb * H + h) * T, (bb * H + h + 1) * T)
                for q0 in range(0, T, 128):
                    q1 = min(T, q0 + 128)
                    rd = [(q, (bb * T + q0, bb * T + q1, *cs)), (k, (bb * T, bb * T + q1, *cs)), (v, (bb * T, bb * T + q1, *cs)),
                          (f'do.{l}', (bb * T + q0, bb * T + q1, *cs)), (lse, lr), (delta, lr)]
                    self.task('attn_bwd_dq', rd, [(f'dq.{l}', (bb * T + q0, bb * T + q1, *cs))], q=q, k=k, v=v, do=f'do.{l}', lse=lse, delta=delta,
                              dq=f'dq.{l}', b=bb, h=h, q0=q0, T=T, H=H, Hkv=H, hd=hd, scale=scale)
                    rd = [(q, (bb * T + q0, bb * T + T, *cs)), (k, (bb * T + q0, bb * T + q1, *cs)), (v, (bb * T + q0, bb * T + q1, *cs)),
                          (f'do.{l}', (bb * T + q0, bb * T + T, *cs)), (lse, lr), (delta, lr)]
                    self.task('attn_bwd_dkv', rd, [(f'dk.{l}', (bb * T + q0, bb * T + q1, *cs)), (f'dv.{l}', (bb * T + q0, bb * T + q1, *cs))],
                              q=q, k=k, v=v, do=f'do.{l}', lse=lse, delta=delta, dk=f'dk.{l}', dv=f'dv.{l}', b=bb, kvh=h, k0=q0, T=T, H=H, hd=hd,
                              scale=scale)

    def optimizer(self):
        """Global grad norm (clip) -> AdamW on every parameter chunk (fp32 master weights)."""
        c = self.c
        chunks = []
        for (p, g, m, v, sh, dec) in self.params:
            R, C = self.shapes[p]
            n = R * C
            for e0, e1 in row_chunks(R, C, self.c.opt_chunk):
                chunks.append((p, g, m, v, sh, dec, e0, e1, C))
        if 'gn' not in self.shapes:
            self.buf('gn', len(chunks)), self.buf('gscale', 2)
        for i, (p, g, m, v, sh, dec, e0, e1, C) in enumerate(chunks):
            self.task('gradnorm_partial', [(g, (e0 // C, (e1 - 1) // C + 1))], [('gn', (i, i + 1))], g=g, partial='gn', slot=i, e0=e0, e1=e1)
        self.task('gradnorm_finish', [('gn', ())], [('gscale', ())], partial='gn', nslots=len(chunks), out='gscale', max_norm=c.clip)
        for (p, g, m, v, sh, dec, e0, e1, C) in chunks:
            rows = (e0 // C, (e1 - 1) // C + 1)
            kw = dict(p=p, g=g, m=m, v=v, gscale='gscale', step='step', e0=e0, e1=e1, lr=c.lr, b1=c.b1, b2=c.b2, eps=c.eps,
                      wd=c.wd if dec else 0.0)
            if sh:   # the bf16 GEMM copy of the new weight is written by the same pass
                self.task('adamw_bf16', [(g, rows), ('gscale', ()), ('step', ())], [(p, rows), (m, rows), (v, rows), (sh, rows)], sh=sh, **kw)
            else:
                self.task('adamw', [(g, rows), ('gscale', ()), ('step', ())], [(p, rows), (m, rows), (v, rows)], **kw)


def build(c: GPTConfig) -> Workload:
    return GPTBuilder(c).build()
