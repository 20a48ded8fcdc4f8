"""Small workloads, one or a few tasks each, that together exercise every operator this executor implements.

Each case is a workload JSON dict. `make_golden.py` compiles every case with the reference compiler and runs it on the
reference CPU VM to record the fixtures; the tests recompile the same dicts with kvm_amd.compiler and rerun them on the
oracle and on the GPU. Inputs are `seeded` (f32) or explicit `values` (i32, bf16) so the JSON stays small.
"""
from __future__ import annotations

import math
import random


def _bf16(x):
    import struct
    u = struct.unpack('<I', struct.pack('<f', x))[0]
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return struct.unpack('<f', struct.pack('<I', u))[0]


class W:
    """Workload builder."""

    def __init__(self, seed=1):
        self.bufs, self.tasks, self.vars = [], [], []
        self.seed = seed
        self.rng = random.Random(seed)

    def buf(self, name, rows, cols=1, dtype='f32', init=None, scale=1.0, dist='normal'):
        if init is None:
            if dtype == 'f32':
                self.seed += 1
                init = {'kind': 'seeded', 'seed': self.seed * 7919, 'scale': scale, 'dist': dist}
            elif dtype == 'bf16':
                init = {'kind': 'values', 'values': [_bf16(self.rng.gauss(0, scale)) for _ in range(rows * cols)]}
            else:
                init = {'kind': 'fill', 'value': 0}
        self.bufs.append({'name': name, 'rows': rows, 'cols': cols, 'dtype': dtype, 'init': init})
        return name

    def pos(self, name, n, scale):
        """n positive f32 values (second moments)."""
        return self.buf(name, n, 1, 'f32', {'kind': 'values', 'values': [scale * self.rng.random() + 1e-12 for _ in range(n)]})

    def zeros(self, name, rows, cols=1, dtype='f32'):
        return self.buf(name, rows, cols, dtype, {'kind': 'fill', 'value': 0})

    def ints(self, name, values, rows=None, cols=1):
        rows = rows or len(values) // cols
        return self.buf(name, rows, cols, 'i32', {'kind': 'values', 'values': list(values)})

    def task(self, op, after=(), **args):
        tid = f't{len(self.tasks)}'
        t = {'id': tid, 'op': op, 'args': args}
        if after:
            t['after'] = list(after)
        self.tasks.append(t)
        return tid

    def spec(self, name='g'):
        s = {'buffers': self.bufs, 'graphs': [{'name': name, 'tasks': self.tasks}]}
        if self.vars:
            s['variables'] = self.vars
        return s


def core():
    w = W(10)
    a, b = w.buf('a', 4, 8), w.buf('b', 4, 8)
    out, cp = w.zeros('out', 4, 8), w.zeros('cp', 4, 8)
    w.task('add', a=a, b=b, out=out, n=32)
    w.task('copy', src=a, dst=cp, n=30)
    sc = w.zeros('sc', 4, 8)
    w.task('scale', x=b, out=sc, alpha=0.37, n=32)
    r = w.zeros('r', 4, 8)
    w.task('relu', x=a, out=r, n=32)
    ww, g = w.buf('w', 4, 8), w.buf('g', 4, 8)
    w.task('sgd', w=ww, g=g, lr=0.05, n=32)
    x, s = w.buf('x', 16), w.buf('s', 1)
    pred, tgt = w.zeros('pred', 16), w.buf('tgt', 16)
    t0 = w.task('predict', x=x, w=s, out=pred, n=16)
    loss, grad = w.zeros('loss', 1), w.zeros('grad', 1)
    w.task('mse_grad', after=[t0], pred=pred, target=tgt, x=x, loss=loss, grad=grad, n=16)
    A, B, C = w.buf('A', 5, 7), w.buf('B', 7, 6), w.zeros('C', 5, 6)
    w.task('matmul', a=A, b=B, out=C, m=5, n=6, k=7)
    f = w.zeros('f', 3, 3)
    w.task('fill', x=f, value=2.5, n=7)
    w.task('noop')
    w.task('spin', us=0)
    return w.spec()


def versions():
    """Publishes, exact and at_least reads, gates (a task with two waiting reads) and write-after-read edges."""
    w = W(20)
    w.vars = ['wt', 'aux']
    p, out1, out2, out3 = w.buf('p', 8), w.zeros('o1', 8), w.zeros('o2', 8), w.zeros('o3', 8)
    g = w.buf('g', 8)
    ts = w.tasks

    def t(tid, op, after=(), publishes=None, reads=(), **args):
        d = {'id': tid, 'op': op, 'args': args}
        if after:
            d['after'] = list(after)
        if publishes:
            d['publishes'] = publishes
        if reads:
            d['reads'] = [{'var': v, 'policy': pol, 'version': n} for v, pol, n in reads]
        ts.append(d)
    t('upd1', 'sgd', publishes='wt', w=p, g=g, lr=0.1, n=8)
    t('rd1', 'scale', reads=[('wt', 'exact', 1)], x=p, out=out1, alpha=2.0, n=8)
    t('upd2', 'sgd', after=['upd1'], publishes='wt', w=p, g=g, lr=0.1, n=8)
    t('aux1', 'copy', publishes='aux', src=g, dst=out3, n=8)
    t('rd2', 'add', reads=[('wt', 'at_least', 2), ('aux', 'exact', 1)], a=p, b=out3, out=out2, n=8)
    t('rd0', 'relu', reads=[('wt', 'exact', 0)], x=g, out=w.zeros('o4', 8), n=8)
    return w.spec('v')


def gpt_ops():
    w = W(30)
    T, H, Hkv, hd, B = 40, 4, 2, 16, 2
    R, D, Dkv = B * T, H * hd, Hkv * hd
    V = 50
    ids = w.ints('ids', [w.rng.randrange(V) for _ in range(R)])
    wte, wpe = w.buf('wte', V, D, scale=0.5), w.buf('wpe', T, D, scale=0.5)
    emb = w.zeros('emb', R, D)
    te = w.task('embedding_fwd', ids=ids, wte=wte, wpe=wpe, out=emb, r0=3, r1=R, T=T, d=D)
    dtab, dpos = w.zeros('dtab', V, D), w.zeros('dpos', T, D)
    w.task('embedding_bwd', after=[te], ids=ids, dout=emb, dtab=dtab, N=R, mod=0, v0=0, v1=V, d=D, acc=0)
    w.task('embedding_bwd', after=[te], ids=None, dout=emb, dtab=dpos, N=R, mod=T, v0=1, v1=T, d=D, acc=0)
    # matmul_tile variants
    M, N, K = 70, 80, 24
    A, At, Bm, Bt = w.buf('A', M, K), w.buf('At', K, M), w.buf('Bm', K, N), w.buf('Bt', N, K)
    bias, res = w.buf('bias', 1, N), w.buf('res', M, N)
    for fl, a_, b_ in ((0, A, Bm), (1, At, Bm), (2, A, Bt), (3, At, Bt), (16, A, Bm), (32, A, Bm), (64, A, Bm)):
        o = w.zeros(f'mm{fl}', M, N)
        for m0 in range(0, M, {32: 128, 64: 256}.get(fl, 64)):
            for n0 in range(0, N, 128 if fl in (32, 64) else 64):
                w.task('matmul_tile', a=a_, b=b_, out=o, bias=None, res=None, pre=None, m0=m0, n0=n0, M=M, N=N, K=K,
                       flags=fl, alpha=0.75)
    o8, pre = w.buf('mm8', M, N), w.zeros('pre8', M, N)
    for m0 in (0, 64):
        for n0 in (0, 64):
            w.task('matmul_tile', a=A, b=Bm, out=o8, bias=bias, res=res, pre=pre, m0=m0, n0=n0, M=M, N=N, K=K, flags=4 | 8, alpha=1.0)
    o512 = w.zeros('mm512', M, N)
    for m0 in (0, 64):
        for n0 in (0, 64):
            w.task('matmul_tile', a=A, b=Bm, out=o512, bias=None, res=None, pre=res, m0=m0, n0=n0, M=M, N=N, K=K, flags=512, alpha=1.0)
    # norms
    x, dy = w.buf('x', 12, 20), w.buf('dy', 12, 20)
    gam, bet = w.buf('gam', 20, scale=0.3), w.buf('bet', 20)
    ln, mean, rstd = w.zeros('ln', 12, 20), w.zeros('mean', 12), w.zeros('rstd', 12)
    t1 = w.task('layernorm_fwd', x=x, gamma=gam, beta=bet, out=ln, mean=mean, rstd=rstd, r0=0, r1=12, d=20, eps=1e-5)
    rms, rrstd = w.zeros('rms', 12, 20), w.zeros('rrstd', 12)
    t2 = w.task('rmsnorm_fwd', x=x, gamma=gam, out=rms, rstd=rrstd, r0=1, r1=12, d=20, eps=1e-6)
    dx1, dx2 = w.buf('dx1', 12, 20), w.zeros('dx2', 12, 20)
    w.task('layernorm_bwd_dx', after=[t1], x=x, dy=dy, gamma=gam, mean=mean, rstd=rstd, dx=dx1, r0=0, r1=12, d=20, acc=1)
    w.task('rmsnorm_bwd_dx', after=[t2], x=x, dy=dy, gamma=gam, rstd=rrstd, dx=dx2, r0=0, r1=12, d=20, acc=0)
    dg, db, dg2 = w.zeros('dg', 20), w.buf('db', 20), w.zeros('dg2', 20)
    w.task('norm_bwd_params', after=[t1], x=x, dy=dy, mean=mean, rstd=rstd, dgamma=dg, dbeta=db, R=12, d=20, c0=0, c1=20, acc=0)
    w.task('norm_bwd_params', after=[t2], x=x, dy=dy, mean=None, rstd=rrstd, dgamma=dg2, dbeta=None, R=12, d=20, c0=3, c1=17, acc=0)
    ge, gb = w.zeros('ge', 12, 20), w.buf('gb', 12, 20)
    w.task('gelu_fwd', x=x, out=ge, e0=0, e1=240)
    w.task('gelu_bwd', x=x, dy=dy, dx=gb, e0=5, e1=230, acc=1)
    ra = w.zeros('ra', 12, 20)
    w.task('residual_add', a=x, b=dy, out=ra, e0=0, e1=240)
    sw = w.buf('sw', 12, 20)
    w.task('sgd_range', w=sw, g=dy, lr=0.01, e0=10, e1=200)
    cs = w.buf('cs', 20)
    w.task('colsum', x=x, out=cs, R=12, c0=2, c1=20, acc=1)
    rt = w.zeros('rt', 12, 20)
    w.task('round_tf32', x=x, out=rt, e0=0, e1=240)
    # rope
    pos = w.ints('pos', [7])
    qr, qb = w.zeros('qr', R, D), w.zeros('qb', R, D)
    q = w.buf('q', R, D)
    t3 = w.task('rope_fwd', x=q, out=qr, pos=pos, r0=0, r1=R, T=T, H=H, hd=hd, theta=10000.0)
    w.task('rope_bwd', after=[t3], x=qr, out=qb, pos=None, r0=0, r1=R, T=T, H=H, hd=hd, theta=10000.0)
    # attention fwd/bwd, GQA
    k, v, do = w.buf('k', R, Dkv), w.buf('v', R, Dkv), w.buf('do', R, D)
    o, lse = w.zeros('o', R, D), w.zeros('lse', B * H * T)
    fw = [w.task('attn_fwd', q=q, k=k, v=v, o=o, lse=lse, b=b, h=h, q0=0, T=T, H=H, Hkv=Hkv, hd=hd, scale=0.25)
          for b in range(B) for h in range(H)]
    delta = w.zeros('delta', B * H * T)
    td = w.task('attn_bwd_delta', after=fw, o=o, do=do, delta=delta, r0=0, r1=R, T=T, H=H, hd=hd)
    dq, dk, dv = w.zeros('dq', R, D), w.zeros('dk', R, Dkv), w.zeros('dv', R, Dkv)
    for b in range(B):
        for h in range(H):
            w.task('attn_bwd_dq', after=[td], q=q, k=k, v=v, do=do, lse=lse, delta=delta, dq=dq, b=b, h=h, q0=0, T=T, H=H,
                   Hkv=Hkv, hd=hd, scale=0.25)
        for kh in range(Hkv):
            w.task('attn_bwd_dkv', after=[td], q=q, k=k, v=v, do=do, lse=lse, delta=delta, dk=dk, dv=dv, b=b, kvh=kh, k0=0,
                   T=T, H=H, hd=hd, scale=0.25)
    # KV cache + decode
    Tmax = 24
    kc, vc = w.buf('kc', B * Hkv * Tmax, hd), w.buf('vc', B * Hkv * Tmax, hd)
    lens = w.ints('lens', [9, 17])
    kn, vn = w.buf('kn', B, Dkv), w.buf('vn', B, Dkv)
    qd, od = w.buf('qd', B, D), w.zeros('od', B, D)
    ta = w.task('kv_append', knew=kn, vnew=vn, kc=kc, vc=vc, lens=lens, b0=0, b1=B, n_new=1, Hkv=Hkv, hd=hd, Tmax=Tmax)
    for b in range(B):
        for h in range(H):
            w.task('attn_decode', after=[ta], q=qd, kc=kc, vc=vc, lens=lens, o=od, b=b, h=h, H=H, Hkv=Hkv, hd=hd, Tmax=Tmax, scale=0.25)
    # cross entropy
    Vc = 37
    lg = w.buf('lg', 10, Vc, scale=2.0)
    tg = w.ints('tg', [w.rng.randrange(Vc) for _ in range(9)] + [-1])
    rl, ls, loss = w.zeros('rl', 10), w.zeros('ls', 10), w.zeros('loss', 2)
    tf = w.task('softmax_ce_fwd', logits=lg, tgt=tg, rowloss=rl, lse=ls, r0=0, r1=10, V=Vc, ignore=-1)
    tr = w.task('softmax_ce_reduce', after=[tf], rowloss=rl, tgt=tg, loss=loss, N=10, ignore=-1)
    dl = w.zeros('dl', 10, Vc)
    w.task('softmax_ce_bwd', after=[tr], logits=lg, tgt=tg, lse=ls, loss=loss, dlogits=dl, r0=0, r1=10, V=Vc, ignore=-1, scale=1.0)
    tg2 = w.ints('tg2', [w.rng.randrange(Vc) for _ in range(10)])
    rl2, ls2, dl2 = w.zeros('rl2', 10), w.zeros('ls2', 10), w.zeros('dl2', 10, Vc)
    w.task('softmax_ce_fused', logits=lg, tgt=tg2, rowloss=rl2, lse=ls2, dlogits=dl2, r0=2, r1=10, V=Vc, ignore=-1, N=10, scale=0.5)
    # optimizer
    n = 300
    p, g = w.buf('p', n), w.buf('g', n, scale=0.1)
    m, vv = w.buf('m', n, scale=0.01), w.pos('vv', n, 1e-4)
    step = w.ints('step', [3])
    part, gsc = w.zeros('part', 3), w.zeros('gsc', 2)
    gp = [w.task('gradnorm_partial', g=g, partial=part, slot=s, e0=s * 100, e1=(s + 1) * 100) for s in range(3)]
    gf = w.task('gradnorm_finish', after=gp, partial=part, nslots=3, out=gsc, max_norm=0.5)
    w.task('adamw', after=[gf], p=p, g=g, m=m, v=vv, gscale=gsc, step=step, e0=0, e1=n, lr=1e-3, b1=0.9, b2=0.95, eps=1e-8, wd=0.1)
    # sampling / plumbing
    sl = w.buf('sl', 6, 33, scale=2.0)
    am, smp = w.buf('am', 6, 1, 'i32'), w.buf('smp', 6, 1, 'i32')
    ctr = w.ints('ctr', [5])
    w.task('argmax', logits=sl, out=am, r0=0, r1=6, V=33)
    w.task('sample', logits=sl, out=smp, ctr=ctr, r0=0, r1=3, V=33, temp=0.8, topk=5, seed=1234)
    w.task('sample', logits=sl, out=smp, ctr=None, r0=3, r1=6, V=33, temp=1.3, topk=0, seed=99)
    zb = w.buf('zb', 20)
    w.task('zero_buf', x=zb, e0=3, e1=17)
    cnt = w.ints('cnt', [1, 2, 3, 4])
    w.task('counter_inc', x=cnt, i0=1, i1=3, delta=5)
    src = w.ints('src', list(range(100)))
    sel = w.buf('sel', 10, 1, 'i32')
    stp = w.ints('stp', [2])
    w.task('select_window', src=src, step=stp, dst=sel, i0=0, i1=10, stride=30, off=4)
    gi = w.ints('gi', [3, 0, 7, 7, 1])
    gr = w.zeros('gr', 5, 20)
    w.task('gather_rows', src=x, idx=gi, dst=gr, r0=0, r1=5, d=20)
    return w.spec()


def extra_ops():
    w = W(40)
    x, dy = w.buf('x', 10, 16), w.buf('dy', 10, 16)
    for kind in range(4):
        w.task('act_fwd', x=x, out=w.zeros(f'af{kind}', 10, 16), kind=kind, e0=0, e1=160)
        w.task('act_bwd', x=x, dy=dy, dx=w.buf(f'ab{kind}', 10, 16), kind=kind, e0=2, e1=150, acc=kind & 1)
    up = w.buf('up', 10, 16)
    w.task('silu_mul_fwd', gate=x, up=up, out=w.zeros('sm', 10, 16), e0=0, e1=160)
    w.task('silu_mul_bwd', gate=x, up=up, dy=dy, dgate=w.zeros('sdg', 10, 16), dup=w.buf('sdu', 10, 16), e0=0, e1=160, acc=0)
    sp = w.zeros('sp', 10, 16)
    t = w.task('softmax_rows_fwd', x=x, out=sp, r0=0, r1=10, d=16, scale=0.7)
    w.task('softmax_rows_bwd', after=[t], p=sp, dp=dy, dx=w.buf('sdx', 10, 16), r0=1, r1=10, d=16, scale=0.7, acc=1)
    idx = w.ints('idx', [2, -1, 5, 9, 2, 0, 11])
    scl = w.buf('scl', 7)
    w.task('gather_rows_scaled', src=x, idx=idx, scale=scl, dst=w.zeros('grs', 6, 16), r0=0, r1=6, d=16, acc=0, idx0=1)
    w.task('scatter_add_rows', src=w.buf('sa_src', 6, 16), idx=idx, scale=None, dst=w.buf('sa', 10, 16), N=6, v0=0, v1=10, d=16,
           acc=1, idx0=1)
    w.task('row_dot', a=x, b=w.buf('rdb', 6, 16), idx=idx, out=w.zeros('rd', 7), r0=0, r1=6, d=16, acc=0, idx0=1)
    # bf16 storage conversions
    xb = w.zeros('xb', 10, 16, 'bf16')
    t1 = w.task('round_bf16', x=x, out=xb, e0=0, e1=160)
    w.task('round_bf16', after=[t1], x=xb, out=w.zeros('xw', 10, 16), e0=0, e1=160)
    w.task('round_bf16', x=x, out=w.zeros('xe', 10, 16), e0=4, e1=160)
    # bf16 GEMM tiles, f32 and bf16 storage operands/outputs
    M, N, K = 72, 136, 40
    A, Bt = w.buf('A', M, K), w.buf('Bt', N, K)
    Ab, Bb = w.buf('Ab', M, K, 'bf16'), w.buf('Bb', K, N, 'bf16')
    bias = w.buf('bias', 1, N)
    for m0 in (0, 64):
        for n0 in (0, 64, 128):
            w.task('matmul_tile_bf16', a=A, b=Bt, out=w.zeros(f'mtb_{m0}_{n0}', M, N), bias=bias, res=None, pre=None, m0=m0, n0=n0,
                   M=M, N=N, K=K, flags=2 | 8, alpha=1.0)
    ob = w.zeros('ob', M, N, 'bf16')
    prb = w.zeros('prb', M, N, 'bf16')
    for m0 in (0, 64):
        for n0 in (0, 64, 128):
            w.task('matmul_tile_bf16', a=Ab, b=Bb, out=ob, bias=bias, res=None, pre=prb, m0=m0, n0=n0, M=M, N=N, K=K, flags=8, alpha=0.5)
    om = w.zeros('om', M, N, 'bf16')
    w.task('matmul_mma_bf16', a=Ab, b=Bb, out=om, bias=None, res=None, pre=None, m0=0, n0=0, M=M, N=N, K=K, flags=0, alpha=1.0)
    # decode GEMV
    Kg, Ng = 64, 40
    wg = w.buf('wg', Ng, Kg, 'bf16', scale=0.2)
    xg, x2 = w.buf('xg', 1, Kg), w.buf('x2', 1, Kg)
    gg = w.buf('gg', Kg, scale=0.5)
    resg = w.buf('resg', 1, Ng)
    for pro in range(3):
        w.task('gemv_bf16', x=xg, x2=x2 if pro == 2 else None, gamma=gg if pro == 1 else None, w=wg,
               out=w.zeros(f'gv{pro}', 1, Ng, 'bf16' if pro == 2 else 'f32'), res=resg if pro else None, n0=0 if pro else 3,
               n1=Ng, K=Kg, pro=pro, eps=1e-6)
    # split-context decode attention, with and without fused RoPE + append
    B, H, Hkv, hd, Tmax, S = 2, 4, 2, 16, 40, 3
    lens = w.ints('dlens', [13, 30])
    for fl in (0, 1, 3):
        kc, vc = w.buf(f'kc{fl}', B * Hkv * Tmax, hd, 'bf16'), w.buf(f'vc{fl}', B * Hkv * Tmax, hd, 'bf16')
        q = w.buf(f'dq{fl}', B, H * hd)
        kn = w.buf(f'kn{fl}', B, Hkv * hd) if fl else None
        vn = w.buf(f'vn{fl}', B, Hkv * hd) if fl else None
        part = w.zeros(f'part{fl}', B * S * H, hd + 2)
        o = w.zeros(f'do{fl}', B, H * hd, 'bf16' if fl == 3 else 'f32')
        for b in range(B):
            ps = [w.task('attn_decode_part', q=q, kc=kc, vc=vc, lens=lens, part=part, knew=kn, vnew=vn, b=b, kvh=kh, s=s, S=S, H=H,
                         Hkv=Hkv, hd=hd, Tmax=Tmax, scale=0.25, theta=10000.0, flags=fl) for kh in range(Hkv) for s in range(S)]
            w.task('attn_decode_merge', after=ps, part=part, o=o, b=b, h0=0, h1=H, S=S, H=H, hd=hd)
    # optimizer schedule and misc
    st = w.ints('st', [7])
    lr = w.zeros('lr', 1)
    t2 = w.task('lr_schedule', step=st, lr=lr, kind=1, base=3e-3, warmup=4, total=20, min_ratio=0.1)
    p, g, m, v = w.buf('p', 50), w.buf('g', 50), w.buf('m', 50, scale=0.01), w.pos('v', 50, 1e-5)
    w.task('adamw_lr', after=[t2], p=p, g=g, m=m, v=v, gscale=None, step=st, e0=0, e1=50, lr=lr, b1=0.9, b2=0.999, eps=1e-8, wd=0.0)
    for kind, wu in ((0, 0), (2, 10)):
        w.task('lr_schedule', step=st, lr=w.zeros(f'lr{kind}', 1), kind=kind, base=1e-3, warmup=wu, total=30, min_ratio=0.0)
    w.task('scale_flat', x=x, out=w.zeros('sf', 10, 16), alpha=-1.5, e0=0, e1=160)
    w.task('add_rowtile', x=x, pos=w.buf('pt', 4, 16), out=w.zeros('art', 10, 16), r0=1, r1=10, T=4, d=16)
    # fused GEMM epilogues
    Mf, Nf, Kf = 40, 70, 24
    Af, Bf = w.buf('Af', Mf, Kf), w.buf('Bf', Kf, Nf)
    gate = w.buf('gatef', Mf, Nf)
    upf, outf = w.zeros('upf', Mf, Nf), w.zeros('outf', Mf, Nf)
    dgf, duf = w.zeros('dgf', Mf, Nf), w.zeros('duf', Mf, Nf)
    upv = w.buf('upv', Mf, Nf)
    for n0 in (0, 64):
        w.task('matmul_tile_silu_mul', a=Af, b=Bf, out=outf, gate=gate, up=upf, m0=0, n0=n0, M=Mf, N=Nf, K=Kf, flags=0, alpha=1.0)
        w.task('matmul_tile_silu_mul_bwd', a=Af, b=Bf, gate=gate, up=upv, dgate=dgf, dup=duf, m0=0, n0=n0, M=Mf, N=Nf, K=Kf, flags=0,
               alpha=1.0)
    return w.spec()


def bf16_storage_ops():
    """GPT-pack operators on bf16-storage buffers (the bf16 training and serving paths)."""
    w = W(50)
    T, H, hd, B = 32, 2, 32, 2
    R, D = B * T, H * hd
    x = w.buf('x', R, D, 'bf16')
    gam, bet = w.buf('gam', D, scale=0.3), w.buf('bet', D)
    ln, mean, rstd = w.zeros('ln', R, D, 'bf16'), w.zeros('mean', R), w.zeros('rstd', R)
    t1 = w.task('layernorm_fwd', x=x, gamma=gam, beta=bet, out=ln, mean=mean, rstd=rstd, r0=0, r1=R, d=D, eps=1e-5)
    dy = w.buf('dy', R, D, 'bf16')
    dx = w.zeros('dx', R, D, 'bf16')
    w.task('layernorm_bwd_dx', after=[t1], x=x, dy=dy, gamma=gam, mean=mean, rstd=rstd, dx=dx, r0=0, r1=R, d=D, acc=0)
    w.task('norm_bwd_params', after=[t1], x=x, dy=dy, mean=mean, rstd=rstd, dgamma=w.zeros('dg', D), dbeta=w.zeros('db', D), R=R, d=D,
           c0=0, c1=D, acc=0)
    w.task('residual_add', a=x, b=dy, out=w.zeros('ra', R, D, 'bf16'), e0=0, e1=R * D)
    w.task('gelu_bwd', x=x, dy=dy, dx=w.zeros('gb', R, D, 'bf16'), e0=0, e1=R * D, acc=0)
    w.task('colsum', x=x, out=w.zeros('cs', D), R=R, c0=0, c1=D, acc=0)
    q, k, v, do = (w.buf(n, R, D, 'bf16') for n in ('q', 'k', 'v', 'do'))
    o, lse = w.zeros('o', R, D, 'bf16'), w.zeros('lse', B * H * T)
    fw = [w.task('attn_fwd', q=q, k=k, v=v, o=o, lse=lse, b=b, h=h, q0=0, T=T, H=H, Hkv=H, hd=hd, scale=0.17) for b in range(B) for h in range(H)]
    delta = w.zeros('delta', B * H * T)
    td = w.task('attn_bwd_delta', after=fw, o=o, do=do, delta=delta, r0=0, r1=R, T=T, H=H, hd=hd)
    dq, dk, dv = w.zeros('dq', R, D, 'bf16'), w.zeros('dk', R, D, 'bf16'), w.zeros('dv', R, D, 'bf16')
    for b in range(B):
        for h in range(H):
            w.task('attn_bwd_dq', after=[td], q=q, k=k, v=v, do=do, lse=lse, delta=delta, dq=dq, b=b, h=h, q0=0, T=T, H=H, Hkv=H, hd=hd, scale=0.17)
            w.task('attn_bwd_dkv', after=[td], q=q, k=k, v=v, do=do, lse=lse, delta=delta, dk=dk, dv=dv, b=b, kvh=h, k0=0, T=T, H=H, hd=hd, scale=0.17)
    w.task('rope_fwd', x=q, out=w.zeros('qr', R, D, 'bf16'), pos=None, r0=0, r1=R, T=T, H=H, hd=hd, theta=10000.0)
    lg = w.buf('lg', 8, 40, 'bf16', scale=2.0)
    tg = w.ints('tg', [w.rng.randrange(40) for _ in range(8)])
    w.task('softmax_ce_fused', logits=lg, tgt=tg, rowloss=w.zeros('rl', 8), lse=w.zeros('ls', 8), dlogits=w.zeros('dl', 8, 40, 'bf16'),
           r0=0, r1=8, V=40, ignore=-1, N=8, scale=1.0)
    ids = w.ints('ids', [w.rng.randrange(20) for _ in range(R)])
    w.task('embedding_fwd', ids=ids, wte=w.buf('wte', 20, D), wpe=None, out=w.zeros('emb', R, D, 'bf16'), r0=0, r1=R, T=T, d=D)
    w.task('silu_mul_fwd', gate=x, up=dy, out=w.zeros('sm', R, D, 'bf16'), e0=0, e1=R * D)
    return w.spec()


CASES = {'core': core, 'versions': versions, 'gpt_ops': gpt_ops, 'extra_ops': extra_ops, 'bf16_storage': bf16_storage_ops}
