"""GPU parity of causal attention (ops 45-48) on bf16 and on f32 storage, at shapes that take the MFMA bodies (T a
multiple of 64, hd 32 / 64 / 128, 16-byte aligned head slices), against the CPU oracle (double arithmetic on the same
inputs, reference: runtime/ref_gpt.py:279-364).

Tolerances: o, dq, dk, dv are bf16 storage; the device rounds P (and dS) to bf16 for the second product of each pair,
so these are held to a relative L2 error of 1e-2 (the reference's own bf16 attention deviates from fp64 by up to
1.69e-2 in its step-1 gradients, reference README.md:212). lse is f32 computed from fp32-accumulated exact bf16
products: 2e-5. delta = rowsum(dO * O) is f32 but inherits the deviation of the bf16 O it is computed from: 1e-2. On f32 storage every
product is an exact f32 product accumulated in f32 (v_mfma_f32_32x32x2f32): every output within 2e-5.
"""
import math

import numpy as np
import pytest

import oracle
from gpu_check import compare_run
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.executor import Executor
from kvm_amd.workloads import Builder, Workload

pytestmark = pytest.mark.gpu
TOL_BF16 = 1e-2


def _attn_graph(B, H, Hkv, T, hd, ops, dt='bf16'):
    b = Builder(11)
    N = B * T
    b.normal('q', N, H * hd, dt, scale=1.0)
    b.normal('k', N, Hkv * hd, dt, scale=1.0)
    b.normal('v', N, Hkv * hd, dt, scale=1.0)
    b.normal('do', N, H * hd, dt, scale=1.0)
    b.fill('o', N, H * hd, dt)
    b.fill('lse', B * H * T)
    b.fill('delta', B * H * T)
    for nm, cols in (('dq', H * hd), ('dk', Hkv * hd), ('dv', Hkv * hd)):
        b.fill(nm, N, cols, dt)
    sc = 1.0 / math.sqrt(hd)
    fw = [b.task('attn_fwd', q='q', k='k', v='v', o='o', lse='lse', b=bb, h=h, q0=q0, T=T, H=H, Hkv=Hkv, hd=hd, scale=sc)
          for bb in range(B) for h in range(H) for q0 in range(0, T, 128)]
    if 'bwd' in ops:
        de = [b.task('attn_bwd_delta', after=fw, o='o', do='do', delta='delta', r0=0, r1=N, T=T, H=H, hd=hd)]
        for bb in range(B):
            for h in range(H):
                for q0 in range(0, T, 128):
                    b.task('attn_bwd_dq', after=de, q='q', k='k', v='v', do='do', lse='lse', delta='delta', dq='dq', b=bb, h=h, q0=q0, T=T,
                           H=H, Hkv=Hkv, hd=hd, scale=sc)
            for kh in range(Hkv):
                for k0 in range(0, T, 128):
                    b.task('attn_bwd_dkv', after=de, q='q', k='k', v='v', do='do', lse='lse', delta='delta', dk='dk', dv='dv', b=bb, kvh=kh,
                           k0=k0, T=T, H=H, hd=hd, scale=sc)
    return Workload(b.spec(), b.init_override)


def _check(w, f32=False):
    lb = bl.load(compiler.compile_spec(w.spec))
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    ref = oracle.run(lb, [x.copy() for x in init])
    ex = Executor.from_bundle(lb, buffers=init)
    ex.run()
    if f32:
        bad = compare_run(ex, lb.metadata, ref, tol_f32=2e-5)
        ex.close()
        assert not bad, bad
        return
    bad = compare_run(ex, lb.metadata, ref, tol_bf16=TOL_BF16, skip=('delta',))
    names = [m['name'] for m in lb.metadata['buffers']]
    bad += compare_run(ex, {'buffers': [lb.metadata['buffers'][names.index('delta')]]}, {'buffers': [ref['buffers'][names.index('delta')]]},
                       tol_f32=TOL_BF16)
    ex.close()
    assert not bad, bad


@pytest.mark.parametrize('hd', [64, 32, 128])
def test_attention_fwd_mfma(hd):
    print(f'attn fwd hd {hd}', flush=True)
    _check(_attn_graph(2, 2, 2, 256, hd, ('fwd',)))


def test_attention_fwd_gqa_partial_task():
    """GQA (4 query heads on 2 kv heads) and T = 192: the last task of each head covers only 64 rows."""
    print('attn fwd gqa T192', flush=True)
    _check(_attn_graph(1, 4, 2, 192, 64, ('fwd',)))


@pytest.mark.parametrize('hd,H,Hkv', [(64, 2, 2), (64, 4, 2), (32, 2, 2)])
def test_attention_bwd(hd, H, Hkv):
    print(f'attn bwd hd {hd} H {H} Hkv {Hkv}', flush=True)
    _check(_attn_graph(1, H, Hkv, 256, hd, ('fwd', 'bwd')))


@pytest.mark.parametrize('hd,H,Hkv,T,ops', [(64, 2, 2, 256, ('fwd', 'bwd')), (32, 4, 2, 192, ('fwd', 'bwd')), (128, 2, 1, 256, ('fwd',))])
def test_attention_f32_mfma(hd, H, Hkv, T, ops):
    """f32 storage on the fp32 MFMA bodies: forward (hd 32 / 64 / 128), dQ and dK / dV (hd 32 / 64), MHA and GQA, a
    T whose last task covers 64 rows."""
    print(f'attn f32 hd {hd} H {H} Hkv {Hkv} T {T} {ops}', flush=True)
    _check(_attn_graph(1, H, Hkv, T, hd, ops, dt='f32'), f32=True)
