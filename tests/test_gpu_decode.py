"""GPU parity of the decode GEMVs at Qwen3-8B widths (K = 4096 and 12288) against the CPU oracle: the one-row
reference op gemv_bf16 (134) and this executor's batched form gemv_bf16_rows (301), with the RMSNorm and SwiGLU
prologues and a residual. v = bf16(prologue(x)) on both sides; the oracle sums exact products in double, the device
in fp32 on MFMA: f32 outputs within a relative L2 error of 2e-5."""
import pytest

import oracle
from gpu_check import compare_run
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.executor import Executor
from kvm_amd.workloads import Builder, Workload, split

pytestmark = pytest.mark.gpu


def _run(b, tol=2e-5):
    w = Workload(b.spec(), b.init_override)
    lb = bl.load(compiler.compile_spec(w.spec))
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    ref = oracle.run(lb, [x.copy() for x in init])
    ex = Executor.from_bundle(lb, buffers=init)
    ex.run()
    bad = compare_run(ex, lb.metadata, ref, tol_f32=tol)
    ex.close()
    assert not bad, bad


@pytest.mark.parametrize('pro,K', [(0, 4096), (1, 4096), (2, 12288)])
def test_gemv_one_row(pro, K):
    print(f'gemv_bf16 pro {pro} K {K}', flush=True)
    N = 1200
    b = Builder(21)
    b.normal('x', 1, K, 'f32', scale=1.0)
    b.normal('x2', 1, K, 'f32', scale=1.0)
    b.normal('g', 1, K, 'f32', scale=1.0)
    b.normal('w', N, K, 'bf16', scale=0.02)
    b.normal('res', 1, N, 'f32', scale=1.0)
    b.fill('out', 1, N)
    for lo, hi in split(N, 13):                       # ragged row ranges (92 or 93 rows: partial 16-row blocks)
        b.task('gemv_bf16', x='x', x2='x2' if pro == 2 else None, gamma='g' if pro == 1 else None, w='w', out='out', res='res',
               n0=lo, n1=hi, K=K, pro=pro, eps=1e-6)
    _run(b)


@pytest.mark.parametrize('M,pro,K', [(8, 1, 4096), (8, 2, 12288), (3, 0, 4096), (16, 0, 4096)])
def test_gemv_rows(M, pro, K):
    print(f'gemv_bf16_rows M {M} pro {pro} K {K}', flush=True)
    N = 512
    b = Builder(23)
    b.normal('x', M, K, 'f32', scale=1.0)
    b.normal('x2', M, K, 'f32', scale=1.0)
    b.normal('g', 1, K, 'f32', scale=1.0)
    b.normal('w', N, K, 'bf16', scale=0.02)
    b.normal('res', M, N, 'f32', scale=1.0)
    b.fill('out', M, N)
    for lo, hi in split(N // 16, 5):
        b.task('gemv_bf16_rows', x='x', x2='x2' if pro == 2 else None, gamma='g' if pro == 1 else None, w='w', out='out', res='res',
               n0=16 * lo, n1=16 * hi, K=K, M=M, pro=pro, eps=1e-6)
    _run(b)


LONG = [1500, 700]      # splits of 751 / 351 tokens at S = 2, 501 / 234 at S = 3: the MFMA form (over 256 tokens)


@pytest.mark.parametrize('G,fl,S,lens', [(4, 3, 3, None), (4, 1, 16, None), (4, 0, 40, None), (8, 3, 5, None), (2, 1, 7, None),
                                         (1, 0, 9, None), (4, 3, 2, LONG), (8, 1, 2, LONG), (2, 0, 3, LONG), (1, 3, 2, LONG)])
def test_attn_decode_parts(G, fl, S, lens):
    """Split-context decode attention (op 135) and the merge (op 136) at hd = 128 (the streaming form): two sequences
    of different lengths, splits longer than one 128-token block (S = 3), short ones and empty ones (S = 40 with a
    30-token context), with RoPE + cache append + bf16 rounding of the rotated query (flags 3), RoPE + append (1) or
    neither (0); splits over 256 tokens (LONG) take the MFMA form, with a partial last chunk."""
    print(f'attn_decode_part G {G} flags {fl} S {S} lens {lens}', flush=True)
    B, Hkv, hd = 2, 2, 128
    H = G * Hkv
    lens = lens or ([700, 30] if S == 40 else [700, 301])
    Tmax = max(lens) + 1
    b = Builder(31)
    b.normal('q', B, H * hd, 'bf16', scale=1.0)
    b.normal('kc', B * Hkv * Tmax, hd, 'bf16', scale=1.0)
    b.normal('vc', B * Hkv * Tmax, hd, 'bf16', scale=1.0)
    b.normal('kn', B, Hkv * hd, 'bf16', scale=1.0)
    b.normal('vn', B, Hkv * hd, 'bf16', scale=1.0)
    b.values('lens', lens, B, 1, 'i32')
    b.fill('part', B * S * H, hd + 2, 'f32')
    b.fill('o', B, H * hd, 'f32')
    for bb in range(B):
        ts = [b.task('attn_decode_part', q='q', kc='kc', vc='vc', lens='lens', part='part', knew='kn', vnew='vn', b=bb, kvh=kh, s=s, S=S,
                     H=H, Hkv=Hkv, hd=hd, Tmax=Tmax, scale=1.0 / hd ** 0.5, theta=1e6, flags=fl)
              for kh in range(Hkv) for s in range(S)]
        b.task('attn_decode_merge', after=ts, part='part', o='o', b=bb, h0=0, h1=H, S=S, H=H, hd=hd)
    _run(b, tol=1e-4)


@pytest.mark.parametrize('G,fl,S,qdt,lens', [(4, 1, 32, 'f32', None), (4, 3, 3, 'f32', None), (8, 1, 5, 'bf16', None), (1, 3, 9, 'f32', None),
                                              (4, 1, 2, 'f32', LONG), (8, 3, 2, 'bf16', LONG)])
def test_attn_decode_parts_qkn(G, fl, S, qdt, lens):
    """Op 306: per-head RMSNorm of the query heads and of the new key inside the split-context attention task (the
    Qwen3 q/k norm), against the oracle's op 300 + op 135 composition. eps 0.25 (comparable to the mean square of
    the unit-scale inputs) so that a misread eps fails."""
    print(f'attn_decode_part_qkn G {G} flags {fl} S {S} q {qdt} lens {lens}', flush=True)
    B, Hkv, hd = 2, 2, 128
    H = G * Hkv
    lens = lens or [700, 301]
    Tmax = max(lens) + 1
    b = Builder(37)
    b.normal('q', B, H * hd, qdt, scale=1.0)
    b.normal('kc', B * Hkv * Tmax, hd, 'bf16', scale=1.0)
    b.normal('vc', B * Hkv * Tmax, hd, 'bf16', scale=1.0)
    b.normal('kn', B, Hkv * hd, qdt, scale=1.0)
    b.normal('vn', B, Hkv * hd, 'f32', scale=1.0)
    b.normal('qg', 1, hd, 'f32', scale=1.0)
    b.normal('kg', 1, hd, 'f32', scale=1.0)
    b.values('lens', lens, B, 1, 'i32')
    b.fill('part', B * S * H, hd + 2, 'f32')
    b.fill('o', B, H * hd, 'f32')
    for bb in range(B):
        ts = [b.task('attn_decode_part_qkn', q='q', kc='kc', vc='vc', lens='lens', part='part', knew='kn', vnew='vn', b=bb, kvh=kh, s=s,
                     S=S, H=H, Hkv=Hkv, hd=hd, Tmax=Tmax, scale=1.0 / hd ** 0.5, theta=1e6, flags=fl, qgamma='qg', kgamma='kg', eps=0.25)
              for kh in range(Hkv) for s in range(S)]
        b.task('attn_decode_merge', after=ts, part='part', o='o', b=bb, h0=0, h1=H, S=S, H=H, hd=hd)
    _run(b, tol=1e-4)


@pytest.mark.parametrize('G,S,path,lens', [(4, 32, 0, None), (4, 32, 1, None), (8, 5, 0, None), (2, 3, 1, None), (4, 2, 0, LONG),
                                           (4, 2, 1, LONG)])
def test_attn_decode_part_merge(G, S, path, lens):
    """Op 310 (op 306 whose last split per kv head merges that head's query heads) against the oracle's op 306 + op
    136 composition, on the dynamic and the static path (where the GQA-4 body is inlined and its first block staged
    before the wait); two launches in a row, so the split counts must have returned to 0."""
    print(f'attn_decode_part_merge G {G} S {S} path {path} lens {lens}', flush=True)
    B, Hkv, hd = 2, 2, 128
    H = G * Hkv
    lens = lens or [700, 301]
    Tmax = max(lens) + 1
    b = Builder(53)
    b.normal('q', B, H * hd, 'f32', scale=1.0)
    b.normal('kc', B * Hkv * Tmax, hd, 'bf16', scale=1.0)
    b.normal('vc', B * Hkv * Tmax, hd, 'bf16', scale=1.0)
    b.normal('kn', B, Hkv * hd, 'f32', scale=1.0)
    b.normal('vn', B, Hkv * hd, 'f32', scale=1.0)
    b.normal('qg', 1, hd, 'f32', scale=1.0)
    b.normal('kg', 1, hd, 'f32', scale=1.0)
    b.values('lens', lens, B, 1, 'i32')
    b.fill('part', B * S * H, hd + 2, 'f32')
    b.fill('o', B, H * hd, 'f32')
    b.fill('cnt', B * Hkv, 1, 'i32')
    for bb in range(B):
        for kh in range(Hkv):
            for s in range(S):
                b.task('attn_decode_part_merge', q='q', kc='kc', vc='vc', lens='lens', part='part', knew='kn', vnew='vn', b=bb, kvh=kh,
                       s=s, S=S, H=H, Hkv=Hkv, hd=hd, Tmax=Tmax, scale=1.0 / hd ** 0.5, theta=1e6, flags=1, qgamma='qg', kgamma='kg',
                       eps=0.25, o='o', cnt='cnt')
    w = Workload(b.spec(), b.init_override)
    lb = bl.load(compiler.compile_spec(w.spec))
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    ref = oracle.run(lb, [x.copy() for x in init])
    ex = Executor.from_bundle(lb, buffers=init, path=path)
    for launch in range(2):      # the second launch re-appends the same new row: the same results
        if launch:
            ex.relaunch()
            ex.finish()
        else:
            ex.run()
        assert ex.path() == path
        bad = compare_run(ex, lb.metadata, ref, tol_f32=1e-4)
        assert not bad, (launch, bad)
    ex.close()


@pytest.mark.parametrize('M,N,path', [(1, 768, 1), (1, 768, 0), (8, 512, 1), (3, 200, 0)])
def test_gemv_swiglu(M, N, path):
    """Op 311 (fused gate / up / silu(g) u) at K = 4096: bit for bit the device's own op 301 on the gate rows and on the
    up rows followed by op 98 (silu_mul_fwd) into bf16, and the bf16 result within the bf16 tolerance of the oracle;
    on the static path (pre-wait weight ring, inlined body) and the dynamic one; N = 200: ragged 16-row blocks."""
    print(f'gemv_swiglu M {M} N {N} path {path}', flush=True)
    K = 4096
    b = Builder(29)
    b.normal('x', M, K, 'f32', scale=1.0)
    b.normal('g', 1, K, 'f32', scale=1.0)
    b.normal('wg', N, K, 'bf16', scale=0.02)
    b.normal('wu', N, K, 'bf16', scale=0.02)
    b.buf('h', M, N, 'bf16', {'kind': 'fill', 'value': 0})
    b.buf('h2', M, N, 'bf16', {'kind': 'fill', 'value': 0})
    b.fill('gg', M, N), b.fill('uu', M, N)
    parts = split(N // 16, 7) if N % 16 == 0 else [(0, 5), (5, 9), (9, 12.5)]
    for lo, hi in parts:
        b.task('gemv_swiglu', x='x', gamma='g', wg='wg', wu='wu', out='h', n0=int(16 * lo), n1=int(16 * hi), K=K, M=M, eps=1e-6)
    tg = b.task('gemv_bf16_rows', x='x', x2=None, gamma='g', w='wg', out='gg', res=None, n0=0, n1=N, K=K, M=M, pro=1, eps=1e-6)
    tu = b.task('gemv_bf16_rows', x='x', x2=None, gamma='g', w='wu', out='uu', res=None, n0=0, n1=N, K=K, M=M, pro=1, eps=1e-6)
    b.task('silu_mul_fwd', after=[tg, tu], gate='gg', up='uu', out='h2', e0=0, e1=M * N)
    w = Workload(b.spec(), b.init_override)
    lb = bl.load(compiler.compile_spec(w.spec))
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    ref = oracle.run(lb, [x.copy() for x in init])
    ex = Executor.from_bundle(lb, buffers=init, path=path)
    ex.run()
    assert ex.path() == path
    h, h2 = ex.read_raw('h'), ex.read_raw('h2')
    assert (h != 0).any() and (h == h2).all()
    bad = compare_run(ex, lb.metadata, ref, tol_f32=2e-5)
    ex.close()
    assert not bad, bad
