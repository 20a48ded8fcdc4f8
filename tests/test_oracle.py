"""Pins of the CPU oracle: the reference VM's own outputs (tests/golden), its SplitMix64 vectors, and closed forms."""
import json
import math
import struct

import numpy as np
import pytest

import oracle
from conftest import GOLDEN, REPO, golden_cases
from kvm_amd import bundle as bl
from kvm_amd import compiler, initgen
from cases import W


@pytest.mark.parametrize('case', golden_cases())
def test_oracle_matches_reference_vm_bitwise(case):
    d = GOLDEN / case
    g = json.loads((d / 'golden.json').read_text())
    r = oracle.run(d)
    meta = json.loads((d / 'metadata.json').read_text())
    for m, x in zip(meta['buffers'], r['buffers']):
        want = np.array(g['buffers'][m['name']], np.int32 if m['dtype'] == 1 else np.float32)
        assert np.array_equal(want.view(np.uint32), x.view(np.uint32)), m['name']
    assert r['versions'] == g['versions']
    assert [x['observed'] for x in g['reads']] == r['observed']


def _vectors():
    lines = (REPO / 'tests/golden/data/initgen_vectors.txt').read_text().split('\n')
    for k in range(0, len(lines) - 1, 2):
        seed, draws, bh, ch, n = lines[k].split()
        f = lambda h: struct.unpack('<f', struct.pack('<I', int(h, 16)))[0]
        yield int(seed), int(draws), f(bh), f(ch), int(n), [int(h, 16) for h in lines[k + 1].split()]


def test_seeded_init_vectors():
    """The reference's SplitMix64 known answers (tests/gpu/initgen_vectors.txt of the reference)."""
    for seed, draws, bias, coef, n, want in _vectors():
        assert initgen.seeded(seed, n, draws, bias, coef).view(np.uint32).tolist() == want
        assert oracle.seeded(n, seed, draws, bias, coef).view(np.uint32).tolist() == want


def _run_one(w):
    b = compiler.compile_spec(w.spec())
    return oracle.run(b), b


def _get(r, b, name):
    return r['buffers'][[m['name'] for m in b.metadata['buffers']].index(name)]


def test_matmul_tile_closed_form():
    """Tile GEMM against an fp64 product (a transposed operand or dropped term fails this)."""
    w = W(3)
    M, N, K = 70, 50, 33
    w.buf('A', K, M), w.buf('B', N, K), w.buf('bias', 1, N), w.zeros('out', M, N)
    for m0 in (0, 64):
        w.task('matmul_tile', a='A', b='B', out='out', bias='bias', res=None, pre=None, m0=m0, n0=0, M=M, N=N, K=K, flags=3, alpha=0.5)
    r, b = _run_one(w)
    A, B, bias = (_get(r, b, n).astype(np.float64) for n in ('A', 'B', 'bias'))
    want = 0.5 * (A.reshape(K, M).T @ B.reshape(N, K).T) + bias
    got = _get(r, b, 'out').reshape(M, N)
    assert np.abs(got - want).max() < 1e-5 * np.abs(want).max()


def test_attention_closed_form_and_decode_consistency():
    """Causal attention = softmax(QK^T*scale)V in fp64; decode attention of the last token = last row of the forward."""
    w = W(4)
    T, H, hd = 17, 2, 16
    w.buf('q', T, H * hd), w.buf('k', T, H * hd), w.buf('v', T, H * hd)
    w.zeros('o', T, H * hd), w.zeros('lse', H * T)
    for h in range(H):
        w.task('attn_fwd', q='q', k='k', v='v', o='o', lse='lse', b=0, h=h, q0=0, T=T, H=H, Hkv=H, hd=hd, scale=0.3)
    r, b = _run_one(w)
    q, k, v = (_get(r, b, n).astype(np.float64).reshape(T, H, hd) for n in 'qkv')
    o = _get(r, b, 'o').reshape(T, H, hd)
    for h in range(H):
        s = q[:, h] @ k[:, h].T * 0.3
        s[np.triu_indices(T, 1)] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        want = (p / p.sum(1, keepdims=True)) @ v[:, h]
        assert np.abs(o[:, h] - want).max() < 1e-6
    # decode: the cache holds k/v rows 0..T-1 (lens = T-1: the last token was just appended)
    w2 = W(4)
    w2.buf('q', T, H * hd), w2.buf('k', T, H * hd), w2.buf('v', T, H * hd)   # same seeds as above
    qd = q[T - 1].reshape(1, -1).astype(np.float32)
    w2.buf('qd', 1, H * hd, init={'kind': 'values', 'values': qd.ravel().tolist()})
    for name, src in (('kc', k), ('vc', v)):
        cache = np.zeros((H * T, hd), np.float32)
        for h in range(H):
            cache[h * T:(h + 1) * T] = src[:, h]
        w2.buf(name, H * T, hd, init={'kind': 'values', 'values': cache.ravel().tolist()})
    w2.ints('lens', [T - 1])
    w2.zeros('od', 1, H * hd)
    for h in range(H):
        w2.task('attn_decode', q='qd', kc='kc', vc='vc', lens='lens', o='od', b=0, h=h, H=H, Hkv=H, hd=hd, Tmax=T, scale=0.3)
    r2, b2 = _run_one(w2)
    assert np.abs(_get(r2, b2, 'od') - o[T - 1].ravel()).max() < 1e-6


def test_adamw_step1_fp64():
    """AdamW at t=1 reduces to p(1-lr*wd) - lr*sign-like(g) (m/(1-b1) = g, v/(1-b2) = g^2)."""
    w = W(5)
    n = 64
    w.buf('p', n), w.buf('g', n), w.zeros('m', n), w.zeros('v', n), w.ints('step', [1])
    w.task('adamw', p='p', g='g', m='m', v='v', gscale=None, step='step', e0=0, e1=n, lr=1e-2, b1=0.9, b2=0.95, eps=1e-8, wd=0.1)
    r, b = _run_one(w)
    w0 = bl.materialize(b.metadata['buffers'][0]).astype(np.float64)
    g = _get(r, b, 'g').astype(np.float64)
    want = w0 * (1 - 1e-3) - 1e-2 * g / (np.abs(g) + 1e-8)
    assert np.abs(_get(r, b, 'p') - want).max() < 1e-6


def _rne_bf16(x):
    """float32 -> bf16 (round to nearest, ties to even) by integer arithmetic on the bits, back as float32."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def test_adamw_bf16_matches_adamw_and_rounds_the_new_weight():
    """Op 305 leaves p, m, v exactly as op 54 does and stores bf16(p_new) in sh (bf16 storage)."""
    w = W(11)
    n = 203
    for pre in ('a', 'b'):
        w.buf(pre + 'p', n), w.buf(pre + 'm', n, scale=0.1), w.pos(pre + 'v', n, 0.01)
    w.buf('g', n), w.ints('step', [4]), w.zeros('sh', n, 1, 'bf16')
    kw = dict(g='g', gscale=None, step='step', e0=0, e1=n, lr=1e-2, b1=0.9, b2=0.95, eps=1e-8, wd=0.1)
    r, b = _run_one(w)
    # same initial state for both: copy a* into b* through the materialised init
    meta = b.metadata['buffers']
    init = {m['name']: bl.materialize(m) for m in meta}
    w2 = W(11)
    for nm in ('p', 'm', 'v'):
        w2.buf(nm, n, 1, 'f32', {'kind': 'values', 'values': init['a' + nm].tolist()})
    w2.buf('g', n, 1, 'f32', {'kind': 'values', 'values': init['g'].tolist()})
    w2.ints('step', [4]), w2.zeros('sh', n, 1, 'bf16')
    for nm in ('p', 'm', 'v'):
        w2.buf('q' + nm, n, 1, 'f32', {'kind': 'values', 'values': init['a' + nm].tolist()})
    w2.task('adamw', p='p', m='m', v='v', **kw)
    w2.task('adamw_bf16', p='qp', m='qm', v='qv', sh='sh', **kw)
    r, b = _run_one(w2)
    for nm in ('p', 'm', 'v'):
        assert np.array_equal(_get(r, b, nm).view(np.uint32), _get(r, b, 'q' + nm).view(np.uint32)), nm
    assert not np.array_equal(_get(r, b, 'p'), init['ap'])
    assert np.array_equal(_get(r, b, 'sh').view(np.uint32), _rne_bf16(_get(r, b, 'p')).view(np.uint32))


def test_gpt_bf16_shadow_starts_as_rounded_master():
    """The bf16 GEMM copies of a bf16 GPT start as the fp32 masters rounded to bf16 (they are not rewritten before the
    first forward; AdamW refreshes them afterwards)."""
    from kvm_amd.workloads import gpt
    wl = gpt.build(gpt.GPTConfig.tiny(dtype='bf16', layers=1, steps=1))
    bufs = {m['name']: m for m in compiler.compile_spec(wl.spec).metadata['buffers']}
    for name in ('wte', 'wq.0', 'w2.0'):
        a = oracle.materialize(bufs[name], wl.init_override.get(name))
        s = oracle.materialize(bufs[name + '.bf'], wl.init_override.get(name + '.bf'))
        assert np.array_equal(s.view(np.uint32), _rne_bf16(a).view(np.uint32)), name


def test_attn_decode_part_qkn_is_head_norm_then_part():
    """Op 306 equals op 300 on q and the new key followed by op 135 (bitwise), and differs from op 135 alone."""
    H, Hkv, hd, L, S = 4, 2, 128, 37, 3
    Tm = L + 2

    def graph(fused):
        w = W(41)
        w.buf('q', 1, H * hd), w.buf('kn', 1, Hkv * hd), w.buf('vn', 1, Hkv * hd), w.buf('qg', hd), w.buf('kg', hd)
        w.buf('kc', Hkv * Tm, hd), w.buf('vc', Hkv * Tm, hd), w.ints('lens', [L]), w.zeros('part', S * H, hd + 2)
        w.zeros('qn', 1, H * hd), w.zeros('kn2', 1, Hkv * hd)
        kw = dict(kc='kc', vc='vc', lens='lens', part='part', vnew='vn', b=0, S=S, H=H, Hkv=Hkv, hd=hd, Tmax=Tm,
                  scale=1.0 / hd ** 0.5, theta=1e6, flags=1)
        if fused == 'fused':
            for kh in range(Hkv):
                for s in range(S):
                    w.task('attn_decode_part_qkn', q='q', knew='kn', kvh=kh, s=s, qgamma='qg', kgamma='kg', eps=1e-6, **kw)
        else:
            pre = []
            if fused == 'composed':
                pre = [w.task('head_rmsnorm', x='q', gamma='qg', out='qn', r0=0, r1=1, H=H, hd=hd, eps=1e-6),
                       w.task('head_rmsnorm', x='kn', gamma='kg', out='kn2', r0=0, r1=1, H=Hkv, hd=hd, eps=1e-6)]
            q, kn = ('qn', 'kn2') if fused == 'composed' else ('q', 'kn')
            for kh in range(Hkv):
                for s in range(S):
                    w.task('attn_decode_part', after=pre, q=q, knew=kn, kvh=kh, s=s, **kw)
        r, b = _run_one(w)
        return _get(r, b, 'part'), _get(r, b, 'kc')
    f, c, p = graph('fused'), graph('composed'), graph('plain')
    assert np.array_equal(f[0].view(np.uint32), c[0].view(np.uint32))
    assert np.array_equal(f[1].view(np.uint32), c[1].view(np.uint32))
    assert not np.array_equal(f[0], p[0])


def test_attn_decode_part_merge_is_part_then_merge():
    """Op 310 equals op 306 followed by op 136 over each kv head's query heads (bitwise: part, caches and the merged
    output), whichever split completes last, and leaves every split count at 0."""
    H, Hkv, hd, L, S = 8, 2, 128, 41, 4
    Tm = L + 2
    G = H // Hkv

    def graph(fused, order):
        w = W(43)
        w.buf('q', 1, H * hd), w.buf('kn', 1, Hkv * hd), w.buf('vn', 1, Hkv * hd), w.buf('qg', hd), w.buf('kg', hd)
        w.buf('kc', Hkv * Tm, hd), w.buf('vc', Hkv * Tm, hd), w.ints('lens', [L]), w.zeros('part', S * H, hd + 2)
        w.zeros('att', 1, H * hd), w.ints('cnt', [0] * Hkv)
        kw = dict(q='q', kc='kc', vc='vc', lens='lens', part='part', knew='kn', vnew='vn', b=0, S=S, H=H, Hkv=Hkv, hd=hd, Tmax=Tm,
                  scale=1.0 / hd ** 0.5, theta=1e6, flags=1, qgamma='qg', kgamma='kg', eps=1e-6)
        parts = []
        for kh, s in order:
            if fused:
                parts.append(w.task('attn_decode_part_merge', kvh=kh, s=s, o='att', cnt='cnt', after=parts[-1:], **kw))
            else:
                parts.append(w.task('attn_decode_part_qkn', kvh=kh, s=s, after=parts[-1:], **kw))
        if not fused:
            for kh in range(Hkv):
                w.task('attn_decode_merge', after=parts, part='part', o='att', b=0, h0=kh * G, h1=kh * G + G, S=S, H=H, hd=hd)
        r, b = _run_one(w)
        return [_get(r, b, n) for n in ('part', 'kc', 'att')] + ([_get(r, b, 'cnt')] if fused else [])
    fwd = [(kh, s) for kh in range(Hkv) for s in range(S)]
    ref = graph(False, fwd)
    for order in (fwd, fwd[::-1], sorted(fwd, key=lambda x: (x[1], -x[0]))):
        got = graph(True, order)
        for g, r in zip(got, ref):
            assert np.array_equal(np.asarray(g).view(np.uint32), np.asarray(r).view(np.uint32))
        assert (got[3] == 0).all()
    assert np.abs(ref[2]).sum() > 0


def test_rope_inverse_and_head_rmsnorm():
    w = W(6)
    R, H, hd = 6, 2, 8
    w.buf('x', R, H * hd), w.zeros('y', R, H * hd), w.zeros('z', R, H * hd), w.buf('g', hd), w.zeros('n', R, H * hd)
    t = w.task('rope_fwd', x='x', out='y', pos=None, r0=0, r1=R, T=R, H=H, hd=hd, theta=1e6)
    w.task('rope_bwd', after=[t], x='y', out='z', pos=None, r0=0, r1=R, T=R, H=H, hd=hd, theta=1e6)
    w.task('head_rmsnorm', x='x', gamma='g', out='n', r0=0, r1=R, H=H, hd=hd, eps=1e-6)
    r, b = _run_one(w)
    x = _get(r, b, 'x').reshape(R, H, hd).astype(np.float64)
    assert np.abs(_get(r, b, 'z').reshape(R, H, hd) - x).max() < 1e-5
    g = _get(r, b, 'g').astype(np.float64)
    want = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * g
    assert np.abs(_get(r, b, 'n').reshape(R, H, hd) - want).max() < 1e-5


def test_gemv_bf16_closed_form():
    """Decode GEMV with the RMSNorm prologue = bf16(rmsnorm(x)) @ W^T in fp64."""
    w = W(7)
    K, N = 64, 24
    w.buf('x', 1, K), w.buf('gm', K), w.buf('w', N, K, 'bf16'), w.zeros('o', 1, N)
    w.task('gemv_bf16', x='x', x2=None, gamma='gm', w='w', out='o', res=None, n0=0, n1=N, K=K, pro=1, eps=1e-6)
    r, b = _run_one(w)
    x, gm = (_get(r, b, n).astype(np.float64) for n in ('x', 'gm'))
    W_ = _get(r, b, 'w').reshape(N, K).astype(np.float64)
    v = bl.bf16_round((x / math.sqrt((x * x).mean() + 1e-6) * gm).astype(np.float32)).astype(np.float64)
    assert np.abs(_get(r, b, 'o') - W_ @ v).max() < 1e-5


@pytest.mark.parametrize('TM', [128, 256])
@pytest.mark.parametrize('flags', [0, 3])
def test_splitk_closed_form(flags, TM):
    """Split-K (ops 302 + 303): the in-order sum of the K-range partials equals the fp64 product of the bf16 operands
    (a wrong k0 / om0 offset, a transposed operand or a dropped range fails this); each partial block equals the
    product over its own K range."""
    w = W(5)
    M, N, K, S = 130, 260, 96, 3
    ta, tb = flags & 1, flags & 2
    w.buf('A', K if ta else M, M if ta else K, 'bf16'), w.buf('B', N if tb else K, K if tb else N, 'bf16')
    w.zeros('P', S * M, N), w.zeros('C', M, N, 'bf16')
    bounds = [0, 32, 64, 96]
    ts = []
    for s in range(S):
        for m0 in range(0, M, TM):
            for n0 in (0, 256):
                ts.append(w.task('matmul_mma_bf16_kr', a='A', b='B', out='P', bias=None, res=None, pre=None, m0=m0, n0=n0, M=M, N=N,
                                 K=bounds[s + 1] - bounds[s], flags=flags | (64 if TM == 256 else 0), alpha=1.0, k0=bounds[s], om0=s * M))
    w.task('splitk_reduce', after=ts, part='P', out='C', M=M, N=N, S=S, r0=0, r1=M)
    r, b = _run_one(w)
    A = _get(r, b, 'A').astype(np.float64).reshape(K if ta else M, M if ta else K)
    B = _get(r, b, 'B').astype(np.float64).reshape(N if tb else K, K if tb else N)
    A = A.T if ta else A
    B = B.T if tb else B
    P = _get(r, b, 'P').reshape(S, M, N)
    for s in range(S):
        k0, k1 = bounds[s], bounds[s + 1]
        want = A[:, k0:k1] @ B[k0:k1, :]
        assert np.abs(P[s] - want).max() < 1e-5 * np.abs(want).max()
    full = A @ B
    got = _get(r, b, 'C').reshape(M, N).astype(np.float64)
    assert np.abs(got - full).max() < 2 ** -7 * np.abs(full).max()
    assert np.array_equal(got, bl.bf16_round((P[0] + P[1] + P[2]).astype(np.float32)).astype(np.float64))


def test_mma_delta_is_tile_then_delta():
    """Op 308 equals op 122 on the tile followed by op 46 over the tile's rows and heads, bit for bit."""
    M, N, K, T, H = 128, 256, 64, 64, 4

    def graph(fused):
        w = W(47)
        w.buf('A', M, K, 'bf16'), w.buf('B', K, N, 'bf16'), w.buf('O', M, N, 'bf16'), w.zeros('C', M, N, 'bf16'), w.zeros('D', (M // T) * H * T)
        kw = dict(a='A', b='B', out='C', bias=None, res=None, pre=None, m0=0, n0=0, M=M, N=N, K=K, flags=0, alpha=1.0)
        if fused:
            w.task('matmul_mma_bf16_delta', o='O', delta='D', T=T, H=H, hd=64, **kw)
        else:
            t = w.task('matmul_mma_bf16', **kw)
            w.task('attn_bwd_delta', after=[t], o='O', do='C', delta='D', r0=0, r1=M, T=T, H=H, hd=64)
        r, b = _run_one(w)
        return _get(r, b, 'C'), _get(r, b, 'D')
    f, u = graph(True), graph(False)
    assert np.array_equal(f[0].view(np.uint32), u[0].view(np.uint32))
    assert np.array_equal(f[1].view(np.uint32), u[1].view(np.uint32))
    assert np.abs(f[1]).max() > 0


def test_layernorm_bwd_dx_res_is_copy_then_accumulate():
    """Op 309 (dx = res + LayerNorm input gradient) equals copying res into dx and running op 37 with acc 1, bitwise."""
    R, d = 6, 64

    def graph(fused):
        w = W(53)
        w.buf('x', R, d), w.buf('dy', R, d), w.buf('g', d), w.buf('mu', R), w.pos('rs', R, 2.0), w.buf('res', R, d), w.zeros('dx', R, d)
        if fused:
            w.task('layernorm_bwd_dx_res', x='x', dy='dy', gamma='g', mean='mu', rstd='rs', dx='dx', res='res', r0=0, r1=R, d=d)
        else:
            t = w.task('copy', src='res', dst='dx', n=R * d)
            w.task('layernorm_bwd_dx', after=[t], x='x', dy='dy', gamma='g', mean='mu', rstd='rs', dx='dx', r0=0, r1=R, d=d, acc=1)
        r, b = _run_one(w)
        return _get(r, b, 'dx')
    f, u = graph(True), graph(False)
    assert np.array_equal(f.view(np.uint32), u.view(np.uint32)) and np.abs(f).max() > 0


@pytest.mark.parametrize('flags', [0, 1, 2, 3, 4, 8, 512])
def test_mma_256_is_two_128x256_tiles(flags):
    """Op 304 (256x256 tile) equals op 122 (golden-pinned 128x256 tile) at (m0, n0) and (m0 + 128, n0), bit for bit,
    for every operand orientation and epilogue (bias, pre-activation store, GELU, residual, accumulate, GELU'),
    including ragged edge tiles; and the plain product equals the fp64 product of the bf16-rounded operands."""
    M, N, K = 300, 290, 48
    ta, tb = flags & 1, flags & 2

    def graph(fused):
        w = W(61)
        w.buf('A', K if ta else M, M if ta else K), w.buf('B', N if tb else K, K if tb else N)
        w.buf('bias', 1, N), w.buf('res', M, N), w.buf('pre', M, N), w.buf('out', M, N)
        ep = dict(bias=None, res=None, pre=None)
        if flags & 512:
            ep['pre'] = 'pre'
        elif flags in (0, 8):
            ep = dict(bias='bias', res='res', pre='pre')
        kw = dict(a='A', b='B', out='out', M=M, N=N, K=K, flags=flags, alpha=0.75, **ep)
        for m0 in (0, 256):
            for n0 in (0, 256):
                if fused:
                    w.task('matmul_mma_bf16_256', m0=m0, n0=n0, **kw)
                else:
                    for dm in (0, 128):
                        if m0 + dm < M:
                            w.task('matmul_mma_bf16', m0=m0 + dm, n0=n0, **kw)
        r, b = _run_one(w)
        return r, b
    (rf, bf), (ru, bu) = graph(True), graph(False)
    for nm in ('out', 'pre'):
        f, u = _get(rf, bf, nm), _get(ru, bu, nm)
        assert np.array_equal(f.view(np.uint32), u.view(np.uint32)), nm
    if flags in (0, 1, 2, 3):
        A = bl.bf16_round(_get(rf, bf, 'A')).astype(np.float64).reshape(K if ta else M, M if ta else K)
        B = bl.bf16_round(_get(rf, bf, 'B')).astype(np.float64).reshape(N if tb else K, K if tb else N)
        want = 0.75 * ((A.T if ta else A) @ (B.T if tb else B))
        if flags == 0:
            want = want + _get(rf, bf, 'bias').astype(np.float64) + _get(rf, bf, 'res').astype(np.float64).reshape(M, N)
        got = _get(rf, bf, 'out').reshape(M, N)
        assert np.abs(got - want).max() < 1e-5 * np.abs(want).max()


@pytest.mark.parametrize('pro', [0, 1, 2])
@pytest.mark.parametrize('with_res', [False, True])
def test_gemv_rows_is_gemv_per_row(pro, with_res):
    """Op 301 over M rows equals op 134 (golden-pinned decode GEMV) run on each row alone, bit for bit, for the three
    prologues (none, RMSNorm, SwiGLU) with and without the residual; a row mix-up or a shared statistic fails this."""
    M, K, N = 5, 128, 40
    rng = np.random.default_rng(3 + pro)
    X, X2, R = (rng.standard_normal((M, n)).astype(np.float32) for n in (K, K, N))
    g = rng.standard_normal(K).astype(np.float32)
    Wt = bl.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.1)
    vals = lambda a: {'kind': 'values', 'values': a.ravel().tolist()}
    w = W(71)
    w.buf('W', N, K, 'bf16', vals(Wt)), w.buf('g', K, 1, 'f32', vals(g))
    w.buf('X', M, K, 'f32', vals(X)), w.buf('X2', M, K, 'f32', vals(X2)), w.buf('R', M, N, 'f32', vals(R)), w.zeros('O', M, N)
    opt = dict(x2='X2' if pro == 2 else None, gamma='g' if pro == 1 else None)
    w.task('gemv_bf16_rows', x='X', w='W', out='O', res='R' if with_res else None, n0=3, n1=N, K=K, M=M, pro=pro, eps=1e-6, **opt)
    for m in range(M):
        w.buf(f'x{m}', 1, K, 'f32', vals(X[m])), w.buf(f'y{m}', 1, K, 'f32', vals(X2[m])), w.buf(f'r{m}', 1, N, 'f32', vals(R[m]))
        w.zeros(f'o{m}', 1, N)
        w.task('gemv_bf16', x=f'x{m}', x2=f'y{m}' if pro == 2 else None, gamma='g' if pro == 1 else None, w='W', out=f'o{m}',
               res=f'r{m}' if with_res else None, n0=3, n1=N, K=K, pro=pro, eps=1e-6)
    r, b = _run_one(w)
    O = _get(r, b, 'O').reshape(M, N)
    assert np.abs(O[:, 3:]).max() > 0 and not O[:, :3].any()
    for m in range(M):
        assert np.array_equal(O[m].view(np.uint32), _get(r, b, f'o{m}').view(np.uint32)), m
    assert not np.array_equal(O[0], O[1])


@pytest.mark.parametrize('case', golden_cases())
def test_threaded_oracle_matches_reference_vm_bitwise(case):
    """The N-thread oracle (ready tasks in parallel) gives the reference VM's final buffers and versions bit for bit."""
    d = GOLDEN / case
    g = json.loads((d / 'golden.json').read_text())
    r = oracle.run(d, threads=4)
    meta = json.loads((d / 'metadata.json').read_text())
    for m, x in zip(meta['buffers'], r['buffers']):
        want = np.array(g['buffers'][m['name']], np.int32 if m['dtype'] == 1 else np.float32)
        assert np.array_equal(want.view(np.uint32), x.view(np.uint32)), m['name']
    assert r['versions'] == g['versions']
    assert sorted(r['order'].tolist()) == list(range(len(r['order'])))


def test_threaded_oracle_matches_one_thread_on_generated_graphs():
    """Tiny GPT (2 steps) and the 8-MLP graph (1 step): 8 threads give the 1-thread buffers bit for bit."""
    from kvm_amd.workloads import gpt, mlp
    for w in (gpt.build(gpt.GPTConfig.tiny(steps=2)), mlp.build(mlp.MLPConfig(steps=1, widths=(64, 96, 128)))):
        b = bl.load(compiler.compile_spec(w.spec))
        init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in b.metadata['buffers']]
        r1 = oracle.run(b, [x.copy() for x in init])
        r8 = oracle.run(b, [x.copy() for x in init], threads=8)
        for m, x, y in zip(b.metadata['buffers'], r1['buffers'], r8['buffers']):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), m['name']


def test_decode_reference_deviation_from_fp64_fixture():
    """The oracle on the full-width one-layer Qwen3 decode graph (batch 1) against an independent fp64 numpy model of
    the same step: the same greedy token, a deviation below 1e-2 (bf16 activation stores and f32 RoPE angles are the
    reference's rounding points), and the committed deviation fixture the GPU decode tolerances are derived from."""
    import decode_fp64  # noqa: F401
    from golden.make_decode_deviation import deviation
    fix = json.loads((REPO / 'tests/golden/data/decode_fp64_deviation.json').read_text())['b1']
    got = deviation(1)
    assert got['tok'] == got['tok_fp64'] == fix['tok']
    for k, v in got['deviation'].items():
        assert 0 < v < 1e-2 and abs(v - fix['deviation'][k]) <= 1e-3 * v, (k, v, fix['deviation'][k])


def test_gpt_fp64_model_matches_the_f32_oracle():
    """tests/gpt_fp64.py (the fp64 model the full-depth GPT tolerances are measured with) computes the graph's step:
    on an f32 GPT graph (2 layers, d 128, 4 heads, T 64, vocab 256, batch 8) the oracle's loss, logits, gradients and
    AdamW-updated parameters agree with it to f32 rounding (relative L2 below 2e-5 everywhere)."""
    import gpt_fp64 as G
    from kvm_amd.workloads import gpt
    c = gpt.GPTConfig(layers=2, d=128, heads=4, T=64, vocab=256, ffn=512, batch=8, dtype='f32')
    w = gpt.build(c)
    lb = bl.load(compiler.compile_spec(w.spec))
    names = [m['name'] for m in lb.metadata['buffers']]
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    ref = G.step(c, {n: x.copy() for n, x in zip(names, init)})
    r = oracle.run(lb, init, threads=4)
    dev = G.deviations(names, r['buffers'], ref)
    assert dev.pop('loss_abs') < 1e-5
    assert max(dev.values()) < 2e-5, sorted(dev.items(), key=lambda kv: -kv[1])[:3]


@pytest.mark.parametrize('M', [1, 3])
def test_gemv_swiglu_is_gate_up_gemvs_then_silu_mul(M):
    """Op 311 equals op 301 with the RMSNorm prologue on the gate rows and on the up rows (f32 outputs), followed by
    op 98 (silu_mul_fwd, the reference's SwiGLU) into a bf16 buffer, bit for bit; a swapped gate / up or a missing
    prologue fails this (silu is not symmetric in its factors)."""
    K, N = 256, 48
    rng = np.random.default_rng(11 + M)
    X = rng.standard_normal((M, K)).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    Wg, Wu = (bl.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.1) for _ in range(2))
    vals = lambda a: {'kind': 'values', 'values': a.ravel().tolist()}
    w = W(72)
    w.buf('Wg', N, K, 'bf16', vals(Wg)), w.buf('Wu', N, K, 'bf16', vals(Wu)), w.buf('g', K, 1, 'f32', vals(g))
    w.buf('X', M, K, 'f32', vals(X)), w.buf('H', M, N, 'bf16', {'kind': 'fill', 'value': 0})
    w.task('gemv_swiglu', x='X', gamma='g', wg='Wg', wu='Wu', out='H', n0=16, n1=N, K=K, M=M, eps=1e-6)
    w.zeros('G', M, N), w.zeros('U', M, N), w.buf('H2', M, N, 'bf16', {'kind': 'fill', 'value': 0})
    tg = w.task('gemv_bf16_rows', x='X', x2=None, res=None, gamma='g', w='Wg', out='G', n0=16, n1=N, K=K, M=M, pro=1, eps=1e-6)
    tu = w.task('gemv_bf16_rows', x='X', x2=None, res=None, gamma='g', w='Wu', out='U', n0=16, n1=N, K=K, M=M, pro=1, eps=1e-6)
    w.task('silu_mul_fwd', after=[tg, tu], gate='G', up='U', out='H2', e0=0, e1=M * N)
    r, b = _run_one(w)
    H, H2 = _get(r, b, 'H').reshape(M, N), _get(r, b, 'H2').reshape(M, N)
    assert np.abs(H[:, 16:]).max() > 0 and not H[:, :16].any()
    assert np.array_equal(H[:, 16:].view(np.uint32), H2[:, 16:].view(np.uint32))
    G, U = _get(r, b, 'G').reshape(M, N), _get(r, b, 'U').reshape(M, N)
    swapped = bl.bf16_round((U / (1.0 + np.exp(-U.astype(np.float64))) * G).astype(np.float32))
    assert not np.array_equal(H[:, 16:], swapped[:, 16:])
