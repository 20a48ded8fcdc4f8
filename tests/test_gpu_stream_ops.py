"""GPU parity of the streaming forms of the bandwidth-bound operators (row norms, column reductions, softmax cross
entropy, bf16 conversion, gradient norm, attention delta) at the widths of the GPT-162M workload (d = 768, 4096
rows), in bf16 and f32 storage, against the CPU oracle. The oracle sums in double; the device sums in fp32 in a fixed
tree order: f32 outputs within a relative L2 error of 2e-5, bf16 outputs 4e-3 (one bf16 ulp is 2^-8)."""
import numpy as np
import pytest

import oracle
from gpu_check import compare_run
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.executor import Executor
from kvm_amd.workloads import Builder, Workload, split

pytestmark = pytest.mark.gpu


def _run(b):
    w = Workload(b.spec(), b.init_override)
    lb = bl.load(compiler.compile_spec(w.spec))
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    ref = oracle.run(lb, [x.copy() for x in init])
    ex = Executor.from_bundle(lb, buffers=init)
    ex.run()
    bad = compare_run(ex, lb.metadata, ref)
    ex.close()
    assert not bad, bad


@pytest.mark.parametrize('dt', ['bf16', 'f32'])
def test_norms_and_column_sums(dt):
    print(f'norms {dt}', flush=True)
    N, d = 1024, 768
    b = Builder(3)
    for nm in ('x', 'dy'):
        b.normal(nm, N, d, dt, scale=1.0)
    b.normal('g', 1, d, 'f32', scale=1.0)
    b.normal('be', 1, d, 'f32', scale=1.0)
    b.normal('dx', N, d, dt, scale=1.0)
    b.fill('h', N, d, dt)
    b.fill('hr', N, d, dt)
    for nm in ('mu', 'rs', 'rsr'):
        b.fill(nm, N)
    for nm in ('dg', 'db', 'cs'):
        b.fill(nm, 1, d)
    ts = []
    for r0, r1 in split(N, 64):
        ts.append(b.task('layernorm_fwd', x='x', gamma='g', beta='be', out='h', mean='mu', rstd='rs', r0=r0, r1=r1, d=d, eps=1e-5))
        ts.append(b.task('rmsnorm_fwd', x='x', gamma='g', out='hr', rstd='rsr', r0=r0, r1=r1, d=d, eps=1e-6))
    for r0, r1 in split(N, 64):
        b.task('layernorm_bwd_dx', after=ts, x='x', dy='dy', gamma='g', mean='mu', rstd='rs', dx='dx', r0=r0, r1=r1, d=d, acc=1)
    for c0, c1 in split(d, 12):
        b.task('norm_bwd_params', after=ts, x='x', dy='dy', mean='mu', rstd='rs', dgamma='dg', dbeta='db', R=N, d=d, c0=c0, c1=c1, acc=0)
        b.task('colsum', x='dy', out='cs', R=N, c0=c0, c1=c1, acc=0)
    _run(b)


def test_rmsnorm_bwd_and_wide_rows():
    print('rmsnorm bwd d=4096', flush=True)
    N, d = 128, 4096
    b = Builder(5)
    for nm in ('x', 'dy'):
        b.normal(nm, N, d, 'bf16', scale=1.0)
    b.normal('g', 1, d, 'f32', scale=1.0)
    b.fill('h', N, d, 'bf16')
    b.fill('rs', N)
    b.fill('dx', N, d, 'bf16')
    t = [b.task('rmsnorm_fwd', x='x', gamma='g', out='h', rstd='rs', r0=r0, r1=r1, d=d, eps=1e-6) for r0, r1 in split(N, 8)]
    for r0, r1 in split(N, 8):
        b.task('rmsnorm_bwd_dx', after=t, x='x', dy='dy', gamma='g', rstd='rs', dx='dx', r0=r0, r1=r1, d=d, acc=0)
    _run(b)


@pytest.mark.parametrize('dt,N,V,scale', [('bf16', 256, 5000, 1.0), ('f32', 256, 5000, 1.0), ('bf16', 64, 50304, 1.0),
                                           ('bf16', 64, 5000, -0.5), ('bf16', 64, 5000, 0.0)])
def test_cross_entropy(dt, N, V, scale):
    """Fused softmax cross entropy: ignored rows (every 17th target is -1), GPT's vocabulary width (the row parked in
    LDS), and scales other than positive (the gradient formula's other form)."""
    print(f'cross entropy {dt} N{N} V{V} scale {scale}', flush=True)
    b = Builder(9)
    b.normal('lg', N, V, dt, scale=3.0)
    b.values('tgt', [(37 * i + 11) % V if i % 17 else -1 for i in range(N)], N, 1, 'i32')
    b.fill('rl', N)
    b.fill('ls', N)
    b.fill('dl', N, V, dt)
    b.fill('loss', 2)
    ts = [b.task('softmax_ce_fused', logits='lg', tgt='tgt', rowloss='rl', lse='ls', dlogits='dl', r0=r0, r1=r1, V=V, ignore=-1, N=N, scale=scale)
          for r0, r1 in split(N, 16)]
    b.task('softmax_ce_reduce', after=ts, rowloss='rl', tgt='tgt', loss='loss', N=N, ignore=-1)
    _run(b)


def test_flat_streams():
    print('round_bf16 / gradnorm / delta', flush=True)
    b = Builder(13)
    n = 100003
    b.normal('f', 1, n, 'f32', scale=1.0)
    b.normal('hb', 1, n, 'bf16', scale=1.0)
    b.fill('f2b', 1, n, 'bf16')
    b.fill('b2b', 1, n, 'bf16')
    b.fill('b2f', 1, n, 'f32')
    b.fill('gn', 8)
    for e0, e1 in ((3, 50001), (50001, n)):
        b.task('round_bf16', x='f', out='f2b', e0=e0, e1=e1)
        b.task('round_bf16', x='hb', out='b2b', e0=e0, e1=e1)
        b.task('round_bf16', x='hb', out='b2f', e0=e0, e1=e1)
    for i, (e0, e1) in enumerate(split(n, 8)):
        b.task('gradnorm_partial', g='f', partial='gn', slot=i, e0=e0, e1=e1)
    N, H, hd, T = 256, 12, 64, 128
    b.normal('o', N, H * hd, 'bf16', scale=1.0)
    b.normal('do', N, H * hd, 'bf16', scale=1.0)
    b.fill('delta', N * H)
    for r0, r1 in split(N, 16):
        b.task('attn_bwd_delta', o='o', do='do', delta='delta', r0=r0, r1=r1, T=T, H=H, hd=hd)
    _run(b)


def test_bf16_rounding_special_values():
    """f32 -> bf16 storage rounding on the device (hardware conversion) against round-to-nearest-even on the bits:
    ties in both directions, carries into the exponent, the largest finite values (rounding to infinity), denormals,
    signed zeros and infinities must match bit for bit; NaNs must stay NaN."""
    print('bf16 rounding special values', flush=True)
    rng = np.random.default_rng(5)
    pats = [0x00000000, 0x80000000, 0x7f800000, 0xff800000, 0x7f7fffff, 0xff7fffff, 0x7f7f8000, 0x3f808000, 0x3f818000,
            0x3f80ffff, 0x3fffffff, 0x00000001, 0x00008000, 0x00018000, 0x007fffff, 0x80000001, 0x807fffff, 0x00800000,
            0x7fc00000, 0x7f800001, 0xffc12345]
    pats += [int(x) for x in rng.integers(0, 2 ** 32, 4000, dtype=np.uint64)]
    pats += [int(x) & 0xffff8000 | 0x8000 for x in rng.integers(0, 2 ** 32, 2000, dtype=np.uint64)]   # exact ties
    n = len(pats)
    b = Builder(3)
    b.fill('x', 1, n, 'f32')                      # overwritten with the raw bit patterns below
    b.fill('y', 1, n, 'bf16')
    b.task('round_bf16', x='x', out='y', e0=0, e1=n)
    w = Workload(b.spec(), b.init_override)
    lb = bl.load(compiler.compile_spec(w.spec))
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    ex = Executor.from_bundle(lb, buffers=init)
    ex.write('x', np.array(pats, dtype=np.uint32).view(np.float32))
    ex.run()
    got = ex.read_raw('y').reshape(-1).astype(np.uint32)
    ex.close()
    u = np.array(pats, dtype=np.uint64)
    want = ((u + 0x7fff + ((u >> 16) & 1)) >> 16).astype(np.uint32) & 0xffff
    nan = ((u & 0x7fffffff) > 0x7f800000)
    assert np.array_equal(got[~nan], want[~nan]), np.nonzero(got[~nan] != want[~nan])
    assert np.all(((got[nan] & 0x7fff) > 0x7f80))


@pytest.mark.parametrize('acc', [0, 1])
def test_embedding_bwd_ids(acc):
    """Token-embedding backward with ids: repeated keys, several key ranges per table, N over one 4096-row batch of
    the id scan, accumulate or overwrite; the rows of a key are added in ascending order as in the oracle."""
    print(f'embedding_bwd acc {acc}', flush=True)
    rng = np.random.default_rng(9)
    N, V, d = 5000, 700, 192
    b = Builder(21)
    b.values('ids', [int(x) for x in rng.integers(0, V, N)] , N, 1, 'i32')
    b.normal('dout', N, d, 'f32', scale=1.0)
    b.normal('dtab', V, d, 'f32', scale=1.0)
    for v0, v1 in split(V, 7):
        b.task('embedding_bwd', ids='ids', dout='dout', dtab='dtab', N=N, mod=0, v0=v0, v1=v1, d=d, acc=acc)
    _run(b)


@pytest.mark.parametrize('sh_dt', ['bf16', 'f32'])
def test_adamw_bf16_shadow(sh_dt):
    """Op 305: AdamW plus the rounded copy of the new weight, over unaligned ranges (scalar heads/tails), a range
    shorter than one 16-byte group and the two-groups-per-pass main loop."""
    print(f'adamw_bf16 sh={sh_dt}', flush=True)
    b = Builder(29)
    n = 300007
    for nm in ('p', 'g', 'm'):
        b.normal(nm, 1, n, 'f32', scale=1.0)
    b.normal('v', 1, n, 'f32', scale=0.01)
    b.values('step', [3], 1, 1, 'i32')
    b.fill('gs', 1, value=0.75)
    b.fill('sh', 1, n, sh_dt)
    for e0, e1 in ((1, 3), (3, 150001), (150001, 150003), (150003, n)):
        b.task('adamw_bf16', p='p', g='g', m='m', v='v', gscale='gs', step='step', e0=e0, e1=e1, lr=3e-4, b1=0.9, b2=0.95,
               eps=1e-8, wd=0.1, sh='sh')
    _run(b)


@pytest.mark.parametrize('tdt,odt,d,pos', [('f32', 'bf16', 768, True), ('f32', 'bf16', 256, False), ('f32', 'f32', 1024, True),
                                            ('f32', 'f32', 4096, False), ('f32', 'bf16', 4104, True)])
def test_embedding_fwd_rows(tdt, odt, d, pos):
    """Op 32 (streaming form): token rows of wte (+ the position row), ragged row ranges, one and two vectors per lane, and rows wider than 2048 (flat form)."""
    print(f'embedding_fwd table {tdt} out {odt} d {d} pos {pos}', flush=True)
    b = Builder(43)
    V, T, N = 997, 64, 203
    b.values('ids', [(37 * i + 11) % V for i in range(N)], N, 1, 'i32')
    b.normal('wte', V, d, tdt, scale=1.0)
    if pos:
        b.normal('wpe', T, d, tdt, scale=1.0)
    b.fill('out', N, d, odt)
    for r0, r1 in ((0, 5), (5, 77), (77, 203)):
        b.task('embedding_fwd', ids='ids', wte='wte', wpe='wpe' if pos else None, out='out', r0=r0, r1=r1, T=T, d=d)
    _run(b)


@pytest.mark.parametrize('dt,d', [('bf16', 768), ('f32', 512)])
def test_layernorm_bwd_dx_res(dt, d):
    """Op 309: dx = res + the LayerNorm input gradient, ragged row ranges."""
    print(f'layernorm_bwd_dx_res {dt} d {d}', flush=True)
    b = Builder(59)
    R = 203
    b.normal('x', R, d, dt, scale=1.0)
    b.normal('dy', R, d, dt, scale=1.0)
    b.normal('res', R, d, dt, scale=1.0)
    b.normal('g', 1, d, 'f32', scale=1.0)
    b.normal('mu', R, 1, 'f32', scale=0.1)
    b.fill('rs', R, 1, 'f32', value=1.3)
    b.fill('dx', R, d, dt)
    for r0, r1 in ((0, 7), (7, 130), (130, R)):
        b.task('layernorm_bwd_dx_res', x='x', dy='dy', gamma='g', mean='mu', rstd='rs', dx='dx', res='res', r0=r0, r1=r1, d=d)
    _run(b)


@pytest.mark.parametrize('acc', [0, 1])
def test_embedding_bwd_id_scan(acc):
    """Table gradient from token ids: ragged N (not a multiple of the 64-id ballot or of the four waves' quarters),
    repeated keys (each row must add its matches in ascending r), ids outside the table, ranges of one row and of
    many; plus the position form (rows key, key + T, ...). Adds are in the reference's order, so f32 within 2e-5."""
    print(f'embedding_bwd acc={acc}', flush=True)
    N, V, d, T = 1001, 300, 96, 77
    rng = np.random.default_rng(11 + acc)
    ids = [int(x) for x in rng.integers(0, V, N)]
    ids[5] = ids[900] = ids[17] = 42                 # one row hit often, from every wave's quarter
    ids[3], ids[600] = -1, V + 5                     # ignored ids
    b = Builder(5)
    b.values('ids', ids, N, 1, 'i32')
    b.normal('dout', N, d, 'f32', scale=1.0)
    b.normal('dtab', V, d, 'f32', scale=1.0)
    b.normal('dpos', T, d, 'f32', scale=1.0)
    for v0, v1 in ((0, 1), (1, 42), (42, 43), (43, 299), (299, 300)):
        b.task('embedding_bwd', ids='ids', dout='dout', dtab='dtab', N=N, mod=0, v0=v0, v1=v1, d=d, acc=acc)
    for v0, v1 in ((0, 3), (3, 77)):
        b.task('embedding_bwd', ids=None, dout='dout', dtab='dpos', N=N, mod=T, v0=v0, v1=v1, d=d, acc=acc)
    _run(b)


def test_argmax_rows():
    """Op 58 over decode-width rows: lowest index among equal maxima, NaN never wins (all-NaN and all -inf rows give 0),
    V below the row width and not a multiple of 4."""
    print('argmax rows', flush=True)
    V, C, R = 151933, 151936, 7
    rng = np.random.default_rng(5)
    lg = rng.standard_normal((R, C)).astype(np.float32)
    lg[0, C - 1] = 100.0                         # beyond V: ignored
    lg[1, [5, 100000, 151932]] = 50.0            # ties: the lowest index wins
    lg[2, :] = np.nan
    lg[3, :] = -np.inf
    lg[4, ::3] = np.nan
    lg[4, 77777] = 9.0
    lg[5, 151930:] = 60.0                        # the maximum in the scalar tail (151932 is V - 1)
    lg[6, :] = 1.0                               # all equal
    want = [None, 5, 0, 0, 77777, 151930, 0]
    for dt in ('f32',):
        b = Builder(44)
        b.fill('lg', R, C, dt)
        b.fill('tok', R, 1, 'i32')
        b.fill('tok2', R, 1, 'i32')
        for r in range(R):
            b.task('argmax', logits='lg', out='tok', r0=r, r1=r + 1, V=V)
        b.task('argmax', logits='lg', out='tok2', r0=0, r1=R, V=V)     # several rows in one task
        w = Workload(b.spec(), b.init_override)
        lb = bl.load(compiler.compile_spec(w.spec))
        init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
        ex = Executor.from_bundle(lb, buffers=init)
        ex.write('lg', lg)
        ex.run()
        got, got2 = ex.read('tok').reshape(-1), ex.read('tok2').reshape(-1)
        ex.close()
        assert (got == got2).all(), (got, got2)
        ref = lg
        for r in range(R):
            row = ref[r, :V]
            exp = want[r] if want[r] is not None else int(np.argmax(np.where(np.isnan(row), -np.inf, row)))
            assert got[r] == exp, (dt, r, got[r], exp)
