"""GPU parity of the bf16 GEMM tile operators (matmul_mma_bf16, op 122; matmul_tile_bf16, op 114) against the CPU oracle.

Shapes are chosen so that both device paths run: whole tiles with K a multiple of 32 take the direct-to-LDS pipeline,
partial tiles / odd K / f32 operands take the register-staged path. All four operand orientations (flags 1 and 2) and
every epilogue (bias, GELU with pre-activation store, dGELU, residual, accumulate, alpha) are covered. The oracle
rounds operands to bf16 and sums exact products in double (reference: runtime/ref_extra.py:312-331); the device sums
in fp32 on MFMA, so outputs are held to a relative L2 error of 2e-5 (f32 outputs) or 4e-3 (bf16 outputs: one bf16
ulp is 2^-8 relative).
"""
import numpy as np
import pytest

import oracle
from gpu_check import compare_run
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.executor import PATH_DYNAMIC, PATH_STATIC, Executor
from kvm_amd.workloads import Builder, Workload

pytestmark = pytest.mark.gpu


def _gemm_graph(M, N, K, flags, op='matmul_mma_bf16', adt='bf16', bdt='bf16', odt='bf16', bias=False, res=False, pre=False,
                alpha=1.0, tiles=(128, 256)):
    b = Builder(7)
    ta, tb = flags & 1, flags & 2
    b.normal('A', K if ta else M, M if ta else K, adt, scale=1.0)
    b.normal('B', N if tb else K, K if tb else N, bdt, scale=1.0)
    b.normal('C', M, N, odt, scale=1.0)           # nonzero start: flag 4 accumulates into it
    if bias:
        b.normal('bias', 1, N, 'f32', scale=1.0)
    if res:
        b.normal('R', M, N, odt, scale=1.0)
    if pre:
        b.normal('P', M, N, odt, scale=1.0)
    TM, TN = tiles
    for m0 in range(0, M, TM):
        for n0 in range(0, N, TN):
            b.task(op, a='A', b='B', out='C', bias='bias' if bias else None, res='R' if res else None, pre='P' if pre else None,
                   m0=m0, n0=n0, M=M, N=N, K=K, flags=flags, alpha=alpha)
    return Workload(b.spec(), b.init_override)


def _check(w, tol_f32=2e-5, tol_bf16=4e-3):
    """Each graph on both device paths: the dynamic kernel runs the 128x256 and 128x128 whole tiles inlined, the static
    kernel calls the operator bodies; both against the same oracle run."""
    lb = bl.load(compiler.compile_spec(w.spec))
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    ref = oracle.run(lb, [x.copy() for x in init])
    for path in (PATH_DYNAMIC, PATH_STATIC):
        ex = Executor.from_bundle(lb, buffers=[x.copy() for x in init], path=path)
        ex.run()
        assert ex.path() == path
        bad = compare_run(ex, lb.metadata, ref, tol_f32=tol_f32, tol_bf16=tol_bf16)
        ex.close()
        assert not bad, (path, bad)


@pytest.mark.parametrize('flags', [0, 1, 2, 3])
def test_mma_whole_tiles_all_orientations(flags):
    print(f'mma whole tiles flags {flags}', flush=True)
    _check(_gemm_graph(256, 512, 192, flags))


@pytest.mark.parametrize('flags', [0, 3])
def test_mma_f32_output_k4096(flags):
    print(f'mma f32 out K=4096 flags {flags}', flush=True)
    _check(_gemm_graph(128, 256, 4096, flags, odt='f32'))


@pytest.mark.parametrize('flags,kw', [
    (2, dict(bias=True)),
    (2 | 8, dict(bias=True, pre=True)),           # GELU epilogue, pre-activation stored
    (512, dict(pre=True)),                        # dGELU epilogue
    (2, dict(bias=True, res=True)),
    (4, dict()),                                  # accumulate into out
    (1, dict(alpha=0.5, odt='f32')),
])
def test_mma_epilogues(flags, kw):
    print(f'mma epilogue flags {flags} {kw}', flush=True)
    _check(_gemm_graph(256, 256, 128, flags, **kw))


@pytest.mark.parametrize('flags', [0, 1, 2, 3])
def test_mma_edge_tiles(flags):
    """Partial tiles in M and N, K not a multiple of the slab: the register-staged path."""
    print(f'mma edge tiles flags {flags}', flush=True)
    _check(_gemm_graph(200, 300, 100, flags, bias=True))


def test_mma_f32_operands():
    print('mma f32 operands', flush=True)
    _check(_gemm_graph(128, 256, 64, 2, adt='f32', bdt='f32', odt='f32'))


@pytest.mark.parametrize('tiles,fl', [((64, 64), 0), ((128, 128), 32), ((256, 128), 64)])
def test_tile_bf16_sizes(tiles, fl):
    print(f'tile_bf16 {tiles}', flush=True)
    _check(_gemm_graph(256, 256, 96, fl | 2, op='matmul_tile_bf16', tiles=tiles, bias=True))
    _check(_gemm_graph(256, 256, 128, fl | 1, op='matmul_tile_bf16', tiles=tiles))


def _splitk_graph(M, N, K, flags, S, odt='bf16', TM=128):
    """Split-K as the GPT generator emits it: op 302 tiles (TM 256: flag 64, 256x256 tiles) over S K ranges into an
    f32 partial buffer of S row blocks, then op 303 sums the blocks in order into C."""
    b = Builder(11)
    ta, tb = flags & 1, flags & 2
    b.normal('A', K if ta else M, M if ta else K, 'bf16', scale=1.0)
    b.normal('B', N if tb else K, K if tb else N, 'bf16', scale=1.0)
    b.fill('P', S * M, N, 'f32')
    b.fill('C', M, N, odt)
    slabs = K // 32
    bounds = [32 * (slabs * s // S) for s in range(S + 1)]
    ts = []
    for s in range(S):
        for m0 in range(0, M, TM):
            for n0 in range(0, N, 256):
                ts.append(b.task('matmul_mma_bf16_kr', a='A', b='B', out='P', bias=None, res=None, pre=None, m0=m0, n0=n0, M=M, N=N,
                                 K=bounds[s + 1] - bounds[s], flags=flags | (64 if TM == 256 else 0), alpha=1.0, k0=bounds[s], om0=s * M))
    for r0 in range(0, M, 64):
        b.task('splitk_reduce', after=ts, part='P', out='C', M=M, N=N, S=S, r0=r0, r1=min(M, r0 + 64))
    return Workload(b.spec(), b.init_override)


@pytest.mark.parametrize('TM', [128, 256])
@pytest.mark.parametrize('flags', [0, 1, 2, 3])
def test_splitk_all_orientations(flags, TM):
    print(f'split-K flags {flags} TM {TM}', flush=True)
    _check(_splitk_graph(512, 512, 416, flags, S=3, TM=TM))


def test_splitk_256_partial_tiles():
    """256-row split-K tiles where the shape leaves partial tiles (the two-128-row fallback inside the tile)."""
    print('split-K 256 partial tiles', flush=True)
    _check(_splitk_graph(300, 300, 640, 0, S=2, odt='f32', TM=256))


def test_splitk_partial_tiles_f32_out():
    print('split-K partial tiles, f32 out', flush=True)
    _check(_splitk_graph(200, 300, 640, 0, S=4, odt='f32'))


@pytest.mark.parametrize('flags', [0, 1, 2, 3])
def test_mma256_whole_tiles_all_orientations(flags):
    """matmul_mma_bf16_256 (op 304): 256x256 tiles, two-half epilogue."""
    print(f'mma256 whole tiles flags {flags}', flush=True)
    _check(_gemm_graph(512, 512, 192, flags, op='matmul_mma_bf16_256', tiles=(256, 256)))


@pytest.mark.parametrize('flags,kw', [
    (2 | 8, dict(bias=True, pre=True)),
    (512, dict(pre=True)),
    (2, dict(bias=True, res=True)),
    (4, dict(odt='f32')),
])
def test_mma256_epilogues(flags, kw):
    print(f'mma256 epilogue flags {flags} {kw}', flush=True)
    _check(_gemm_graph(256, 512, 128, flags, op='matmul_mma_bf16_256', tiles=(256, 256), **kw))


def test_mma256_partial_tiles():
    """Partial tiles and K off the slab: two 128x256 register-path tiles."""
    print('mma256 partial tiles', flush=True)
    _check(_gemm_graph(300, 400, 100, 1, op='matmul_mma_bf16_256', tiles=(256, 256), bias=True))


@pytest.mark.parametrize('flags', [0, 2])
def test_mma_delta_tiles(flags):
    """Op 308: op 122's 128x256 tiles (plain epilogue) that also write the attention-backward statistic
    delta = rowsum(o * out) of each 64-column head, two sequences of T = 256 rows."""
    print(f'mma delta flags {flags}', flush=True)
    M, N, K, T, H = 512, 512, 192, 256, 8
    b = Builder(9)
    b.normal('A', M, K, 'bf16', scale=1.0)
    b.normal('B', N if flags & 2 else K, K if flags & 2 else N, 'bf16', scale=1.0)
    b.normal('O', M, N, 'bf16', scale=1.0)
    b.fill('C', M, N, 'bf16')
    b.fill('D', (M // T) * H * T)
    for m0 in range(0, M, 128):
        for n0 in range(0, N, 256):
            b.task('matmul_mma_bf16_delta', a='A', b='B', out='C', bias=None, res=None, pre=None, m0=m0, n0=n0, M=M, N=N, K=K,
                   flags=flags, alpha=0.5, o='O', delta='D', T=T, H=H, hd=64)
    _check(Workload(b.spec(), b.init_override))


@pytest.mark.parametrize('flags,tiles', [(0, (64, 64)), (32 | 2, (128, 128)), (64 | 1, (256, 128))])
def test_f32_whole_tiles_both_paths(flags, tiles):
    """matmul_tile (op 34) on fp32 operands, whole tiles of each size (flag 32: 128x128, flag 64: 256x128), with bias:
    the direct-to-LDS fp32 form, inlined into the static kernel at 64x64 / 128x128 and called from the dynamic one."""
    print(f'f32 whole tiles flags {flags}', flush=True)
    _check(_gemm_graph(256, 256, 128, flags, op='matmul_tile', adt='f32', bdt='f32', odt='f32', tiles=tiles, bias=True))
