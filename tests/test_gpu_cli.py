"""The kvm_exec CLI (counterpart of the reference's mvm_exec, mvm_exec.cu:1962-2315) run as a harness runs it: result
line, exit codes, --golden, --dump-buffers, --dump-bin, device errors and refused metadata."""
import json
import re
import subprocess

import numpy as np
import pytest

import oracle
from conftest import GOLDEN, REPO, golden_cases
from kvm_amd import bundle as bl
from kvm_amd import compiler
from cases import W

CLI = REPO / 'kvm_amd' / '_build' / 'kvm_exec'
LINE = re.compile(r'^(OK|FAIL): (\d+)/(\d+) tasks, [0-9.]+ ms \((static|dynamic) path\)(, golden (match|MISMATCH))?$')


def _run(*args, timeout=120):
    r = subprocess.run([str(CLI), *map(str, args)], capture_output=True, text=True, timeout=timeout)
    return r.returncode, r.stdout, r.stderr


def test_usage_and_check_ops_need_no_gpu():
    rc, out, err = _run()
    assert rc == 2 and 'usage' in err
    rc, out, err = _run('--bogus', 'x')
    assert rc == 2
    rc, out, err = _run('--check-ops')
    assert rc == 0
    ops = dict(line.split() [::-1] for line in out.strip().split('\n'))
    assert ops['matmul_tile'] == '34' and ops['gemv_bf16_rows'] == '301'


@pytest.mark.gpu
@pytest.mark.parametrize('path', ['auto', 'dynamic', 'static'])
@pytest.mark.parametrize('case', golden_cases())
def test_golden_bundle_through_the_cli(case, path):
    """Every golden bundle on each scheduler path. The static path is refused only for a graph whose version waits
    it cannot plan (exit 1 with the reason); auto then falls back to the dynamic path."""
    print(f'cli golden {case} --path {path}', flush=True)
    n = json.loads((GOLDEN / case / 'metadata.json').read_text())['task_count']
    rc, out, err = _run('--golden', '--golden-tol', '2e-5', '--path', path, GOLDEN / case)
    if path == 'static' and rc == 1 and 'static' in err:
        pytest.skip(f'static path refused: {err.strip()}')
    m = LINE.match(out.strip().split('\n')[-1])
    assert rc == 0 and m, (rc, out, err)
    assert m.group(1) == 'OK' and int(m.group(2)) == int(m.group(3)) == n and m.group(6) == 'match'
    if path != 'auto':
        assert m.group(4) == path


@pytest.mark.gpu
def test_dump_buffers_and_dump_bin_match_the_oracle(tmp_path):
    print('cli dump', flush=True)
    d = GOLDEN / 'gpt_ops'
    meta = json.loads((d / 'metadata.json').read_text())
    ref = oracle.run(d)
    rc, out, err = _run('--dump-buffers', '--dump-bin', tmp_path, '0,1', d)
    assert rc == 0, err
    lines = [ln for ln in out.split('\n') if ln.startswith('buffer ')]
    assert len(lines) == len(meta['buffers'])
    for ln, m, want in zip(lines, meta['buffers'], ref['buffers']):
        idx, vals = ln.split(':', 1)
        got = np.array(vals.split(), np.float64).astype(np.float32)
        want = want.view(np.float32) if m['dtype'] == bl.DT_I32 else want   # i32 bits printed as floats (reference format)
        assert got.size == want.size, m['name']
        if m['dtype'] == bl.DT_I32:   # bit patterns printed as floats: exact, except that NaN patterns (e.g. -1) print as nan
            nan = np.isnan(want)
            assert np.array_equal(np.isnan(got), nan) and np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), m['name']
        else:
            assert np.linalg.norm(got - want) <= 2e-5 * max(np.linalg.norm(want), 1e-30) + 1e-30, m['name']
    for i in (0, 1):
        b = np.fromfile(tmp_path / f'{i}.bin', np.float32)
        w = ref['buffers'][i].view(np.float32)
        assert b.size == w.size and np.linalg.norm(b - w) <= 2e-5 * max(np.linalg.norm(w), 1e-30)


def _write(w, path):
    compiler.compile_spec(w.spec()).write(path)
    return path


@pytest.mark.gpu
def test_device_error_exits_1(tmp_path):
    print('cli device error', flush=True)
    w = W(1)
    w.ints('ids', [1, 2, 99, 3]), w.buf('wte', 16, 8), w.zeros('out', 4, 8)
    w.task('embedding_fwd', ids='ids', wte='wte', wpe=None, out='out', r0=0, r1=4, T=4, d=8)
    rc, out, err = _run(_write(w, tmp_path / 'b'))
    assert rc == 1 and out.startswith('FAIL: ') and 'device error 1005' in err


@pytest.mark.gpu
def test_short_values_array_is_refused(tmp_path):
    print('cli init size', flush=True)
    w = W(1)
    w.buf('x', 2, 4, 'f32', {'kind': 'values', 'values': [1.0] * 8}), w.zeros('o', 2, 4)
    w.task('relu', x='x', out='o', n=8)
    d = _write(w, tmp_path / 'b')
    meta = json.loads((d / 'metadata.json').read_text())
    meta['buffers'][0]['init']['values'] = meta['buffers'][0]['init']['values'][:5]
    (d / 'metadata.json').write_text(json.dumps(meta))
    rc, out, err = _run(d)
    assert rc == 1 and 'buffer init size 5 != 8' in err
