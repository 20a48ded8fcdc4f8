"""The manifest runner's host side (kvm_run --check-only; reference: demo/mvm_run.cu): a well-formed demo passes the
checks without a GPU, its serial simulation orders train / serve as their versions require, and malformed manifests
are refused with the reason before any GPU work."""
import json
import subprocess

import numpy as np
import pytest

import manifest_demo
from conftest import REPO
from kvm_amd import manifest as mf

RUNNER = REPO / 'kvm_amd' / '_build' / 'kvm_run'


def _run(*args):
    r = subprocess.run([str(RUNNER), *map(str, args)], capture_output=True, text=True, timeout=120)
    return r.returncode, r.stdout, r.stderr


def test_demo_checks_and_serial_order(tmp_path):
    root = manifest_demo.build(tmp_path / 'demo')
    rc, out, err = _run(root, '--check-only')
    assert rc == 0 and out.startswith('OK'), (out, err)
    assert mf.serial_order(mf.load(root)) == ['train1', 'serve1', 'train2', 'serve2', 'train3', 'serve3']


def test_replay_is_the_closed_form(tmp_path):
    """The CPU replay: W_k = W_{k-1} - 0.1 G (f32), Y_k = X W_k."""
    root = manifest_demo.build(tmp_path / 'demo')
    r = mf.replay(root)
    from kvm_amd import bundle as bl
    m0 = bl.load(root / 'train').metadata['buffers']
    W = bl.materialize(next(x for x in m0 if x['name'] == 'W'))
    G = bl.materialize(next(x for x in m0 if x['name'] == 'G'))
    X = bl.materialize(next(x for x in bl.load(root / 'serve1').metadata['buffers'] if x['name'] == 'X'))
    for k in range(1, 4):
        W = (W - np.float32(0.1) * G).astype(np.float32)
        want = X.reshape(4, 8).astype(np.float64) @ W.reshape(8, 8).astype(np.float64)
        assert np.allclose(r['buffers'][f'Y{k}'].reshape(4, 8), want, rtol=1e-5, atol=1e-6), k
    assert r['versions'] == {'w': 3}


def _edit(root, fn):
    p = root / 'MANIFEST.json'
    m = json.loads(p.read_text())
    fn(m)
    p.write_text(json.dumps(m))


@pytest.mark.parametrize('edit, msg', [
    (lambda m: m['admissions'][1].update(when=[{'var': 'w', 'min': 5, 'max': 5}]), 'cannot complete'),
    (lambda m: m['admissions'][0].update(after_bundles=['serve3']), 'cannot complete'),
    (lambda m: m['admissions'][0].update(workload='nope'), "unknown workload 'nope'"),
    (lambda m: m['admissions'][0].update(publishes={'w': 1}, base_versions={}), 'has no base version'),
    (lambda m: m.update(manifest_version=2), 'manifest_version must be 1'),
    (lambda m: m['buffers']['W'].update(dtype='f64'), 'is not f32, i32 or bf16'),
    (lambda m: m['classes']['serve'].update(speed=3), "unknown scheduler parameter 'speed'"),
    (lambda m: m['admissions'][1].update(bundle_dir='../x'), 'relative path'),
    (lambda m: m['admissions'][0].update(after_bundles=['train1']), 'waits for itself'),
])
def test_malformed_manifests_are_refused(tmp_path, edit, msg):
    root = manifest_demo.build(tmp_path / 'demo')
    _edit(root, edit)
    rc, out, err = _run(root, '--check-only')
    assert rc == 1 and msg in err, (rc, out, err)


def test_a_bundle_that_does_not_fit_the_table_is_refused(tmp_path):
    root = manifest_demo.build(tmp_path / 'demo')
    _edit(root, lambda m: m['buffers']['X'].update(rows=2))
    rc, out, err = _run(root, '--check-only')
    assert rc == 1 and 'admission serve1' in err, (out, err)


def test_an_admission_compiled_on_demand(tmp_path):
    """The probe admission has no bundle: the runner compiles its workload file (file init read from its data dir)."""
    root = manifest_demo.build(tmp_path / 'demo', probe=True)
    rc, out, err = _run(root, '--check-only')
    assert rc == 0 and out.startswith('OK') and 'probe1' in out, (out, err)
    r = mf.replay(root)
    P = np.arange(32, dtype=np.float32).reshape(4, 8) * np.float32(0.125)
    want = P.astype(np.float64) @ r['buffers']['W'].reshape(8, 8).astype(np.float64)
    assert np.allclose(r['buffers']['Z'].reshape(4, 8), want, rtol=1e-5, atol=1e-6)
    (root / 'data' / 'p.bin').write_bytes(bytes(12))
    rc, out, err = _run(root, '--check-only')
    assert rc == 1 and 'compiling workloads/probe.json' in err and 'bytes' in err, (out, err)
    (root / 'workloads' / 'probe.json').unlink()
    rc, out, err = _run(root, '--check-only')
    assert rc == 1 and 'probe1' in err, (out, err)
