"""The manifest runner's host side (kvm_run --check-only; reference: demo/mvm_run.cu): well-formed demos pass the
checks without a GPU, the serial version flow orders train / serve as their versions require with `publishes` read as
an increment (frontend/mvmfe/demo.py:136), bundles whose publications disagree with their admission are refused,
scheduler classes are accepted (a static split needs one share per class), and malformed manifests are refused with
the reason."""
import json
import subprocess

import numpy as np
import pytest

import manifest_demo
from conftest import REPO
from manifest_replay import replay, serial_order
from kvm_amd import bundle as bl
from kvm_amd import manifest as mf

RUNNER = REPO / 'kvm_amd' / '_build' / 'kvm_run'


def _run(*args):
    r = subprocess.run([str(RUNNER), *map(str, args)], capture_output=True, text=True, timeout=120)
    return r.returncode, r.stdout, r.stderr


def _check(root, *extra):
    return _run(root, '--check-only', '--sched', 'off', *extra)


def test_demo_checks_and_serial_order(tmp_path):
    root = manifest_demo.build(tmp_path / 'demo')
    rc, out, err = _check(root)
    want = ['train1', 'serve1', 'train2', 'serve2', 'train3', 'serve3']
    assert rc == 0 and out.startswith('OK') and out.split('serial order ')[1].split() == want, (out, err)
    assert serial_order(mf.load(root)) == want


def test_window_demo_publishes_are_increments(tmp_path):
    """demo.py's training windows: base 2 * start, publishes 2 * steps. With publishes read as an absolute version
    the flow would stop after the first window."""
    root = manifest_demo.build_windows(tmp_path / 'demo', windows=3, steps=2)
    want = ['serve_s0', 'train_w0', 'serve_s2', 'train_w1', 'serve_s4', 'train_w2', 'serve_s6']
    rc, out, err = _run(root, '--check-only')
    assert rc == 0 and out.split('serial order ')[1].split() == want, (out, err)
    assert serial_order(mf.load(root)) == want


def test_window_replay_is_the_closed_form(tmp_path):
    """Each step subtracts lr G1 from W1 and lr G2 from W2; serve_s{k} sees the weights after k steps."""
    root = manifest_demo.build_windows(tmp_path / 'demo', windows=3, steps=2, lr=0.05)
    r = replay(root)
    assert r['versions'] == {'weights': 12}
    meta = {x['name']: x for x in bl.load(root / 'train_window').metadata['buffers']}
    X = bl.materialize(next(x for x in bl.load(root / 'serve_s0').metadata['buffers'] if x['name'] == 'X')).reshape(4, 8)
    W1, W2 = (bl.materialize(meta[n]).reshape(8, 8) for n in ('W1', 'W2'))
    G1, G2 = (bl.materialize(meta[n]).reshape(8, 8) for n in ('G1', 'G2'))
    for k in range(7):
        if k % 2 == 0:
            for out, W in (('Y', W1), ('Z', W2)):
                want = X.astype(np.float64) @ W.astype(np.float64)
                assert np.allclose(r['buffers'][f'{out}{k}'].reshape(4, 8), want, rtol=1e-5, atol=1e-6), (out, k)
        W1 = (W1 - np.float32(0.05) * G1).astype(np.float32)
        W2 = (W2 - np.float32(0.05) * G2).astype(np.float32)


def test_replay_is_the_closed_form(tmp_path):
    """The CPU replay: W_k = W_{k-1} - 0.1 G (f32), Y_k = X W_k."""
    root = manifest_demo.build(tmp_path / 'demo')
    r = replay(root)
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


def test_classes_and_sched_modes(tmp_path):
    """Declared classes run under the default dynamic scheduler; --sched static needs one share per class (train,
    serve), and an unknown mode or a share below 1 is a usage error (exit 2)."""
    root = manifest_demo.build(tmp_path / 'demo')
    for extra in ((), ('--sched', 'off'), ('--sched', 'global'), ('--sched', 'static', '--shares', '1,3')):
        rc, out, err = _run(root, '--check-only', *extra)
        assert rc == 0 and out.startswith('OK'), (extra, out, err)
    rc, out, err = _run(root, '--check-only', '--sched', 'static')
    assert rc == 1 and '--shares' in err and '2 classes' in err, (out, err)
    rc, out, err = _run(root, '--check-only', '--sched', 'static', '--shares', '1,2,3')
    assert rc == 1 and '--shares' in err, (out, err)
    assert _run(root, '--check-only', '--sched', 'fifo')[0] == 2
    assert _run(root, '--check-only', '--sched', 'static', '--shares', '1,0')[0] == 2
    rc, out, err = _run(manifest_demo.build(tmp_path / 'plain', classes=False), '--check-only')
    assert rc == 0, (out, err)


@pytest.mark.parametrize('edit, msg', [
    (lambda m: m['admissions'][1].update(when=[{'var': 'w', 'min': 5, 'max': 5}]), 'version flow: stuck after 1 of 6'),
    (lambda m: m['admissions'][0].update(after_bundles=['serve3']), 'version flow: stuck after 0 of 6'),
    (lambda m: m['admissions'][0].update(workload='nope'), 'no workload is called "nope"'),
    (lambda m: m['admissions'][0].update(publishes={'w': 1}, base_versions={}), 'needs an entry in base_versions'),
    (lambda m: m['admissions'][0].update(publishes={'w': 0}), '$.admissions[0].publishes.w: is 0'),
    (lambda m: m.update(manifest_version=2), 'reads manifest_version 1'),
    (lambda m: m['buffers']['W'].update(dtype='f64'), 'is not one of f32, i32, bf16'),
    (lambda m: m['classes']['serve'].update(speed=3), '"speed" is not a scheduler class parameter'),
    (lambda m: m['admissions'][1].update(bundle_dir='../x'), 'leaves the demo directory'),
    (lambda m: m['admissions'][0].update(after_bundles=['train1']), 'lists itself'),
    (lambda m: m['admissions'][1]['when'][0].update(max=0), 'the window is empty'),
    (lambda m: m['buffers']['W'].update(rows=1.5), '$.buffers.W.rows: must be a whole number'),
])
def test_malformed_manifests_are_refused(tmp_path, edit, msg):
    root = manifest_demo.build(tmp_path / 'demo')
    _edit(root, edit)
    rc, out, err = _check(root)
    assert rc == 1 and msg in err, (rc, out, err)


def test_publications_must_match_the_declared_increment(tmp_path):
    """A bundle that advances `weights` by 4 under an admission that declares 3 (or declares nothing) is refused
    before launch: otherwise later admissions compiled for base + declared would never open."""
    root = manifest_demo.build_windows(tmp_path / 'demo', windows=3, steps=2)
    _edit(root, lambda m: m['admissions'][1].update(publishes={'weights': 3}))
    rc, out, err = _run(root, '--check-only')
    assert rc == 1 and 'admission train_w0: its bundle leaves weights at 4' in err and '0 + 3 = 3' in err, (out, err)
    root = manifest_demo.build_windows(tmp_path / 'demo2', windows=1, steps=2)
    _edit(root, lambda m: [m['admissions'][1].pop('publishes'), m['admissions'][2]['when'][0].update(min=0, max=0)])
    rc, out, err = _run(root, '--check-only')
    assert rc == 1 and 'publishes weights, which the admission' in err, (out, err)


def test_a_bundle_that_does_not_fit_the_table_is_refused(tmp_path):
    root = manifest_demo.build(tmp_path / 'demo')
    _edit(root, lambda m: m['buffers']['X'].update(rows=2))
    rc, out, err = _check(root)
    assert rc == 1 and 'admission serve1' in err, (out, err)


def test_an_admission_compiled_on_demand(tmp_path):
    """The probe admission has no bundle: the runner compiles its workload file (file init read from its data dir)."""
    root = manifest_demo.build(tmp_path / 'demo', probe=True)
    rc, out, err = _check(root)
    assert rc == 0 and out.startswith('OK') and 'probe1' in out, (out, err)
    r = replay(root)
    P = np.arange(32, dtype=np.float32).reshape(4, 8) * np.float32(0.125)
    want = P.astype(np.float64) @ r['buffers']['W'].reshape(8, 8).astype(np.float64)
    assert np.allclose(r['buffers']['Z'].reshape(4, 8), want, rtol=1e-5, atol=1e-6)
    (root / 'data' / 'p.bin').write_bytes(bytes(12))
    rc, out, err = _check(root)
    assert rc == 1 and 'compiling workloads/probe.json failed' in err and 'bytes' in err, (out, err)
    (root / 'workloads' / 'probe.json').unlink()
    rc, out, err = _check(root)
    assert rc == 1 and 'probe1' in err, (out, err)
