"""The manifest runner on the GPU (kvm_run; reference: demo/mvm_run.cu): demos run on one persistent kernel in stream
mode, admissions in the order their version gates allow, results equal to the serial CPU replay of the same manifest.
The window demo has the frontend's training-window shape (frontend/mvmfe/demo.py:185-194): each window is admitted at
base 2 * start and advances `weights` by 2 * steps."""
import json
import subprocess

import numpy as np
import pytest

import manifest_demo
from conftest import REPO
from manifest_replay import replay

pytestmark = pytest.mark.gpu
RUNNER = REPO / 'kvm_amd' / '_build' / 'kvm_run'


def _kvm_run(root, out, *args):
    r = subprocess.run([str(RUNNER), str(root), '--out', str(out), '--timeout-s', '60', *args], capture_output=True, text=True, timeout=120)
    return r, (json.loads((out / 'summary.json').read_text()) if (out / 'summary.json').exists() else None)


def _matches_replay(out, ref, names):
    for name in names:
        got = np.fromfile(out / f'{name}.bin', np.float32)
        want = ref['buffers'][name].reshape(-1)
        assert np.allclose(got, want, rtol=2e-5, atol=1e-6), (name, np.abs(got - want).max())


def test_train_and_serve_demo_matches_the_serial_replay(tmp_path):
    root = manifest_demo.build(tmp_path / 'demo', steps=3)
    out = tmp_path / 'out'
    print('kvm_run train + serve demo', flush=True)
    r, s = _kvm_run(root, out, '--dump', '^(W|Y[0-9])$', '--windows', '2')
    assert r.returncode == 0 and r.stdout.startswith('OK: 6/6 tasks'), (r.stdout, r.stderr)
    assert s['ok'] and s['versions'] == {'w': 3}
    # the manifest's classes (train, serve) scheduled by the device's class scheduler: each task counted in its class
    assert s['sched'] == 'dynamic' and [c['name'] for c in s['classes']] == ['train', 'serve']
    assert [c['tasks'] for c in s['classes']] == [3, 3]
    adm = {a['name']: a for a in s['admissions']}
    for k in range(1, 4):
        assert adm[f'serve{k}']['versions_at_done'] == {'w': k}
        # serve k is admitted once train k has published w = k, which can precede the runner's sight of train k's
        # completion mark; train k + 1 waits for serve k to complete
        assert adm[f'train{k}']['submitted_us'] <= adm[f'serve{k}']['submitted_us']
        if k > 1:
            assert adm[f'serve{k - 1}']['done_us'] <= adm[f'train{k}']['submitted_us']
    assert adm['train2']['how'] == 'reused, versions moved'
    _matches_replay(out, replay(root), ('W', 'Y1', 'Y2', 'Y3'))


def test_training_windows_advance_by_their_publishes(tmp_path):
    """Three windows of two steps: weights 0 -> 4 -> 8 -> 12, windows 2 and 3 reuse window 1's bundle moved to base 4
    and 8, a serving pass on each stable version in between."""
    root = manifest_demo.build_windows(tmp_path / 'demo', windows=3, steps=2)
    out = tmp_path / 'out'
    print('kvm_run training-window demo', flush=True)
    r, s = _kvm_run(root, out, '--dump', '^(W[12]|[YZ][0-9]+)$', '--windows', '2')
    assert r.returncode == 0 and r.stdout.startswith('OK: 20/20 tasks'), (r.stdout, r.stderr)
    assert s['versions'] == {'weights': 12}
    adm = {a['name']: a for a in s['admissions']}
    for i in range(3):
        assert adm[f'train_w{i}']['versions_at_done']['weights'] >= 4 * (i + 1)
        assert adm[f'train_w{i}']['how'] == ('bundle_dir' if i == 0 else 'reused, versions moved')
    for k in (0, 2, 4, 6):
        assert adm[f'serve_s{k}']['versions_at_done'] == {'weights': 2 * k}
    ref = replay(root)
    assert ref['order'] == s['serial_order']
    _matches_replay(out, ref, ['W1', 'W2'] + [f'{p}{k}' for p in 'YZ' for k in (0, 2, 4, 6)])


def test_static_class_split_runs_the_demo(tmp_path):
    """The same demo with the workers split 1:3 between the train and serve classes (--sched static): same results."""
    root = manifest_demo.build(tmp_path / 'demo', steps=3)
    out = tmp_path / 'out'
    print('kvm_run train + serve demo, static class split', flush=True)
    r, s = _kvm_run(root, out, '--dump', '^(W|Y[0-9])$', '--sched', 'static', '--shares', '1,3', '--blocks', '16')
    assert r.returncode == 0 and r.stdout.startswith('OK: 6/6 tasks'), (r.stdout, r.stderr)
    assert s['sched'] == 'static' and [c['tasks'] for c in s['classes']] == [3, 3]
    _matches_replay(out, replay(root), ('W', 'Y1', 'Y2', 'Y3'))


def test_admission_compiled_on_demand_runs(tmp_path):
    root = manifest_demo.build(tmp_path / 'demo', steps=2, probe=True)
    out = tmp_path / 'out'
    print('kvm_run demo with an on-demand compile', flush=True)
    r, s = _kvm_run(root, out, '--dump', '^(W|Z)$', '--sched', 'off')
    assert r.returncode == 0 and r.stdout.startswith('OK: 5/5 tasks'), (r.stdout, r.stderr)
    adm = {a['name']: a for a in s['admissions']}
    assert adm['probe1']['how'] == 'compiled on demand'
    _matches_replay(out, replay(root), ('W', 'Z'))
