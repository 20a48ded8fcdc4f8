"""The manifest runner on the GPU (kvm_run; reference: demo/mvm_run.cu): the train + serve demo runs on one
persistent kernel in stream mode, admissions in the order their version conditions allow (each serve pass on exactly
the weights version it asked for), results equal to the serial CPU replay of the same manifest."""
import json
import subprocess

import numpy as np
import pytest

import manifest_demo
from conftest import REPO
from kvm_amd import manifest as mf

pytestmark = pytest.mark.gpu
RUNNER = REPO / 'kvm_amd' / '_build' / 'kvm_run'


def test_train_and_serve_demo_matches_the_serial_replay(tmp_path):
    root = manifest_demo.build(tmp_path / 'demo', steps=3)
    out = tmp_path / 'out'
    print('kvm_run train + serve demo', flush=True)
    r = subprocess.run([str(RUNNER), str(root), '--out', str(out), '--dump', '^(W|Y[0-9])$', '--windows', '2', '--timeout-s', '60'],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith('OK: 6/6 tasks'), (r.stdout, r.stderr)
    s = json.loads((out / 'summary.json').read_text())
    assert s['ok'] and s['versions'] == {'w': 3}
    adm = {a['name']: a for a in s['admissions']}
    for k in range(1, 4):
        assert adm[f'serve{k}']['versions_at_done'] == {'w': k}
        # serve k is admitted once train k has published w = k, which can precede the runner's sight of train k's
        # completion mark; train k + 1 waits for serve k to complete
        assert adm[f'train{k}']['submitted_us'] <= adm[f'serve{k}']['submitted_us']
        if k > 1:
            assert adm[f'serve{k - 1}']['done_us'] <= adm[f'train{k}']['submitted_us']
    assert adm['train2']['how'].startswith('previous bundle') and 'shifted' in adm['train2']['how']
    ref = mf.replay(root)
    for name in ('W', 'Y1', 'Y2', 'Y3'):
        got = np.fromfile(out / f'{name}.bin', np.float32)
        want = ref['buffers'][name].reshape(-1)
        assert np.allclose(got, want, rtol=2e-5, atol=1e-6), (name, np.abs(got - want).max())


def test_admission_compiled_on_demand_runs(tmp_path):
    root = manifest_demo.build(tmp_path / 'demo', steps=2, probe=True)
    out = tmp_path / 'out'
    print('kvm_run demo with an on-demand compile', flush=True)
    r = subprocess.run([str(RUNNER), str(root), '--out', str(out), '--dump', '^(W|Z)$', '--timeout-s', '60'],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith('OK: 5/5 tasks'), (r.stdout, r.stderr)
    adm = {a['name']: a for a in json.loads((out / 'summary.json').read_text())['admissions']}
    assert adm['probe1']['how'] == 'compiled on demand'
    ref = mf.replay(root)
    for name in ('W', 'Z'):
        got = np.fromfile(out / f'{name}.bin', np.float32)
        assert np.allclose(got, ref['buffers'][name].reshape(-1), rtol=2e-5, atol=1e-6), name
