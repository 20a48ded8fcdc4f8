"""Shared comparison of an executor run with the CPU oracle (used by the GPU tests and smoke())."""
from __future__ import annotations

import numpy as np

from kvm_amd import bundle as bl

# Tolerances on the relative L2 error of a buffer versus the oracle. The oracle computes in double and rounds each
# stored value to f32, like the reference CPU path; the device computes in fp32 (MFMA / FMA, reassociated sums).
# The reference's own device-vs-CPU table allows 1e-5 (norms, activations, losses, optimizer) and 2e-5 (attention);
# f32 buffers here are held to 2e-5. bf16-storage buffers differ where the fp32 result lands on the other side of a
# bf16 rounding boundary (one bf16 ulp = 2^-8 relative), held to 4e-3.
TOL_F32 = 2e-5
TOL_BF16 = 4e-3


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    den = np.sqrt((want * want).sum())
    return float(np.sqrt(((got - want) ** 2).sum()) / max(den, 1e-30))


def compare_run(ex, meta, ref, tol_f32=TOL_F32, tol_bf16=TOL_BF16, skip=()):
    """Returns a list of (buffer, error, tolerance) failures."""
    bad = []
    for m, want in zip(meta['buffers'], ref['buffers']):
        if m['name'] in skip:
            continue
        got = ex.read(m['name'])
        if m['dtype'] == bl.DT_I32:
            if not np.array_equal(got, want):
                bad.append((m['name'], int((got != want).sum()), 0))
            continue
        if not np.all(np.isfinite(got) == np.isfinite(want)):
            bad.append((m['name'], 'nonfinite', 0))
            continue
        tol = tol_bf16 if m['dtype'] == bl.DT_BF16 else tol_f32
        e = rel_l2(got, want)
        if e > tol:
            bad.append((m['name'], e, tol))
    return bad


def check_schedule(ex, b: bl.LoadedBundle):
    """Every task ran exactly once, after all of its predecessors ended."""
    tr = ex.trace()
    assert (tr['exec_count'] == 1).all(), f"exec_count != 1 for tasks {np.nonzero(tr['exec_count'] != 1)[0][:10]}"
    t = b.tasks
    for u in range(t.shape[0]):
        for v in b.succ[t[u, 1]:t[u, 1] + t[u, 2]]:
            assert tr['start'][v] >= tr['end'][u], f'task {v} started before predecessor {u} ended'
    return tr
