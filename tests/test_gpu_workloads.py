"""GPU parity of the generated benchmark workloads at small sizes against the CPU oracle.

Composite graphs accumulate the device's fp32 / MFMA reassociation and bf16 re-roundings of intermediate activations
through every layer, so they are held to end-to-end tolerances (relative L2 per buffer) rather than the per-op ones;
integer buffers (tokens, lengths) must match exactly.
"""
import numpy as np
import pytest

import oracle
from gpu_check import check_schedule, compare_run
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.executor import Executor
from kvm_amd.workloads import qwen3

pytestmark = pytest.mark.gpu

TOL_DECODE_F32 = 2e-3     # logits / residual stream after 2 layers with bf16 activations
TOL_DECODE_BF16 = 2e-2    # bf16 KV-cache rows written this step


def _run_both(w, steps=1):
    lb = bl.load(compiler.compile_spec(w.spec))
    init = [bl.materialize({**m, 'init': w.init_override.get(m['name'], m['init'])}) for m in lb.metadata['buffers']]
    ref = oracle.run(lb, [x.copy() for x in init])
    ex = Executor.from_bundle(lb, buffers=init)
    ex.run()
    return lb, ref, ex


@pytest.mark.parametrize('batch', [1, 2, 8])
def test_qwen3_decode_tiny(batch):
    print(f'qwen3 tiny decode batch {batch}', flush=True)
    w = qwen3.build(qwen3.Qwen3Config.tiny(batch=batch))
    lb, ref, ex = _run_both(w)
    check_schedule(ex, lb)
    bad = compare_run(ex, lb.metadata, ref, tol_f32=TOL_DECODE_F32, tol_bf16=TOL_DECODE_BF16)
    assert not bad, bad
    names = [m['name'] for m in lb.metadata['buffers']]
    assert np.array_equal(ex.read('tok'), ref['buffers'][names.index('tok')])
    assert np.array_equal(ex.read('lens'), ref['buffers'][names.index('lens')])
    ex.close()
