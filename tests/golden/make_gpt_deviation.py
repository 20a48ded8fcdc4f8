"""Writes tests/golden/data/gpt_fp64_deviation.json: the reference CPU path's own deviation from an fp64 run on the
full GPT-162M training step (12 layers, d 768, 12 heads, T 1024, batch 4, vocab 50304, tied, bf16 storage with fp32
master weights). "Reference CPU path" is the oracle (the C++ restatement of the reference's CPU VM and ops, rounding
like the reference); the fp64 run is tests/gpt_fp64.py on the same initial buffers. The full-depth GPT tolerances are
twice these figures. Run from the repository root: python tests/golden/make_gpt_deviation.py
"""
import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / 'tests')]

import gpt_fp64 as G  # noqa: E402
import oracle  # noqa: E402
from kvm_amd import bundle as bl  # noqa: E402
from kvm_amd import compiler  # noqa: E402
from kvm_amd.workloads import gpt  # noqa: E402


def deviation(c, threads=8):
    w = gpt.build(c)
    lb = bl.load(compiler.compile_spec(w.spec))
    names = [m['name'] for m in lb.metadata['buffers']]
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    t0 = time.time()
    ref = G.step(c, {n: x.copy() for n, x in zip(names, init) if not n.startswith(('d.', 'm.', 'v.'))})
    t1 = time.time()
    r = oracle.run(lb, init, threads=threads)
    print(f'fp64 step {t1 - t0:.1f} s, oracle {time.time() - t1:.1f} s', flush=True)
    return {'deviation': G.deviations(names, r['buffers'], ref), 'loss': r['buffers'][names.index('loss')][0].item(),
            'loss_fp64': ref['loss']}


if __name__ == '__main__':
    c = gpt.GPTConfig()
    out = {'graph': 'gpt-162m training step, full depth (12 layers, d 768, H 12, T 1024, B 4, V 50304, tied, bf16 storage)',
           'metric': 'relative L2 of the oracle (reference rounding) against an fp64 run of the same step, per quantity: '
                     'logits, gradient groups (g.*) and parameter groups after AdamW (p.*), pooled over layers; loss_abs '
                     'is the absolute loss difference'}
    out.update(deviation(c))
    print(json.dumps(out, indent=1))
    (ROOT / 'tests/golden/data/gpt_fp64_deviation.json').write_text(json.dumps(out, indent=1) + '\n')
