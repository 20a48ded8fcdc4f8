"""Writes tests/golden/data/decode_fp64_deviation.json: the reference CPU path's own deviation from an fp64 run on the
full-width Qwen3-8B-shape decode graph (hidden 4096, 32/8 heads, hd 128, ffn 12288, vocab 151936, 4096-token cache) cut
to one layer, batch 1 and 8, and at full depth (36 layers), batch 1 and 8 (keys b1_full, b8_full). "Reference CPU path" is the oracle (the C++ restatement of the reference's CPU VM and
ops, rounding like the reference); the fp64 run is tests/decode_fp64.py on the same initial buffers. Decode tolerances
are twice these figures. Run from the repository root: python tests/golden/make_decode_deviation.py
"""
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / 'tests')]

import decode_fp64 as D  # noqa: E402
import oracle  # noqa: E402
from kvm_amd import bundle as bl  # noqa: E402
from kvm_amd import compiler  # noqa: E402
from kvm_amd.workloads import qwen3  # noqa: E402


def deviation(batch, threads=8, layers=1):
    c = qwen3.Qwen3Config(batch=batch, layers=layers, max_new=4)
    w = qwen3.build(c)
    lb = bl.load(compiler.compile_spec(w.spec))
    names = [m['name'] for m in lb.metadata['buffers']]
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    ref64 = D.decode_step(c, dict(zip(names, init)))
    r = oracle.run(lb, init, threads=threads)
    got = D.graph_outputs(c, names, r['buffers'])
    return {'deviation': D.deviations(got, ref64), 'tok': got['tok'].tolist(), 'tok_fp64': ref64['tok'].tolist()}


if __name__ == '__main__':
    out = {'graph': 'qwen3 decode, 1 layer at full width (hidden 4096, H 32, Hkv 8, hd 128, ffn 12288, V 151936, ctx 4096)',
           'metric': 'relative L2 of the oracle (reference rounding) against an fp64 run of the same step'}
    for b in (1, 8):
        out[f'b{b}'] = deviation(b)
        print(b, out[f'b{b}'], flush=True)
    for b in (1, 8):
        out[f'b{b}_full'] = deviation(b, layers=36)
        print(b, 'full depth', out[f'b{b}_full'], flush=True)
    (ROOT / 'tests/golden/data/decode_fp64_deviation.json').write_text(json.dumps(out, indent=1) + '\n')
