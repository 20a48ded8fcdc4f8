"""GPU parity at the BASELINE configurations' full widths against the CPU oracle (the reference's CPU path restated;
run with several threads, same results as one).

- C5 Qwen3-8B-shape decode, one layer at full width (hidden 4096, 32 / 8 heads, hd 128, ffn 12288, vocab 151936,
  4096-token cache), batch 1 and 8: tokens and lengths exact; logits, final residual and the new KV-cache rows within
  twice the reference path's own deviation from an fp64 run of the same step (tests/golden/data/
  decode_fp64_deviation.json, written by tests/golden/make_decode_deviation.py).
- C5 at full depth (36 layers + LM head), batch 1 and 8: the same checks against the full-depth fp64 deviations (b1_full,
  b8_full in the same file); a token may differ from the reference path's only at a near-tie inside that deviation.
- C3 GPT-162M, one layer at full width (d 768, 12 heads, T 1024, batch 4, vocab 50304, tied), bf16 storage: step-1
  weight gradients within 3.4e-2 relative L2 (twice the reference's bf16s deviation from fp64, 1.69e-2, README.md:212
  of the reference), loss within 1e-2.
- C3 GPT-162M, full depth (12 layers): loss, logits, gradient groups and parameter groups after AdamW within twice the
  reference path's own deviation from an fp64 run of the step (tests/golden/data/gpt_fp64_deviation.json, written by
  tests/golden/make_gpt_deviation.py with tests/gpt_fp64.py).
- C4 GPT-355M shape, two layers (d 1024, 16 heads, T 1024, ffn 4096, vocab 50304), f32, batch 1: every buffer after
  the step within the reference's TOL_PRECISE 2e-4 (tests/gptdiff/golden_check.py:28-31 of the reference).
- C2 the eight MLPs (784 -> w -> w -> 10, all eight widths, batch 256), two training steps: every buffer within 2e-4.
"""
import json

import numpy as np
import pytest

import decode_fp64 as D
import oracle
from conftest import REPO
from gpu_check import check_schedule, compare_run, rel_l2
from kvm_amd import bundle as bl
from kvm_amd import compiler
from kvm_amd.executor import Executor

pytestmark = pytest.mark.gpu
THREADS = 16     # oracle worker threads (the box's CPU share)


def _prepare(w):
    lb = bl.load(compiler.compile_spec(w.spec))
    names = [m['name'] for m in lb.metadata['buffers']]
    init = [oracle.materialize(m, w.init_override.get(m['name'])) for m in lb.metadata['buffers']]
    return lb, names, init


def _device(w, lb):
    """The executor seeds its buffers on the device (bit-identical to oracle.materialize)."""
    ex = Executor(num_vars=max(1, len(lb.metadata['variables'])), trace=True, timeout_s=60.0)
    for m in lb.metadata['buffers']:
        ex.add_buffer(m['name'], m['rows'], m['cols'], m['dtype'], init=w.init_override.get(m['name'], m['init']))
    for v in lb.metadata['variables']:
        ex.set_version(v['id'], v['base_version'])
    ex.submit(lb)
    ex.run()
    return ex


@pytest.mark.parametrize('batch', [1, 8])
def test_qwen3_decode_full_width_one_layer(batch):
    from kvm_amd.workloads import qwen3
    print(f'qwen3 full width, 1 layer, batch {batch}', flush=True)
    dev = json.loads((REPO / 'tests/golden/data/decode_fp64_deviation.json').read_text())[f'b{batch}']
    c = qwen3.Qwen3Config(batch=batch, layers=1, max_new=4)
    w = qwen3.build(c)
    lb, names, init = _prepare(w)
    ex = _device(w, lb)
    check_schedule(ex, lb)
    r = oracle.run(lb, init, threads=THREADS)
    want = D.graph_outputs(c, names, r['buffers'])
    got = D.graph_outputs(c, names, [ex.read(n) for n in names])
    assert got['tok'].tolist() == want['tok'].tolist() == dev['tok']
    assert np.array_equal(ex.read('lens'), r['buffers'][names.index('lens')])
    err = D.deviations(got, want)
    print('device vs reference path', err, 'tolerance 2 x', dev['deviation'], flush=True)
    for k, e in err.items():
        assert e <= 2 * dev['deviation'][k], (k, e, dev['deviation'][k])
    ex.close()


@pytest.mark.timeout(600)
@pytest.mark.parametrize('batch', [1, 8])
def test_qwen3_decode_full_depth(batch):
    """The whole 36-layer Qwen3-8B-shape decode step (+ LM head): tokens and lengths exact; logits, final residual and
    the new KV-cache rows of every layer within twice the reference path's own deviation from an fp64 run of the same
    step at full depth (b1_full / b8_full in tests/golden/data/decode_fp64_deviation.json)."""
    import os
    from kvm_amd.workloads import qwen3
    print(f'qwen3 full depth, batch {batch}', flush=True)
    dev = json.loads((REPO / 'tests/golden/data/decode_fp64_deviation.json').read_text())[f'b{batch}_full']
    c = qwen3.Qwen3Config(batch=batch, max_new=4)
    w = qwen3.build(c)
    lb, names, init = _prepare(w)
    ex = _device(w, lb)
    check_schedule(ex, lb)
    need = {'logits', 'x', 'tok', 'lens'} | {f'{k}.{l}' for k in ('kc', 'vc') for l in range(c.layers)}
    got_bufs = [ex.read(n) if n in need else None for n in names]
    ex.close()
    r = oracle.run(lb, init, threads=min(THREADS, os.cpu_count() or 1))
    want = D.graph_outputs(c, names, r['buffers'])
    got = D.graph_outputs(c, names, got_bufs)
    assert want['tok'].tolist() == dev['tok']
    assert np.array_equal(got_bufs[names.index('lens')], r['buffers'][names.index('lens')])
    err = D.deviations(got, want)
    print('device vs reference path', err, 'tolerance 2 x', dev['deviation'], flush=True)
    for k, e in err.items():
        assert e <= 2 * dev['deviation'][k], (k, e, dev['deviation'][k])
    # Tokens: the reference path's, except at a near-tie that the reference path's own deviation from fp64 covers (36
    # layers of bf16 activations move the logits by ~2% RMS): a different token must then score, in the reference
    # path's logits, within twice that deviation (per element, RMS) of the best one.
    for bb, (t_got, t_want) in enumerate(zip(got['tok'].tolist(), want['tok'].tolist())):
        if t_got != t_want:
            lg = want['logits'][bb]
            margin, allow = lg[t_want] - lg[t_got], 2 * dev['deviation']['logits'] * float(np.sqrt(np.mean(lg * lg)))
            print(f'sequence {bb}: token {t_got} (reference path {t_want}), logit margin {margin:.4g}, allowed {allow:.4g}', flush=True)
            assert margin <= allow, (bb, t_got, t_want, margin, allow)


TOL_GPT_BF16_GRAD = 3.4e-2


def test_gpt162m_full_width_one_layer_step():
    from kvm_amd.workloads import gpt
    print('gpt-162m full width, 1 layer, bf16 step', flush=True)
    w = gpt.build(gpt.GPTConfig(layers=1))
    lb, names, init = _prepare(w)
    ex = _device(w, lb)
    check_schedule(ex, lb)
    r = oracle.run(lb, init, threads=THREADS)
    loss, want = ex.read('loss'), r['buffers'][names.index('loss')]
    assert abs(loss[0] - want[0]) <= 1e-2 * abs(want[0]), (loss, want)
    assert abs(want[0] - np.log(50304)) < 0.05 * np.log(50304)          # near ln V at initialisation
    worst = sorted(((rel_l2(ex.read(n), x), n) for n, x in zip(names, r['buffers'])
                    if n.startswith('d.') and not n.startswith('d.bk.')), reverse=True)
    print('worst gradient rel L2', worst[:3], flush=True)
    assert worst[0][0] <= TOL_GPT_BF16_GRAD, worst[:5]
    assert np.array_equal(ex.read('step'), r['buffers'][names.index('step')])
    ex.close()


def test_gpt162m_full_depth_step():
    """The whole GPT-162M training step (12 layers, bf16 storage, fp32 master AdamW) against the oracle: the loss,
    the logits, every gradient group and every parameter group after AdamW (pooled over layers) within twice the
    reference path's own deviation from an fp64 run of the same step (tests/golden/data/gpt_fp64_deviation.json,
    written by tests/golden/make_gpt_deviation.py with tests/gpt_fp64.py)."""
    import os
    import gpt_fp64 as G
    from kvm_amd.workloads import gpt
    print('gpt-162m full depth, bf16 step', flush=True)
    dev = json.loads((REPO / 'tests/golden/data/gpt_fp64_deviation.json').read_text())
    w = gpt.build(gpt.GPTConfig())
    lb, names, init = _prepare(w)
    ex = _device(w, lb)
    check_schedule(ex, lb)
    got = [ex.read(n) for n in names]
    ex.close()
    r = oracle.run(lb, init, threads=min(THREADS, os.cpu_count() or 1))
    err = G.deviations(names, got, G.quantities(names, r['buffers']))
    worst = sorted(((e / dev['deviation'][k], k, e) for k, e in err.items()), reverse=True)
    print('device vs reference path / reference deviation from fp64, worst:', worst[:4], flush=True)
    for ratio, k, e in worst:
        assert ratio <= 2.0, (k, e, dev['deviation'][k])
    assert np.array_equal(got[names.index('step')], r['buffers'][names.index('step')])


test_gpt162m_full_depth_step = pytest.mark.timeout(600)(test_gpt162m_full_depth_step)

TOL_PRECISE = 2e-4


def test_gpt355m_shape_f32_two_layers_step():
    from kvm_amd.workloads import gpt
    print('gpt-355m shape, 2 layers, f32 step', flush=True)
    w = gpt.build(gpt.GPTConfig.gpt355m(layers=2, batch=1))
    lb, names, init = _prepare(w)
    ex = _device(w, lb)
    check_schedule(ex, lb)
    r = oracle.run(lb, init, threads=THREADS)
    # Vectors that start at zero (biases, LayerNorm shifts) hold -lr * g / (|g| + eps) after the first AdamW step: an
    # element whose gradient is near zero takes either sign under any change of summation order, so these are held
    # elementwise to the size of one update instead; their gradients and moments are compared like everything else.
    # The key bias has an exactly zero gradient (softmax is shift-invariant): noise on both sides, skipped.
    zero_init = [m['name'] for m in lb.metadata['buffers'] if m['init'].get('kind') == 'fill' and m['init'].get('value') == 0
                 and f'd.{m["name"]}' in names]
    skip = tuple(zero_init) + tuple(n for n in names if n.startswith(('d.bk.', 'm.bk.', 'v.bk.')))
    bad = compare_run(ex, lb.metadata, r, tol_f32=TOL_PRECISE, skip=skip)
    assert not bad, bad
    lr = w.info['config']['lr']
    for n in zero_init:
        assert np.abs(ex.read(n) - r['buffers'][names.index(n)]).max() <= 2.0 * lr + 1e-7, n
    ex.close()


def test_eight_mlps_two_steps():
    from kvm_amd.workloads import mlp
    print('8 MLPs, 2 steps', flush=True)
    w = mlp.build(mlp.MLPConfig(steps=2))
    lb, names, init = _prepare(w)
    ex = _device(w, lb)
    check_schedule(ex, lb)
    r = oracle.run(lb, init, threads=THREADS)
    bad = compare_run(ex, lb.metadata, r, tol_f32=TOL_PRECISE)
    assert not bad, bad
    for i in range(8):
        got, want = ex.read(f'm{i}.loss')[0], r['buffers'][names.index(f'm{i}.loss')][0]
        assert abs(got - want) <= 1e-4 * abs(want), (i, got, want)
    ex.close()
