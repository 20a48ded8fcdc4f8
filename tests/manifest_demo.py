"""Demo directories for the manifest-runner tests (reference: the frontend's train + serve demos,
frontend/mvmfe/demo.py:120-200).

build(): one weight matrix trained by single SGD steps, each publishing one version of `w`, and serving passes that
each read exactly one version (README.md:236-253 of the reference).

build_windows(): the frontend's training-window shape (demo.py:185-194): training cut into windows of `steps`
steps, window i admitted with base_versions {'weights': 2 * start} and publishes {'weights': 2 * steps} (two
versions per optimizer step: weights_version(n) = 2 n, frontend/mvmfe/train.py:28-30), every window after the first
reusing the first window's bundle moved to its base, and a serving pass on each stable weights version in between.
"""
from kvm_amd.manifest import Demo

N = 8


def _spec(bufs, tasks, variables=()):
    s = {'buffers': bufs, 'graphs': [{'name': 'g', 'tasks': tasks}]}
    if variables:
        s['variables'] = list(variables)
    return s


def _seeded(name, rows, seed, scale=1.0):
    return {'name': name, 'rows': rows, 'cols': N, 'dtype': 'f32', 'init': {'kind': 'seeded', 'seed': seed, 'scale': scale, 'dist': 'normal'}}


def _zeros(name, rows):
    return {'name': name, 'rows': rows, 'cols': N, 'dtype': 'f32', 'init': {'kind': 'fill', 'value': 0}}


def _mm(a, b, out):
    return {'op': 'matmul_tile', 'args': {'a': a, 'b': b, 'out': out, 'bias': None, 'res': None, 'pre': None,
                                          'm0': 0, 'n0': 0, 'M': 4, 'N': N, 'K': N, 'flags': 0, 'alpha': 1.0}}


def build(root, steps=3, probe=False, classes=True):
    """probe: one more workload, admitted after the last serve pass and compiled on demand by the runner from its
    workload file, with an input read from a data file: Z = P W on the final weights."""
    d = Demo(root)
    d.workload('train', variables=['w'], cls='train')
    d.workload('serve', variables=['w'], cls='serve')
    W, G, X = _seeded('W', N, 11, 0.5), _seeded('G', N, 12), _seeded('X', 4, 13)
    d.bundle('train', 'train', _spec([W, G], [{'id': 'sgd', 'op': 'sgd', 'args': {'w': 'W', 'g': 'G', 'lr': 0.1, 'n': N * N},
                                                 'publishes': 'w'}], ['w']), {'w': 0})
    Ys = [_zeros(f'Y{k}', 4) for k in range(1, steps + 1)]
    for k in range(1, steps + 1):   # every serve bundle declares all outputs: the first one initialises them
        d.bundle('serve', f'serve{k}', _spec([W, X, *Ys], [dict(id='mm', **_mm('X', 'W', f'Y{k}'))]))
    d.buffer('W', N, N, 'f32', 'train')
    d.buffer('G', N, N, 'f32', 'train')
    d.buffer('X', 4, N, 'f32', 'serve')
    for k in range(1, steps + 1):
        d.buffer(f'Y{k}', 4, N, 'f32', 'serve')
    prev = None
    for k in range(1, steps + 1):   # train k moves w from k - 1 to k; serve k runs on exactly that version, before train k + 1
        d.admission(f'train{k}', 'train', bundle_dir='train' if k == 1 else None, after=[prev] if prev else (),
                    base_versions={'w': k - 1}, publishes={'w': 1})
        d.admission(f'serve{k}', 'serve', bundle_dir=f'serve{k}', when=[('w', k, k)])
        prev = f'serve{k}'
    if probe:
        import numpy as np
        (d.root / 'data').mkdir(exist_ok=True)
        np.arange(4 * N, dtype=np.float32).reshape(4, N).__mul__(np.float32(0.125)).tofile(d.root / 'data' / 'p.bin')
        P = {'name': 'P', 'rows': 4, 'cols': N, 'dtype': 'f32', 'init': {'kind': 'file', 'path': 'p.bin'}}
        d.workload('probe', variables=['w'], cls='serve')
        probe_mm = dict(id='mm', reads=[{'var': 'w', 'policy': 'at_least', 'version': steps}], **_mm('P', 'W', 'Z'))
        d.workload_file('workloads/probe.json', _spec([W, P, _zeros('Z', 4)], [probe_mm], ['w']))
        d.buffer('P', 4, N, 'f32', 'probe')
        d.buffer('Z', 4, N, 'f32', 'probe')
        d.admission('probe1', 'probe', after=[prev], base_versions={'w': steps}, compile=('workloads/probe.json', 'data'))
    if classes:
        d.classes = {'train': {'weight': 1}, 'serve': {'weight': 4, 'urgent_us': 500}}
    return d.write()


def build_windows(root, windows=3, steps=2, lr=0.05):
    """Training in `windows` windows of `steps` optimizer steps. A step publishes `weights` twice: the first SGD task
    updates W1, the second W2 (so the weights are stable at even versions). serve_s{k} reads the stable weights after
    k steps, exactly (when weights in [2k, 2k]), for k = 0, steps, ..., windows * steps; each window waits for the
    serving pass before it (the exact policy's barrier, demo.py:263-266)."""
    d = Demo(root)
    d.workload('train', variables=['weights'], cls='train')
    d.workload('serve', variables=['weights'], cls='serve')
    W1, W2, G1, G2, X = _seeded('W1', N, 21, 0.5), _seeded('W2', N, 22, 0.5), _seeded('G1', N, 23), _seeded('G2', N, 24), _seeded('X', 4, 25)
    tasks, last = [], None
    for j in range(steps):
        for w, g in (('W1', 'G1'), ('W2', 'G2')):
            t = {'id': f'{w.lower()}_{j}', 'op': 'sgd', 'args': {'w': w, 'g': g, 'lr': lr, 'n': N * N}, 'publishes': 'weights'}
            if last:
                t['after'] = [last]
            tasks.append(t)
            last = t['id']
    d.bundle('train', 'train_window', _spec([W1, W2, G1, G2], tasks, ['weights']), {'weights': 0})
    points = list(range(0, windows * steps + 1, steps))
    outs = [_zeros(f'Y{k}', 4) for k in points] + [_zeros(f'Z{k}', 4) for k in points]
    for k in points:
        d.bundle('serve', f'serve_s{k}', _spec([W1, W2, X, *outs], [dict(id='y', **_mm('X', 'W1', f'Y{k}')),
                                                                     dict(id='z', **_mm('X', 'W2', f'Z{k}'))]))
    for name in ('W1', 'W2', 'G1', 'G2'):
        d.buffer(name, N, N, 'f32', 'train')
    d.buffer('X', 4, N, 'f32', 'serve')
    for k in points:
        d.buffer(f'Y{k}', 4, N, 'f32', 'serve')
        d.buffer(f'Z{k}', 4, N, 'f32', 'serve')
    d.admission('serve_s0', 'serve', bundle_dir='serve_s0', when=[('weights', 0, 0)])
    for i in range(windows):
        start = i * steps
        d.admission(f'train_w{i}', 'train', bundle_dir='train_window' if i == 0 else None,
                    after=[f'train_w{i - 1}', f'serve_s{start}'] if i else ['serve_s0'],
                    base_versions={'weights': 2 * start}, publishes={'weights': 2 * steps})
        k = start + steps
        d.admission(f'serve_s{k}', 'serve', bundle_dir=f'serve_s{k}', when=[('weights', 2 * k, 2 * k)])
    return d.write()
