"""The train + serve demo used by the manifest-runner tests: one weight matrix trained by SGD steps that publish
version variable `w`, and serving passes that each read one version of it (reference: the demo's train / serve
admissions on versioned weights, README.md:236-253 of the reference)."""
from kvm_amd.manifest import Demo

N = 8


def _spec(bufs, tasks, variables=()):
    s = {'buffers': bufs, 'graphs': [{'name': 'g', 'tasks': tasks}]}
    if variables:
        s['variables'] = list(variables)
    return s


def build(root, steps=3, probe=False):
    """probe: one more workload, admitted after the last serve pass and compiled on demand by the runner from its
    workload file, with an input read from a data file: Z = P W on the final weights."""
    d = Demo(root)
    d.workload('train', variables=['w'], cls='train')
    d.workload('serve', variables=['w'], cls='serve')
    W = {'name': 'W', 'rows': N, 'cols': N, 'dtype': 'f32', 'init': {'kind': 'seeded', 'seed': 11, 'scale': 0.5, 'dist': 'normal'}}
    G = {'name': 'G', 'rows': N, 'cols': N, 'dtype': 'f32', 'init': {'kind': 'seeded', 'seed': 12, 'scale': 1.0, 'dist': 'normal'}}
    X = {'name': 'X', 'rows': 4, 'cols': N, 'dtype': 'f32', 'init': {'kind': 'seeded', 'seed': 13, 'scale': 1.0, 'dist': 'normal'}}
    d.bundle('train', 'train', _spec([W, G], [{'id': 'sgd', 'op': 'sgd', 'args': {'w': 'W', 'g': 'G', 'lr': 0.1, 'n': N * N},
                                                 'publishes': 'w'}], ['w']), {'w': 0})
    Ys = [{'name': f'Y{k}', 'rows': 4, 'cols': N, 'dtype': 'f32', 'init': {'kind': 'fill', 'value': 0}} for k in range(1, steps + 1)]
    for k in range(1, steps + 1):   # every serve bundle declares all outputs: the first one initialises them
        d.bundle('serve', f'serve{k}', _spec([W, X, *Ys], [
            {'id': 'mm', 'op': 'matmul_tile', 'args': {'a': 'X', 'b': 'W', 'out': f'Y{k}', 'bias': None, 'res': None, 'pre': None,
                                                       'm0': 0, 'n0': 0, 'M': 4, 'N': N, 'K': N, 'flags': 0, 'alpha': 1.0}}]))
    d.buffer('W', N, N, 'f32', 'train')
    d.buffer('G', N, N, 'f32', 'train')
    d.buffer('X', 4, N, 'f32', 'serve')
    for k in range(1, steps + 1):
        d.buffer(f'Y{k}', 4, N, 'f32', 'serve')
    prev = None
    for k in range(1, steps + 1):   # train k publishes w = k; serve k runs on exactly that version, before train k + 1
        d.admission(f'train{k}', 'train', bundle_dir='train' if k == 1 else None, after=[prev] if prev else (),
                    base_versions={'w': k - 1}, publishes={'w': k})
        d.admission(f'serve{k}', 'serve', bundle_dir=f'serve{k}', when=[('w', k, k)])
        prev = f'serve{k}'
    if probe:
        import numpy as np
        (d.root / 'data').mkdir(exist_ok=True)
        np.arange(4 * N, dtype=np.float32).reshape(4, N).__mul__(np.float32(0.125)).tofile(d.root / 'data' / 'p.bin')
        P = {'name': 'P', 'rows': 4, 'cols': N, 'dtype': 'f32', 'init': {'kind': 'file', 'path': 'p.bin'}}
        Z = {'name': 'Z', 'rows': 4, 'cols': N, 'dtype': 'f32', 'init': {'kind': 'fill', 'value': 0}}
        d.workload('probe', variables=['w'], cls='serve')
        d.workload_file('workloads/probe.json', _spec([W, P, Z], [
            {'id': 'mm', 'op': 'matmul_tile', 'reads': [{'var': 'w', 'policy': 'at_least', 'version': steps}],
             'args': {'a': 'P', 'b': 'W', 'out': 'Z', 'bias': None, 'res': None, 'pre': None,
                      'm0': 0, 'n0': 0, 'M': 4, 'N': N, 'K': N, 'flags': 0, 'alpha': 1.0}}], ['w']))
        d.buffer('P', 4, N, 'f32', 'probe')
        d.buffer('Z', 4, N, 'f32', 'probe')
        d.admission('probe1', 'probe', after=[prev], base_versions={'w': steps}, compile=('workloads/probe.json', 'data'))
    d.classes = {'train': {'weight': 1}, 'serve': {'weight': 4, 'urgent_us': 500}}
    return d.write()
