"""An fp64 numpy model of the GPT training step the generator builds (kvm_amd/workloads/gpt.py), for tests.

It takes the graph's own initial buffers (the f32 master weights, token ids and targets) and computes the same step
with no rounding anywhere: float64 throughout, no bf16 copies of the weights, no bf16 activation stores. The step is
the graph's: embedding (wte[ids] + wpe[t]), pre-LayerNorm blocks (eps 1e-5, biased variance) with causal softmax
attention (scale 1/sqrt(hd)) and a tanh-GELU MLP, final LayerNorm, tied head (logits = hf wte^T), mean
cross-entropy over every token, the backward pass, the global gradient-norm clip (scale min(1, clip / (norm + 1e-6)))
and one AdamW step (bias-corrected, decoupled weight decay on the matrices only), following the reference's operator
definitions (runtime/ref_gpt.py: LayerNorm 107-173, GELU 27-33, attention 279-364, cross entropy 414-453, AdamW
457-471, gradient norm 474-482). The reference CPU path (the oracle) rounds like the reference does; the distance
between the two is the reference's own deviation from an fp64 run, from which the full-depth GPT tolerances are
derived (twice that deviation).
"""
from __future__ import annotations

import numpy as np

GELU_C = np.sqrt(2.0 / np.pi)


def _ln(x, g, b, eps=1e-5):
    mu = x.mean(-1, keepdims=True)
    xc = x - mu
    rs = 1.0 / np.sqrt((xc * xc).mean(-1, keepdims=True) + eps)
    xh = xc * rs
    return xh * g + b, xh, rs


def _ln_bwd(dy, xh, rs, g):
    gs = dy * g
    d = xh.shape[-1]
    dx = rs * (gs - gs.sum(-1, keepdims=True) / d - xh * (gs * xh).sum(-1, keepdims=True) / d)
    return dx, (dy * xh).sum(0), dy.sum(0)


def _gelu(u):
    t = np.tanh(GELU_C * (u + 0.044715 * u ** 3))
    return 0.5 * u * (1.0 + t), t


def _gelu_grad(u, t):
    return 0.5 * (1.0 + t) + 0.5 * u * (1.0 - t * t) * GELU_C * (1.0 + 3.0 * 0.044715 * u * u)


def step(c, buf):
    """One training step of config `c` (the generator's GPTConfig) on the named initial buffers `buf` (float arrays
    as the executor holds them). Returns dict(loss, logits [N, V], grads {param: array}, params {param: array after
    AdamW}) in float64."""
    L, d, H, T, V, F, B = c.layers, c.d, c.heads, c.T, c.vocab, c.ffn, c.batch
    N, hd = B * T, d // H
    P = {}

    def p(name, shape):
        P[name] = np.asarray(buf[name], np.float64).reshape(shape)
        return P[name]

    wte, wpe = p('wte', (V, d)), p('wpe', (T, d))
    layers = []
    for l in range(L):
        layers.append({k: p(f'{k}.{l}', s) for k, s in (('wq', (d, d)), ('wk', (d, d)), ('wv', (d, d)), ('wo', (d, d)),
                                                          ('bq', (d,)), ('bk', (d,)), ('bv', (d,)), ('bo', (d,)),
                                                          ('ln1g', (d,)), ('ln1b', (d,)), ('ln2g', (d,)), ('ln2b', (d,)),
                                                          ('w1', (F, d)), ('b1', (F,)), ('w2', (d, F)), ('b2', (d,)))})
    lnfg, lnfb = p('lnfg', (d,)), p('lnfb', (d,))
    ids = np.asarray(buf['ids'], np.int64).ravel()
    tgt = np.asarray(buf['tgt'], np.int64).ravel()
    pos = np.arange(N) % T
    scale = 1.0 / np.sqrt(hd)
    causal = np.tril(np.ones((T, T), bool))

    # ---- forward
    x = wte[ids] + wpe[pos]
    cache = []
    for W in layers:
        h1, xh1, rs1 = _ln(x, W['ln1g'], W['ln1b'])
        q, k, v = h1 @ W['wq'].T + W['bq'], h1 @ W['wk'].T + W['bk'], h1 @ W['wv'].T + W['bv']
        o = np.empty_like(q)
        probs = np.empty((B, H, T, T))
        for b in range(B):
            for h in range(H):
                sl = (slice(b * T, (b + 1) * T), slice(h * hd, (h + 1) * hd))
                s = (q[sl] @ k[sl].T) * scale
                s = np.where(causal, s, -np.inf)
                e = np.exp(s - s.max(-1, keepdims=True))
                pr = e / e.sum(-1, keepdims=True)
                probs[b, h] = pr
                o[sl] = pr @ v[sl]
        xm = o @ W['wo'].T + W['bo'] + x
        h2, xh2, rs2 = _ln(xm, W['ln2g'], W['ln2b'])
        u = h2 @ W['w1'].T + W['b1']
        a, tu = _gelu(u)
        xn = a @ W['w2'].T + W['b2'] + xm
        cache.append((x, h1, xh1, rs1, q, k, v, o, probs, xm, h2, xh2, rs2, u, a, tu))
        x = xn
    hf, xhf, rsf = _ln(x, lnfg, lnfb)
    logits = hf @ wte.T
    m = logits.max(-1, keepdims=True)
    lse = m[:, 0] + np.log(np.exp(logits - m).sum(-1))
    loss = float((lse - logits[np.arange(N), tgt]).mean())

    # ---- backward
    G = {}
    dl = np.exp(logits - lse[:, None])
    dl[np.arange(N), tgt] -= 1.0
    dl /= N
    G['wte'] = dl.T @ hf
    dhf = dl @ wte
    del dl
    dx, G['lnfg'], G['lnfb'] = _ln_bwd(dhf, xhf, rsf, lnfg)
    for l in reversed(range(L)):
        W = layers[l]
        (x0, h1, xh1, rs1, q, k, v, o, probs, xm, h2, xh2, rs2, u, a, tu) = cache[l]
        G[f'w2.{l}'] = dx.T @ a
        G[f'b2.{l}'] = dx.sum(0)
        du = (dx @ W['w2']) * _gelu_grad(u, tu)
        G[f'w1.{l}'] = du.T @ h2
        G[f'b1.{l}'] = du.sum(0)
        dh2 = du @ W['w1']
        dxm, G[f'ln2g.{l}'], G[f'ln2b.{l}'] = _ln_bwd(dh2, xh2, rs2, W['ln2g'])
        dxm += dx
        G[f'wo.{l}'] = dxm.T @ o
        G[f'bo.{l}'] = dxm.sum(0)
        do = dxm @ W['wo']
        dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
        for b in range(B):
            for h in range(H):
                sl = (slice(b * T, (b + 1) * T), slice(h * hd, (h + 1) * hd))
                pr = probs[b, h]
                dv[sl] = pr.T @ do[sl]
                dp = do[sl] @ v[sl].T
                ds = pr * (dp - (dp * pr).sum(-1, keepdims=True))
                dq[sl] = ds @ k[sl] * scale
                dk[sl] = ds.T @ q[sl] * scale
        for nm, dd in (('q', dq), ('k', dk), ('v', dv)):
            G[f'w{nm}.{l}'] = dd.T @ h1
            G[f'b{nm}.{l}'] = dd.sum(0)
        dh1 = dq @ W['wq'] + dk @ W['wk'] + dv @ W['wv']
        dx1, G[f'ln1g.{l}'], G[f'ln1b.{l}'] = _ln_bwd(dh1, xh1, rs1, W['ln1g'])
        dx = dx1 + dxm
    np.add.at(G['wte'], ids, dx)
    G['wpe'] = np.zeros_like(wpe)
    np.add.at(G['wpe'], pos, dx)

    # ---- gradient-norm clip and AdamW (step 1: m = (1 - b1) g, v = (1 - b2) g^2, bias corrections 1 - b^1)
    norm = np.sqrt(sum(float((g * g).sum()) for g in G.values()))
    gs = min(1.0, c.clip / (norm + 1e-6)) if c.clip > 0 else 1.0
    new = {}
    for name, w in P.items():
        g = G[name] * gs
        mh = (1.0 - c.b1) * g / (1.0 - c.b1)
        vh = (1.0 - c.b2) * g * g / (1.0 - c.b2)
        matrix = name.split('.')[0] in ('wte', 'wpe', 'wq', 'wk', 'wv', 'wo', 'w1', 'w2')
        new[name] = w - c.lr * (c.wd if matrix else 0.0) * w - c.lr * mh / (np.sqrt(vh) + c.eps)
    return {'loss': loss, 'logits': logits, 'grads': G, 'params': new, 'norm': norm}


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


# Parameter groups (pooled over layers) for the deviations: a group's relative L2 is taken over all its buffers at once.
def group_of(name: str) -> str:
    return name.split('.')[0]


def deviations(names, bufs, ref, skip_groups=('bk',)):
    """Relative L2 of a run's final buffers (oracle or device: `names` / `bufs` in metadata order) against `ref`
    (this module's step, or another run's `quantities`): the loss (absolute difference), the logits, every gradient
    group and every parameter group after AdamW. The key bias's gradient is zero in exact arithmetic (softmax is
    shift-invariant), so its group is skipped."""
    got = quantities(names, bufs)
    out = {'loss_abs': abs(got['loss'] - ref['loss']), 'logits': rel_l2(got['logits'], ref['logits'])}
    for kind in ('grads', 'params'):
        groups = {}
        for n in ref[kind]:
            if group_of(n) in skip_groups:
                continue
            groups.setdefault(group_of(n), []).append(n)
        for gname, members in sorted(groups.items()):
            a = np.concatenate([np.asarray(got[kind][n], np.float64).ravel() for n in members])
            b = np.concatenate([np.asarray(ref[kind][n], np.float64).ravel() for n in members])
            out[f'{kind[0]}.{gname}'] = rel_l2(a, b)
    return out


def quantities(names, bufs):
    """The step's loss, logits, gradients and updated parameters read from a run's final buffers."""
    get = {n: b for n, b in zip(names, bufs)}
    params = [n[2:] for n in names if n.startswith('d.')]
    return {'loss': float(np.asarray(get['loss']).ravel()[0]), 'logits': np.asarray(get['logits'], np.float64),
            'grads': {p: np.asarray(get[f'd.{p}'], np.float64) for p in params},
            'params': {p: np.asarray(get[p], np.float64) for p in params}}
