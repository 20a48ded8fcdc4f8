"""An fp64 numpy model of the Qwen3-shape decode step the generator builds (kvm_amd/workloads/qwen3.py), for tests.

It takes the graph's own initial buffers (the bf16 weights and KV caches as values) and computes the same decode step
with no rounding anywhere: float64 throughout, no bf16 activation stores, RoPE angles in float64. The reference CPU
path (the oracle) rounds like the reference does (f32 per store, bf16 where the graph stores bf16, f32 RoPE angles);
the distance between the two is the reference's own deviation from an fp64 run, from which the decode tolerances
are derived (twice that deviation).
"""
from __future__ import annotations

import numpy as np


def _rms(x, g, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * g


def _rope(x, pos, theta):
    """x [..., hd]: pairs (i, i + hd/2) rotated by pos * theta^(-2i/hd)."""
    hd = x.shape[-1]
    half = hd // 2
    ang = pos * theta ** (-(2.0 * np.arange(half)) / hd)
    c, s = np.cos(ang), np.sin(ang)
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], -1)


def _mv(x, w, rows, cols, chunk=8192):
    """x [B, cols] float64 times w^T for a [rows, cols] float32 weight, converted to float64 a row chunk at a time."""
    w = np.asarray(w).reshape(rows, cols)
    out = np.empty((x.shape[0], rows))
    for r0 in range(0, rows, chunk):
        out[:, r0:r0 + chunk] = x @ w[r0:r0 + chunk].astype(np.float64).T
    return out


def decode_step(c, buf):
    """One greedy decode step of config `c` (layers, widths as the generator's Qwen3Config) on the named initial
    buffers `buf` (float arrays as the executor holds them). Returns dict(logits [B, V], x [B, D] final residual,
    tok [B], knew / vnew per layer [B, Hkv, hd] (the rows appended to the caches))."""
    B, D, H, Hkv, hd, F, V = c.batch, c.hidden, c.heads, c.kv_heads, c.head_dim, c.ffn, c.vocab
    G = H // Hkv
    Tmax = c.ctx + c.max_new
    f = lambda n: np.asarray(buf[n], np.float64)
    tok = np.asarray(buf['tok'], np.int64).ravel()
    lens = np.asarray(buf['lens'], np.int64).ravel()
    x = np.asarray(buf['wte']).reshape(V, D)[tok].astype(np.float64)   # [B, D]
    out = {'knew': [], 'vnew': []}
    for l in range(c.layers):
        xn = _rms(x, f(f'ln1.{l}'), c.eps)
        q = _mv(xn, buf[f'wq.{l}'], H * hd, D).reshape(B, H, hd)
        k = _mv(xn, buf[f'wk.{l}'], Hkv * hd, D).reshape(B, Hkv, hd)
        v = _mv(xn, buf[f'wv.{l}'], Hkv * hd, D).reshape(B, Hkv, hd)
        q = _rms(q, f(f'qn.{l}'), c.eps)
        k = _rms(k, f(f'kn.{l}'), c.eps)
        kc = np.asarray(buf[f'kc.{l}']).reshape(B, Hkv, Tmax, hd)
        vc = np.asarray(buf[f'vc.{l}']).reshape(B, Hkv, Tmax, hd)
        att = np.zeros((B, H, hd))
        kn_l, vn_l = np.zeros((B, Hkv, hd)), np.zeros((B, Hkv, hd))
        for bb in range(B):
            p = int(lens[bb])
            qr = _rope(q[bb], float(p), c.theta)                       # [H, hd]
            kr = _rope(k[bb], float(p), c.theta)                       # [Hkv, hd]
            kn_l[bb], vn_l[bb] = kr, v[bb]
            for h in range(H):
                kh = h // G
                keys = np.concatenate([kc[bb, kh, :p].astype(np.float64), kr[kh][None]], 0)
                vals = np.concatenate([vc[bb, kh, :p].astype(np.float64), v[bb, kh][None]], 0)
                s = keys @ qr[h] / np.sqrt(hd)
                w = np.exp(s - s.max())
                att[bb, h] = (w / w.sum()) @ vals
        out['knew'].append(kn_l)
        out['vnew'].append(vn_l)
        x = x + _mv(att.reshape(B, H * hd), buf[f'wo.{l}'], D, H * hd)
        xn = _rms(x, f(f'ln2.{l}'), c.eps)
        g = _mv(xn, buf[f'wg.{l}'], F, D)
        u = _mv(xn, buf[f'wu.{l}'], F, D)
        x = x + _mv(g / (1.0 + np.exp(-g)) * u, buf[f'wd.{l}'], D, F)
    xn = _rms(x, f('lnf'), c.eps)
    logits = _mv(xn, buf['whead'], V, D)
    out.update({'logits': logits, 'x': x, 'tok': logits.argmax(-1)})
    return out


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def graph_outputs(c, names, bufs):
    """The same quantities read from a run's final buffers (oracle or device): logits, x, tok, new cache rows."""
    B, Hkv, hd = c.batch, c.kv_heads, c.head_dim
    Tmax = c.ctx + c.max_new
    get = lambda n: np.asarray(bufs[names.index(n)])
    out = {'logits': get('logits').reshape(B, c.vocab).astype(np.float64), 'x': get('x').reshape(B, c.hidden).astype(np.float64),
           'tok': get('tok').ravel().astype(np.int64), 'knew': [], 'vnew': []}
    for l in range(c.layers):
        kc = get(f'kc.{l}').reshape(B, Hkv, Tmax, hd)
        vc = get(f'vc.{l}').reshape(B, Hkv, Tmax, hd)
        out['knew'].append(kc[:, :, c.ctx].astype(np.float64))
        out['vnew'].append(vc[:, :, c.ctx].astype(np.float64))
    return out


def deviations(got, ref):
    """Relative L2 distances per quantity (new cache rows over all layers together)."""
    return {'logits': rel_l2(got['logits'], ref['logits']), 'x': rel_l2(got['x'], ref['x']),
            'knew': rel_l2(np.stack(got['knew']), np.stack(ref['knew'])), 'vnew': rel_l2(np.stack(got['vnew']), np.stack(ref['vnew']))}
