"""Qwen3-8B-shape greedy decode step as a task graph (no generator exists in the reference).

One step: embed the previous token -> 36 x [RMSNorm -> q, k, v projections -> per-head q/k RMSNorm + RoPE + KV append +
split-context attention (attn_decode_part_qkn: the norm inside the attention tasks) -> merge -> o projection + residual -> RMSNorm -> gate / up ->
SwiGLU -> down projection + residual] -> final RMSNorm -> untied LM head -> argmax -> the token buffer; then the cached
length grows by one. Re-running the graph decodes the next token (the token buffer and lens carry over).

Batch 1 uses the registry's one-row decode GEMV (gemv_bf16, RMSNorm / SwiGLU prologues fused) exactly as the
reference's serving passes lay it out (reference: frontend/mvmfe/serve.py:243-315). Batch > 1 uses this executor's
gemv_bf16_rows (op 301): the weights are streamed once for all sequences, with the RMSNorm prologue fused (statistics
per sequence) and SwiGLU as small streaming tasks writing bf16 activations.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, asdict

from . import Builder, Workload, split


@dataclass
class Qwen3Config:
    layers: int = 36
    hidden: int = 4096
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 12288
    vocab: int = 151936
    ctx: int = 4096            # tokens already in the KV cache
    batch: int = 1
    max_new: int = 64          # cache room for this many decode steps
    theta: float = 1e6
    eps: float = 1e-6
    seed: int = 1234
    splits: int = 0            # attention splits per (sequence, kv head); 0 = auto (256 part tasks)
    tasks_per_phase: int = 256
    fused_norm: bool = True    # q / k head norm inside the attention tasks (op 306) where its shapes allow
    fused_merge: bool = True   # with fused_norm: the last split of each kv head merges its query heads (op 310)
    silu_tasks: int = 0        # batch > 1: SwiGLU tasks per layer; 0 = tasks_per_phase / 2 (measured best of 32-256)
    fused_swiglu: bool = True  # batch > 1: gate, up and silu(g) u as one GEMV phase (op 311) writing bf16 h for the down
    #                            projection, in place of the gate / up GEMVs and the silu_mul phase (batch 8: 7.19 vs 7.27
    #                            ms). Batch 1 keeps the gate / up GEMVs (inlined in the static kernel; op 311 runs through
    #                            the dispatcher there: 5.03 vs 4.87 ms).
    head_tasks: int = 0        # LM-head GEMV tasks; 0 = 2 x tasks_per_phase (measured: 512 best of 256-2048 at 256 per phase)

    @staticmethod
    def tiny(batch=1, **kw):
        base = dict(layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128, ffn=512, vocab=1000, ctx=37, batch=batch, max_new=4,
                    tasks_per_phase=16)
        base.update(kw)
        return Qwen3Config(**base)


def weight_elems(c: Qwen3Config) -> int:
    D, hd = c.hidden, c.head_dim
    per_layer = (c.heads * hd) * D + 2 * (c.kv_heads * hd) * D + D * (c.heads * hd) + 3 * c.ffn * D
    return c.layers * per_layer + c.vocab * D


def build(c: Qwen3Config) -> Workload:
    b = Builder(c.seed)
    B, D, H, Hkv, hd, F, V = c.batch, c.hidden, c.heads, c.kv_heads, c.head_dim, c.ffn, c.vocab
    Tmax = c.ctx + c.max_new
    S = c.splits or max(1, 256 // (B * Hkv))   # B * Hkv * S = 256 part tasks: one round of the workers
    rows_mode = B > 1
    # ---- buffers
    b.values('tok', [(7919 * (i + 1)) % V for i in range(B)], B, 1, 'i32')
    b.values('lens', [c.ctx] * B, B, 1, 'i32')
    b.normal('wte', V, D, 'f32')
    b.fill('x', B, D)
    b.fill('q', B, H * hd)
    b.fill('k', B, Hkv * hd)
    b.fill('v', B, Hkv * hd)
    b.fill('part', B * S * H, hd + 2)
    b.fill('att', B, H * hd, 'bf16' if rows_mode else 'f32')
    b.fill('g', B, F)
    b.fill('u', B, F)
    if rows_mode:
        b.fill('xn', B, D, 'bf16')
        b.fill('rstd', B)
    if rows_mode:
        b.fill('h', B, F, 'bf16')
    b.fill('logits', B, V)
    fused_norm = c.fused_norm and hd == 128 and H // Hkv in (1, 2, 4, 8)      # op 306's streaming-path shapes
    fused_merge = fused_norm and c.fused_merge
    if fused_merge:
        b.fill('acnt', B * Hkv, 1, 'i32')       # split counts of op 310 (0 between steps; shared by the layers in turn)
    for l in range(c.layers):
        b.fill(f'ln1.{l}', D, value=1.0)
        b.fill(f'ln2.{l}', D, value=1.0)
        b.fill(f'qn.{l}', hd, value=1.0)
        b.fill(f'kn.{l}', hd, value=1.0)
        b.normal(f'wq.{l}', H * hd, D, 'bf16')
        b.normal(f'wk.{l}', Hkv * hd, D, 'bf16')
        b.normal(f'wv.{l}', Hkv * hd, D, 'bf16')
        b.normal(f'wo.{l}', D, H * hd, 'bf16')
        b.normal(f'wg.{l}', F, D, 'bf16')
        b.normal(f'wu.{l}', F, D, 'bf16')
        b.normal(f'wd.{l}', D, F, 'bf16')
        b.normal(f'kc.{l}', B * Hkv * Tmax, hd, 'bf16', scale=1.0)
        b.normal(f'vc.{l}', B * Hkv * Tmax, hd, 'bf16', scale=1.0)
    b.fill('lnf', D, value=1.0)
    b.normal('whead', V, D, 'bf16')

    def proj(after, x, w, out, N, K, parts, pro=0, gamma=None, x2=None, res=None):
        """Tasks computing out[:, 0:N] = prologue(x) @ w^T (+ res)."""
        ts = []
        if rows_mode:
            for lo, hi in split(N // 16, max(1, min(parts, N // 16))):
                ts.append(b.task('gemv_bf16_rows', after=after, x=x, x2=x2, gamma=gamma, w=w, out=out, res=res, n0=16 * lo, n1=16 * hi,
                                 K=K, M=B, pro=pro, eps=c.eps))
        else:
            for lo, hi in split(N, parts):
                ts.append(b.task('gemv_bf16', after=after, x=x, x2=x2, gamma=gamma, w=w, out=out, res=res, n0=lo, n1=hi, K=K, pro=pro,
                                 eps=c.eps))
        return ts

    P = c.tasks_per_phase
    prev = [b.task('embedding_fwd', ids='tok', wte='wte', wpe=None, out='x', r0=0, r1=B, T=1, d=D)]
    last_parts = []
    for l in range(c.layers):
        nq, nkv = H * hd, Hkv * hd
        tot = nq + 2 * nkv
        pk = max(1, round(P * nkv / tot))
        pq = max(1, P - 2 * pk)                 # q, k, v together: one round of P tasks
        if rows_mode:   # the RMSNorm of every sequence is the GEMV's prologue (statistics per row, then the rows staged)
            prev = b.join(prev, P)
            tq = proj(prev, 'x', f'wq.{l}', 'q', nq, D, pq, pro=1, gamma=f'ln1.{l}')
            tk = proj(prev, 'x', f'wk.{l}', 'k', nkv, D, pk, pro=1, gamma=f'ln1.{l}')
            tv = proj(prev, 'x', f'wv.{l}', 'v', nkv, D, pk, pro=1, gamma=f'ln1.{l}')
        else:
            tq = proj(prev, 'x', f'wq.{l}', 'q', nq, D, pq, pro=1, gamma=f'ln1.{l}')
            tk = proj(prev, 'x', f'wk.{l}', 'k', nkv, D, pk, pro=1, gamma=f'ln1.{l}')
            tv = proj(prev, 'x', f'wv.{l}', 'v', nkv, D, pk, pro=1, gamma=f'ln1.{l}')
        kw = dict(q='q', kc=f'kc.{l}', vc=f'vc.{l}', lens='lens', part='part', knew='k', vnew='v', S=S, H=H, Hkv=Hkv, hd=hd, Tmax=Tmax,
                  scale=1.0 / math.sqrt(hd), theta=c.theta, flags=1)
        if fused_norm:   # q / k per-head RMSNorm inside the attention tasks (op 306 = op 300 on q and the new key, then op 135)
            after, op = b.join(tq + tk + tv, B * Hkv * S), 'attn_decode_part_qkn'
            kw.update(qgamma=f'qn.{l}', kgamma=f'kn.{l}', eps=c.eps)
            if fused_merge:
                op = 'attn_decode_part_merge'
                kw.update(o='att', cnt='acnt')
        else:
            hq = b.task('head_rmsnorm', after=tq, x='q', gamma=f'qn.{l}', out='q', r0=0, r1=B, H=H, hd=hd, eps=c.eps)
            hk = b.task('head_rmsnorm', after=tk, x='k', gamma=f'kn.{l}', out='k', r0=0, r1=B, H=Hkv, hd=hd, eps=c.eps)
            after, op = [hq, hk, *b.join(tv, 2 * S)], 'attn_decode_part'
        parts = []
        for bb in range(B):
            parts.append([b.task(op, after=after, b=bb, kvh=kh, s=s, **kw) for kh in range(Hkv) for s in range(S)])
        last_parts = [t for pb in parts for t in pb]
        merges = []
        if fused_merge:
            merges = b.join(last_parts, P)
        else:
            for bb in range(B):
                nm = max(1, H // B)             # one merge task per head (batch 1): short, parallel
                for h0, h1 in split(H, nm):
                    merges.append(b.task('attn_decode_merge', after=parts[bb], part='part', o='att', b=bb, h0=h0, h1=h1, S=S, H=H, hd=hd))
        to = proj(merges, 'att', f'wo.{l}', 'x', D, H * hd, P, res='x')
        if rows_mode and c.fused_swiglu and F % 16 == 0 and D % 256 == 0 and B <= 16:
            # gate, up and silu(g) u in one phase of P tasks (op 311, 16-row blocks), h in bf16 for the down projection
            oj = b.join(to, 2 * P)
            sw = [b.task('gemv_swiglu', after=oj, x='x', gamma=f'ln2.{l}', wg=f'wg.{l}', wu=f'wu.{l}', out='h', n0=16 * lo, n1=16 * hi,
                         K=D, M=B, eps=c.eps) for lo, hi in split(F // 16, max(1, min(P, F // 16)))]
            td = proj(b.join(sw, P), 'h', f'wd.{l}', 'x', D, F, P, res='x')
            prev = td if len(td) <= 256 else b.join(td, P)
        elif rows_mode:
            oj = b.join(to, 2 * P)
            tg = proj(oj, 'x', f'wg.{l}', 'g', F, D, P // 2, pro=1, gamma=f'ln2.{l}')     # gate and up: one round of P tasks
            tu = proj(oj, 'x', f'wu.{l}', 'u', F, D, P // 2, pro=1, gamma=f'ln2.{l}')
            sm = [b.task('silu_mul_fwd', after=tg + tu, gate='g', up='u', out='h', e0=lo * 8, e1=hi * 8)
                  for lo, hi in split(B * F // 8, max(1, c.silu_tasks or P // 2))]
            td = proj(sm, 'h', f'wd.{l}', 'x', D, F, P, res='x')
            prev = td if len(td) <= 256 else b.join(td, P)
        else:
            oj = b.join(to, 2 * P)
            tg = proj(oj, 'x', f'wg.{l}', 'g', F, D, P // 2, pro=1, gamma=f'ln2.{l}')     # gate and up: one round of P tasks
            tu = proj(oj, 'x', f'wu.{l}', 'u', F, D, P // 2, pro=1, gamma=f'ln2.{l}')
            gj = b.join(tg + tu, P)
            td = proj(gj, 'g', f'wd.{l}', 'x', D, F, P, pro=2, x2='u', res='x')
            prev = b.join(td, P)
    head_parts = c.head_tasks or 2 * P
    if rows_mode:
        rf = [b.task('rmsnorm_fwd', after=prev, x='x', gamma='lnf', out='xn', rstd='rstd', r0=0, r1=B, d=D, eps=c.eps)]
        th = proj(rf, 'xn', 'whead', 'logits', V, D, head_parts)
    else:
        th = proj(prev, 'x', 'whead', 'logits', V, D, head_parts, pro=1, gamma='lnf')
    for bb in range(B):
        b.task('argmax', after=th, logits='logits', out='tok', r0=bb, r1=bb + 1, V=V)
    b.task('counter_inc', after=last_parts, x='lens', i0=0, i1=B, delta=1)
    info = {'config': asdict(c), 'weight_bytes': 2 * weight_elems(c),
            'kv_bytes_per_step': c.layers * 2 * B * Hkv * (c.ctx + 1) * hd * 2, 'splits': S}
    return Workload(b.spec('decode'), b.init_override, info)
