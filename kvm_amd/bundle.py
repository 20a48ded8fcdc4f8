"""Reading a task bundle (reference format: runtime/compile_workload.py:694-713) and materialising buffer contents."""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import initgen

DT_F32, DT_I32, DT_BF16 = 0, 1, 2


@dataclass
class LoadedBundle:
    metadata: dict
    tasks: np.ndarray       # int32 [n, 16]
    succ: np.ndarray        # int32 [edges]
    args: np.ndarray        # int32 [words]
    root: Path | None = None

    @property
    def buffers(self):
        return self.metadata['buffers']

    @property
    def ntasks(self):
        return self.tasks.shape[0]


def load(src) -> LoadedBundle:
    """`src` is a bundle directory or a kvm_amd.compiler.Bundle."""
    if hasattr(src, 'metadata') and hasattr(src, 'tasks') and isinstance(src.tasks, (bytes, bytearray)):
        return LoadedBundle(src.metadata, np.frombuffer(src.tasks, np.int32).reshape(-1, 16).copy(),
                            np.frombuffer(src.successors, np.int32).copy(), np.frombuffer(src.args, np.int32).copy(),
                            getattr(src, 'data_dir', None))
    d = Path(src)
    meta = json.loads((d / 'metadata.json').read_text())
    return LoadedBundle(meta, np.fromfile(d / 'tasks.bin', np.int32).reshape(-1, 16), np.fromfile(d / 'successors.bin', np.int32),
                        np.fromfile(d / 'args.bin', np.int32), d)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16 value, as float32 (inf/nan kept)."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32)
    # uint32 arithmetic: only non-finite inputs (|u| near 0xFFFFFFFF) can wrap, and those are kept as they are below
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)).view(np.float32)
    return np.where(np.isfinite(x), r, x)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 values (already bf16-representable or not) -> uint16 bf16 storage, nearest even."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def materialize(buf: dict, root: Path | None = None) -> np.ndarray:
    """Initial contents of one metadata buffer entry: float32 for f32/bf16 (bf16 as widened values), int32 for i32."""
    n = buf['rows'] * buf['cols']
    init, dt = buf['init'], buf['dtype']
    np_dt = np.int32 if dt == DT_I32 else np.float32
    k = init['kind']
    if k == 'fill':
        return np.zeros(n, np_dt) if init['value'] == 0 else np.full(n, init['value'], np_dt)
    if k == 'values':
        return np.asarray(init['values'], np_dt)
    if k == 'seeded':   # bf16 buffers (an executor-side override, not a bundle init): rounded once to bf16
        v = initgen.seeded(init['seed'], n, init['draws'], init['bias'], init['coef'])
        return bf16_round(v) if dt == DT_BF16 else v
    if k == 'file':
        raw = (Path(root) / init['path']).read_bytes()
        if dt == DT_BF16:
            return bits_to_f32(np.frombuffer(raw, np.uint16))
        return np.frombuffer(raw, np_dt).copy()
    raise ValueError(f'unknown init kind {k!r}')
