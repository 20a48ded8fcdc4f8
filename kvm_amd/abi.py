"""Task ABI and operator registries, read from the C headers in ``include/`` so Python and the HIP executor share one table.

The registry line format ``X(name, id, "arg:type,...")`` and the descriptor layout are the reference's interface
(reference: runtime/abi.py:52-133, include/mvm_task_abi.h:11-30); this module is this project's own reader of them.
"""
from __future__ import annotations

import re
import struct
from dataclasses import dataclass
from functools import lru_cache
from pathlib import Path

INCLUDE_DIR = Path(__file__).resolve().parents[1] / 'include'
ABSENT_BUF = -1
NO_VAR = -1
ABI_VERSION = 2
EXT_ID_MIN = 300          # ids of this executor's own pack (mvm_ops_kvm.def); not in the reference's registry
DESC_FIELDS = ('op_id', 'succ_off', 'succ_cnt', 'indegree', 'priority', 'deadline_us', 'args_off', 'args_words',
               'wait_var', 'wait_ver', 'pub_var', 'pub_ver', 'workload_id', 'flags', 'reserved0', 'reserved1')
DESC = struct.Struct('<16i')

_LINE = re.compile(r'^X\(\s*(\w+)\s*,\s*(\d+)\s*,\s*"([^"]*)"\s*\)')
_INC = re.compile(r'^\s*#\s*include\s+"([^"]+\.def)"', re.M)


class AbiError(RuntimeError):
    pass


@dataclass(frozen=True)
class Arg:
    name: str
    type: str          # 'buf' | 'i32' | 'f32'
    optional: bool = False


@dataclass(frozen=True)
class Op:
    name: str
    id: int
    args: tuple

    @property
    def arity(self) -> int:
        return len(self.args)

    def index(self, arg: str) -> int:
        for i, a in enumerate(self.args):
            if a.name == arg:
                return i
        raise KeyError(f'{self.name} has no argument {arg!r}')


def _parse_sig(sig: str, where: str) -> tuple:
    out = []
    for item in (s.strip() for s in sig.split(',')):
        if not item:
            continue
        name, _, typ = item.partition(':')
        opt = typ == 'buf?'
        typ = 'buf' if opt else typ
        if typ not in ('buf', 'i32', 'f32') or not name.isidentifier():
            raise AbiError(f'{where}: bad argument {item!r}')
        out.append(Arg(name, typ, opt))
    if len({a.name for a in out}) != len(out):
        raise AbiError(f'{where}: duplicate argument name')
    return tuple(out)


@lru_cache(maxsize=None)
def load_ops(include_dir: str = str(INCLUDE_DIR)) -> dict:
    """name -> Op for every registry file mvm_ops_list.inc includes, in its order."""
    inc = Path(include_dir)
    files = _INC.findall((inc / 'mvm_ops_list.inc').read_text())
    ops, ids = {}, {}
    for f in files:
        for ln, line in enumerate((inc / f).read_text().splitlines(), 1):
            if not line.startswith('X('):
                continue
            m = _LINE.match(line)
            if not m:
                raise AbiError(f'{f}:{ln}: unparsable registry line')
            name, oid = m.group(1), int(m.group(2))
            if name in ops or oid in ids:
                raise AbiError(f'{f}:{ln}: duplicate operator {name}={oid}')
            ops[name] = Op(name, oid, _parse_sig(m.group(3), f'{f}:{ln}'))
            ids[oid] = name
    return ops


@lru_cache(maxsize=None)
def ops_by_id(include_dir: str = str(INCLUDE_DIR)) -> dict:
    return {o.id: o for o in load_ops(include_dir).values()}


def check_header(include_dir: str = str(INCLUDE_DIR)) -> None:
    """The descriptor in mvm_task_abi.h has exactly DESC_FIELDS, all int32, in this order."""
    text = (Path(include_dir) / 'mvm_task_abi.h').read_text()
    body = re.search(r'struct\s+MvmTaskDesc\s*\{(.*?)\}', text, re.S).group(1)
    fields = tuple(re.findall(r'^\s*int32_t\s+(\w+)\s*;', body, re.M))
    if fields != DESC_FIELDS:
        raise AbiError(f'mvm_task_abi.h fields {fields} differ from {DESC_FIELDS}')
    if int(re.search(r'#define\s+MVM_ABI_VERSION\s+(\d+)', text).group(1)) != ABI_VERSION:
        raise AbiError('ABI version mismatch')
