"""The executor's completion protocol relies on every operator storing to global memory only with write-through
(agent-scope, `sc1`) stores: a task's stores are then agent-visible once each wave has waited for them, and no
release fence (an L2 write-back on gfx950) is issued per task. This test compiles the executor for gfx950 to
assembly and checks the compiled code itself:

  * every dispatch case calls an operator that is a function of its own (not inlined into the kernel), and
  * no device function other than the `__global__` kernels holds a global / flat / buffer store without `sc1`
    (scratch stores, i.e. register spills, are private and not counted).

The kernels' own plain stores are executor bookkeeping read by the host after the launch (trace records, error
details), not operator data. Bodies inlined into a kernel (the GEMM tile main loops, the decode GEMV and attention
split) store operator data only through write-through helpers or called epilogues, so the dispatch-case test and the
private-segment test below cover what inlining can change. The assembly is compiled with the library's own flags.
"""
import re
import shutil
import subprocess

import pytest

from kvm_amd import build as kb

KERNELS = ('kvm_exec_kernel', 'kvm_static_kernel', 'kvm_reset_kernel', 'kvm_seed_kernel', 'kvm_seeded_kernel', 'kvm_seeded_bf16_kernel',
           'kvm_fill32_kernel', 'kvm_fill16_kernel', 'kvm_copy_probe_kernel')


@pytest.fixture(scope='module')
def asm(tmp_path_factory):
    if not shutil.which(kb.HIPCC) and not kb.Path(kb.HIPCC).exists():
        pytest.skip('hipcc not available')
    out = tmp_path_factory.mktemp('wt') / 'exec.s'
    r = subprocess.run([kb.HIPCC, *kb.LIB_FLAGS, '--cuda-device-only', '-S', str(kb.CSRC / 'exec.hip'), '-o', str(out)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text()


def _functions(text):
    types = set(re.findall(r'\.type\s+(\S+),@function', text))
    funcs, cur = {}, None
    for line in text.split('\n'):
        m = re.match(r'^([_a-zA-Z][\w.$]*):', line)
        if m and m.group(1) in types:
            cur = m.group(1)
            funcs[cur] = []
        elif cur is not None:
            funcs[cur].append(line.strip())
    return funcs


def _demangle(names):
    r = subprocess.run(['c++filt'], input='\n'.join(names), capture_output=True, text=True)
    return dict(zip(names, r.stdout.split('\n')))


def test_operators_store_write_through_only(asm):
    funcs = _functions(asm)
    dem = _demangle(list(funcs))
    bad = {}
    for name, body in funcs.items():
        plain_name = dem[name][5:] if dem[name].startswith('void ') else dem[name]   # templates demangle with their return type
        if any(plain_name == k or plain_name.startswith(k + '(') or plain_name.startswith(k + '<') for k in KERNELS):
            continue
        plain = [t for t in body if re.match(r'(global|flat|buffer)_store', t) and not re.search(r'\bsc1\b', t)]
        if plain:
            bad[dem[name]] = plain[:3]
    assert not bad, bad


def test_every_dispatch_case_is_a_function(asm):
    src = (kb.CSRC / 'exec.hip').read_text()
    body = src[src.index('dispatch(int op'):src.index('void kvm_exec_kernel')]
    called = set(re.findall(r'\b(op_\w+)(?:<[^>]*>)?\(c\)', body))
    assert len(called) > 50
    have = {d.split('(')[0].split('kvm::')[-1].split('<')[0] for d in _demangle(list(_functions(asm))).values()}
    missing = sorted(f for f in called if f not in have)
    assert not missing, f'operators inlined into the kernel (mark them __noinline__): {missing}'


def test_kernel_private_segments_stay_below_the_residency_guard(asm):
    """kvm_create refuses a build whose persistent kernels need more than KVM_MAX_PRIVATE_BYTES (2,048) of private
    segment per lane; the compiled kernels stay below it (a 2,096-byte build stopped before its first task)."""
    sizes = {}
    for name in ('kvm_exec_kernel', 'kvm_static_kernel'):
        ms = re.findall(r'\.amdhsa_kernel\s+(\S*' + name + r'\S*)\n(.*?)\.end_amdhsa_kernel', asm, re.S)
        assert ms, name
        for sym, body in ms:
            f = re.search(r'\.amdhsa_private_segment_fixed_size\s+(\d+)', body)
            sizes[sym] = int(f.group(1))
    assert len(sizes) == 4                      # the dynamic kernel and the three static instantiations
    assert all(0 < v <= 2048 for v in sizes.values()), sizes
