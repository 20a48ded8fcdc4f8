#!/usr/bin/env python3
"""Write the golden fixtures: for every workload in cases.py (and the reference's own example workloads under data/),
the bundle the reference compiler emits and the final buffers of the reference CPU VM's deterministic run.

    python3 tests/golden/make_golden.py [/root/reference]

Run in the build container only (the reference is not on the GPU box). It imports the reference's
runtime/compile_workload.py and runtime/workload_vm.py (pure-Python, stdlib only) and writes, per case,
tests/golden/<case>/{workload.json,tasks.bin,successors.bin,args.bin,metadata.json,golden.json}. These files are data:
inputs and the reference's outputs.
"""
import json
import shutil
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import cases  # noqa: E402


def main():
    ref = Path(sys.argv[1] if len(sys.argv) > 1 else '/root/reference')
    sys.path.insert(0, str(ref / 'runtime'))
    import compile_workload as cw
    import workload_vm as vm
    specs = {name: fn() for name, fn in cases.CASES.items()}
    specs['abi_diamond'] = json.loads((HERE / 'data/abi_diamond.json').read_text())
    specs['live_training_inference'] = json.loads((HERE / 'data/live_training_inference.json').read_text())
    for name, spec in specs.items():
        out = HERE / name
        if out.exists():
            shutil.rmtree(out)
        out.mkdir()
        (out / 'workload.json').write_text(json.dumps(spec, separators=(',', ':')) + '\n')
        compiled = cw.compile_spec(spec)
        cw.write_bundle(compiled, out)
        golden = vm.run_golden(compiled, timeout=600)
        with open(out / 'golden.json', 'w') as f:
            json.dump(golden, f, separators=(',', ':'))
            f.write('\n')
        print(f'{name}: {compiled.metadata["task_count"]} tasks, {compiled.metadata["edge_count"]} edges')


if __name__ == '__main__':
    main()
