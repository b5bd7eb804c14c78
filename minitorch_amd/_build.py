"""Build the gfx950 shared libraries of the C-ABI in-tree.

Each ``csrc/<name>.hip`` becomes ``cuda_kernels/<name>.so``, the file names the
reference's ctypes loaders open (reference minitorch/paged_kv_cache.py:19-24,
minitorch/kv_cache.py:18-23, minitorch/cuda_storage.py:14-18). Run as
``python -m minitorch_amd._build`` or through ``__graft_entry__.build()``.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
SRC = ROOT / 'csrc'
OUT = ROOT / 'cuda_kernels'
ARCH = 'gfx950'

# name -> extra link arguments. model_kernels links the paged decode library
# (its decoder loop launches mt_paged_decode_split), found next to it at run
# time through an $ORIGIN rpath; that library is therefore built first.
LIBRARIES = {
    'paged_attention_kernel': [],
    'inference_kernels': [],
    'cuda_runtime': [],
    'sched_kernels': [],
    'model_kernels': ['-lhipblaslt', f'-L{OUT}', '-l:paged_attention_kernel.so', '-Wl,-rpath,$ORIGIN'],
}
FIRST = ('paged_attention_kernel',)

HIPCC_FLAGS = [
    '-O3', '-std=c++17', '-fPIC', '-shared', f'--offload-arch={ARCH}',
    # Packed-fp32 VALU forms are kept out of every kernel.
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    # Launches and stream-0 API calls go to the calling thread's default
    # stream, which (unlike the legacy null stream) can be captured into a
    # graph; every library shares it.
    '-fgpu-default-stream=per-thread',
    '-Wno-unused-command-line-argument',
]


def hipcc():
    rocm = os.environ.get('ROCM_PATH', '/opt/rocm')
    return str(Path(rocm) / 'bin' / 'hipcc')


def command(name):
    src = SRC / f'{name}.hip'
    out = OUT / f'{name}.so'
    return [hipcc(), *HIPCC_FLAGS, f'-I{SRC}', str(src), '-o', str(out), *LIBRARIES[name]]


def build_one(name):
    src = SRC / f'{name}.hip'
    if not src.exists():
        return name, None
    out = OUT / f'{name}.so'
    tmp = out.with_suffix('.so.tmp')
    cmd = command(name)
    cmd[cmd.index(str(out))] = str(tmp)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f'hipcc failed for {name}:\n{result.stderr}')
    os.replace(tmp, out)
    return name, out


def build(names=None, jobs=4):
    OUT.mkdir(exist_ok=True)
    names = list(LIBRARIES) if names is None else list(names)
    results = [build_one(n) for n in FIRST if n in names]
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        results += list(pool.map(build_one, [n for n in names if n not in FIRST]))
    return {name: path for name, path in results if path is not None}


if __name__ == '__main__':
    built = build(sys.argv[1:] or None)
    for name, path in built.items():
        print(f'{name}: {path}')
