"""Build the gfx950 shared library `slimkv_amd/libslimkv_hip.so` with hipcc.

The library is the product's only compute path: every Python entry point in
this package calls it through its C ABI (include/slimkv_hip.h).  Building is a
plain hipcc invocation, so it cross-compiles on a machine without a GPU.
"""
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / 'csrc'
LIBRARY = PACKAGE / 'libslimkv_hip.so'
SOURCES = ['attention.hip', 'rope.hip', 'recon.hip', 'paged.hip', 'prefill.hip', 'down.hip', 'project.hip',
           'eager.hip', 'probe.hip']

FLAGS = [
    '--offload-arch=gfx950', '-O3', '-std=c++17', '-fPIC', '-shared',
    # Packed FP32 instructions stay off: only ordinary fp32 VALU and MFMA.
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-fno-gpu-rdc', '-Wno-unused-result',
]


def hipcc():
    for candidate in (os.environ.get('HIPCC'), shutil.which('hipcc'), '/opt/rocm/bin/hipcc'):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError('hipcc not found; the slimkv_amd HIP library cannot be built')


def sources():
    return [CSRC / name for name in SOURCES]


def build(verbose=False, extra=()):
    """Compile every HIP source into one shared library; always recompiles."""
    tmp = LIBRARY.with_suffix('.so.tmp')
    cmd = [hipcc(), *FLAGS, *extra, '-o', str(tmp), *map(str, sources())]
    if verbose:
        print(' '.join(cmd), flush=True)
    result = subprocess.run(cmd, cwd=str(CSRC), capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = '\n'.join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f'hipcc failed ({result.returncode}):\n{stderr}')
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == '__main__':
    print(build(verbose=True))
