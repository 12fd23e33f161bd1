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
           'eager.hip']
# measurement probes: a library of their own (include/slimkv_probe.h)
PROBE_LIBRARY = PACKAGE / 'libslimkv_probe.so'
PROBE_SOURCES = ['probe.hip']

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
    """Compile the serving library and the probe library; always recompiles."""
    _build_one(LIBRARY, sources(), verbose, extra)
    _build_one(PROBE_LIBRARY, [CSRC / name for name in PROBE_SOURCES], verbose, extra)
    return LIBRARY


def _build_one(library, srcs, verbose, extra):
    tmp = library.with_suffix('.so.tmp')
    cmd = [hipcc(), *FLAGS, *extra, '-o', str(tmp), *map(str, srcs)]
    if verbose:
        print(' '.join(cmd), flush=True)
    result = subprocess.run(cmd, cwd=str(CSRC), capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = '\n'.join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f'hipcc failed ({result.returncode}):\n{stderr}')
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)
    os.replace(tmp, library)
    return library


if __name__ == '__main__':
    print(build(verbose=True))
