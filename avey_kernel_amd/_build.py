"""Build libavey_hip.so in-tree for gfx950 (``python -m avey_kernel_amd._build``).

hipcc cross-compiles without a GPU, so this runs on any host with ROCm. Each
HIP source compiles to an object in parallel, then one link produces
``avey_kernel_amd/libavey_hip.so`` next to the Python binding that loads it.
"""

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, 'csrc')
INCLUDE = os.path.join(REPO_DIR, 'include')
BUILD_DIR = os.path.join(PKG_DIR, '_build')
LIB_PATH = os.path.join(PKG_DIR, 'libavey_hip.so')
SOURCES = ('avey_capi.hip', 'avey_generic.hip', 'avey_fused.hip', 'avey_backward.hip') + tuple(
    f'avey_fused_bm{bm}_{t}{k}.hip' for k in ('', '_strided') for bm in (64, 32, 16) for t in ('bf16', 'f16')) + tuple(
    f'avey_fused_bm16_{t}{k}_eg.hip' for k in ('', '_strided') for t in ('bf16', 'f16'))
ARCH = 'gfx950'

# -packed-fp32-ops: keep hipcc from emitting v_pk_{add,mul,fma}_f32; some of their
# forms have given wrong results on MI355X without any error.
HIP_FLAGS = ['-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}',
             '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
             '-Wno-pass-failed', '-I', INCLUDE, '-I', CSRC]


# Accumulators of the 16- and 32-row fused variants fit the 256 architectural VGPRs;
# with MFMA results in VGPRs the compiler stops shuttling them through AGPRs
# (hundreds of v_accvgpr moves per key tile otherwise). The 64-row variants need
# more than 256 registers and keep the compiler's default split.
EXTRA_FLAGS = {f'avey_fused_bm{bm}_{t}{k}{e}.hip': ['-mllvm', '-amdgpu-mfma-vgpr-form']
               for bm in (16, 32) for t in ('bf16', 'f16') for k in ('', '_strided') for e in ('', '_eg')
               if bm == 16 or not e}


def hipcc():
    path = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not os.path.exists(path):
        raise RuntimeError('hipcc not found; install ROCm or put hipcc on PATH')
    return path


def _compile(src):
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + '.o')
    cmd = [hipcc(), *HIP_FLAGS, *EXTRA_FLAGS.get(src, []), '-c', os.path.join(CSRC, src), '-o', obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed for {src}:\n{res.stderr}')
    return obj


def build(verbose=True):
    """Compile every HIP source and link the shared library. Returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIB_PATH + '.tmp'
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', *objs, '-o', tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'link failed:\n{res.stderr}')
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f'built {LIB_PATH}')
    return LIB_PATH


if __name__ == '__main__':
    build()
    sys.exit(0)
