"""Build libtinydeform.so from csrc/*.hip with hipcc for gfx950 (MI355X), in-tree.

    python -m marearts_tinydeform_amd._build            # or: __graft_entry__.build()

Each source is compiled to an object under _build/ (in parallel), then linked into libtinydeform.so next to
this file, where marearts_tinydeform_amd._native loads it. No torch extension machinery (and so no hipify) is
involved: the library exports the C ABI of include/tinydeform.h and is loaded with ctypes.
"""

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, 'csrc')
BUILD = os.path.join(HERE, '_build')
LIB = os.path.join(HERE, 'libtinydeform.so')
ARCH = 'gfx950'

SOURCES = ['td_abi.hip', 'td_fused.hip', 'td_sample.hip', 'td_gemm.hip', 'td_gemm_dma.hip', 'td_gemm_stream.hip',
           'td_layer.hip', 'td_backward.hip', 'td_noalloc.hip', 'td_probe.hip']

# per-source additions: the direct-to-LDS GEMM keeps its MFMA accumulators in architectural VGPRs (in the
# accumulator-register form the compiler copies every accumulator through a temporary in the inner loop)
EXTRA_FLAGS = {'td_gemm_dma.hip': ['-mllvm', '-amdgpu-mfma-vgpr-form=1']}

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in the generated code (the host pass warns that it does not know
# the feature; that warning is expected).
HIPCC_FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-Wall', '-Wno-unused-function',
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-I', os.path.join(ROOT, 'include'),
]


def hipcc():
    path = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not os.path.exists(path):
        raise RuntimeError('hipcc not found: the HIP extension needs ROCm (hipcc) to build')
    return path


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + '.o')
    cmd = [hipcc()] + HIPCC_FLAGS + EXTRA_FLAGS.get(src, []) + ['-c', os.path.join(CSRC, src), '-o', obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed on {src}:\n{res.stdout}\n{res.stderr}')
    return obj


def build(verbose=False):
    """Compile every HIP source and link libtinydeform.so; returns the library path."""
    os.makedirs(BUILD, exist_ok=True)
    workers = min(len(SOURCES), max(1, (os.cpu_count() or 2) // 2))
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + '.tmp'
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', '-o', tmp] + objs
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'link failed:\n{res.stdout}\n{res.stderr}')
    os.replace(tmp, LIB)
    if verbose:
        print('built', LIB)
    return LIB


if __name__ == '__main__':
    build(verbose=True)
    sys.exit(0)
