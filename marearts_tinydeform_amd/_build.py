"""Build libtinydeform.so from csrc/*.hip with hipcc for gfx950 (MI355X), in-tree.

    python -m marearts_tinydeform_amd._build            # or: __graft_entry__.build()

Each source is compiled to an object under _build/ (in parallel), then linked into libtinydeform.so next to
this file, where marearts_tinydeform_amd._native loads it. No torch extension machinery (and so no hipify) is
involved: the library exports the C ABI of include/tinydeform.h and is loaded with ctypes.

The same run links libtinydeform_phases.so, a measurement build: td_fused.hip compiled with TD_PHASE_STAMPS, so
that the fused kernel records when its wavefronts pass each phase (bench.py --phases reads them). The package
never loads it.
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
PHASES_LIB = os.path.join(HERE, 'libtinydeform_phases.so')
PHASES_SOURCE = 'td_fused.hip'  # the one source that differs in the measurement build
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


def _compile(job):
    src, phases = job
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ('_phases' if phases else '') + '.o')
    defs = ['-DTD_PHASE_STAMPS'] if phases else []
    cmd = [hipcc()] + HIPCC_FLAGS + EXTRA_FLAGS.get(src, []) + defs + ['-c', os.path.join(CSRC, src), '-o', obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed on {src}:\n{res.stdout}\n{res.stderr}')
    return obj


def _link(objs, lib):
    tmp = lib + '.tmp'
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', '-o', tmp] + objs
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'link failed:\n{res.stdout}\n{res.stderr}')
    os.replace(tmp, lib)


def build(verbose=False, phases=True):
    """Compile every HIP source and link libtinydeform.so (and, with phases, libtinydeform_phases.so); returns the
    library path."""
    os.makedirs(BUILD, exist_ok=True)
    jobs = [(src, False) for src in SOURCES] + ([(PHASES_SOURCE, True)] if phases else [])
    # the two largest sources first, so that they do not start last
    jobs.sort(key=lambda j: j[0] != PHASES_SOURCE)
    workers = min(len(jobs), max(1, (os.cpu_count() or 2) // 2))
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, jobs))
    plain = [o for o, (_, ph) in zip(objs, jobs) if not ph]
    _link(plain, LIB)
    if verbose:
        print('built', LIB)
    if phases:
        swap = {os.path.join(BUILD, os.path.splitext(PHASES_SOURCE)[0] + '.o'): o
                for o, (_, ph) in zip(objs, jobs) if ph}
        _link([swap.get(o, o) for o in plain], PHASES_LIB)
        if verbose:
            print('built', PHASES_LIB)
    return LIB


if __name__ == '__main__':
    build(verbose=True)
    sys.exit(0)
