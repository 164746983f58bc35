"""The C ABI library (CPU only: no kernel is launched). libtinydeform.so must load, export every function
include/tinydeform.h declares, agree with the header's constants, and reject invalid arguments on the host with
the reference's messages (csrc/ma_deform_fused.cu:236-266, 298-308) before touching a device."""

import ctypes
import os
import re

import pytest

from marearts_tinydeform_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'tinydeform.h')


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r'^\s*(?:const\s+)?\w+\*?\s+\*?(td_\w+)\s*\(', text, flags=re.M)))


def header_defines():
    return {k: int(v) for k, v in re.findall(r'#define\s+(TD_\w+)\s+(-?\d+)', open(HEADER).read())}


@pytest.fixture(scope='module')
def lib():
    assert os.path.exists(_native.LIB_PATH), 'libtinydeform.so is not built: run __graft_entry__.build()'
    lib = _native.load()
    assert lib is not None, _native.load_error
    return lib


def test_header_declares_the_entry_points():
    assert header_functions() == ['td_fused_forward', 'td_fused_forward_masked', 'td_fused_plan', 'td_input_grad',
                                  'td_input_weight_grad', 'td_last_error',
                                  'td_layer_fused_forward', 'td_layer_prologue', 'td_layer_sample_forward',
                                  'td_probe_atomic', 'td_probe_empty', 'td_probe_gather',
                                  'td_project_forward', 'td_project_forward_noalloc', 'td_sample_backward',
                                  'td_sample_forward',
                                  'td_sample_forward_heads', 'td_sample_forward_masked', 'td_sample_forward_v2',
                                  'td_sample_plan',
                                  'td_value_proj', 'td_value_proj_heads', 'td_value_proj_plan', 'td_version',
                                  'td_weight_grad',
                                  'td_weight_grad_workspace']


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(_native.LIB_PATH)
    for name in header_functions():
        assert hasattr(raw, name), name
    assert set(header_functions()) == set(_native.SIGNATURES)


def test_measurement_build_exports_the_same_abi_and_its_stamps(lib):
    # libtinydeform_phases.so (bench.py --phases) is the same library with the fused kernel's phase stamps: every
    # entry point of the header, plus td_phase_stamps, which the product library does not have
    path = os.path.join(os.path.dirname(_native.LIB_PATH), 'libtinydeform_phases.so')
    assert os.path.exists(path), 'libtinydeform_phases.so is not built: run __graft_entry__.build()'
    raw = ctypes.CDLL(path)
    for name in header_functions():
        assert hasattr(raw, name), name
    assert hasattr(raw, 'td_phase_stamps')
    assert not hasattr(ctypes.CDLL(_native.LIB_PATH), 'td_phase_stamps')


def test_header_constants_match_python(lib):
    d = header_defines()
    assert d['TD_MAX_LEVEL_POINTS'] == _native.MAX_LEVEL_POINTS
    assert d['TD_MAX_CHANNELS'] == _native.MAX_CHANNELS
    assert d['TD_NOALLOC_SCRATCH_BYTES'] == _native.NOALLOC_SCRATCH_BYTES
    assert {d['TD_F32'], d['TD_F16'], d['TD_BF16'], d['TD_F64']} == set(_native.DTYPE_CODES.values())
    import torch
    assert _native.DTYPE_CODES[torch.float32] == d['TD_F32']
    assert _native.DTYPE_CODES[torch.float16] == d['TD_F16']
    assert _native.DTYPE_CODES[torch.bfloat16] == d['TD_BF16']
    assert _native.DTYPE_CODES[torch.float64] == d['TD_F64']


def test_version(lib):
    assert lib.td_version() == 100


def fused(lib, dtype=1, B=1, Q=4, N=100, C=256, H=8, D=32, L=3, P=4, ptr=16):
    p = ptr
    return lib.td_fused_forward(dtype, p, p, None, p, p, p, p, p, B, Q, N, C, H, D, L, P, None)


def sample(lib, dtype=1, B=1, Q=4, N=100, H=8, D=32, L=3, P=4, ptr=16):
    p = ptr
    return lib.td_sample_forward(dtype, p, p, p, p, p, p, B, Q, N, H, D, L, P, None)


@pytest.mark.parametrize('kwargs,message', [
    (dict(L=4, P=20), 'levels x points must be <= 64'),
    (dict(H=0), 'need at least one head'),
    (dict(C=8200), 'channels must be <= 8192'),
    (dict(N=2 ** 31), 'too many memory tokens'),
    (dict(B=2 ** 16, Q=2 ** 13, H=2 ** 3), r'too many \(batch, query, head\) rows'),
    (dict(Q=-1), 'sizes must be non-negative'),
    (dict(ptr=None), 'null pointer argument'),
])
def test_fused_rejects_on_host(lib, kwargs, message):
    assert fused(lib, **kwargs) == header_defines()['TD_E_ARG']
    assert re.search(message, lib.td_last_error().decode())


def test_unknown_dtype(lib):
    assert fused(lib, dtype=9) == header_defines()['TD_E_DTYPE']
    assert sample(lib, dtype=-1) == header_defines()['TD_E_DTYPE']
    assert lib.td_value_proj(7, 16, 16, None, 16, 4, 4, 4, None) == header_defines()['TD_E_DTYPE']


def test_sample_and_proj_reject_on_host(lib):
    assert sample(lib, L=8, P=9) == header_defines()['TD_E_ARG']
    assert 'levels x points' in lib.td_last_error().decode()
    assert sample(lib, ptr=None) == header_defines()['TD_E_ARG']
    assert lib.td_value_proj(1, None, None, None, None, 4, 4, 4, None) == header_defines()['TD_E_ARG']
    assert lib.td_value_proj(1, 16, 16, None, 16, -1, 4, 4, None) == header_defines()['TD_E_ARG']


def test_masked_entries_reject_on_host(lib):
    p = 16
    assert lib.td_fused_forward_masked(1, p, p, None, p, p, p, p, None, p, 1, 4, 100, 256, 8, 32, 4, 20, None) == \
        header_defines()['TD_E_ARG']
    assert 'levels x points' in lib.td_last_error().decode()
    assert lib.td_sample_forward_masked(1, p, p, p, p, p, None, p, 1, 0, 100, 8, 32, 3, 4, None) == 0


def project(lib, dtype=1, B=1, Q=4, N=100, C=256, H=8, D=32, L=3, P=4, loc_acc=0, ws=16, ptr=16):
    p = ptr
    return lib.td_project_forward(dtype, p, p, None, p, p, p, p, None, loc_acc, ws, p, B, Q, N, C, H, D, L, P, None)


def test_project_rejects_on_host(lib):
    E = header_defines()
    assert project(lib, L=8, P=9) == E['TD_E_ARG']
    assert 'levels x points' in lib.td_last_error().decode()
    assert project(lib, loc_acc=2) == E['TD_E_ARG']
    assert 'loc_acc' in lib.td_last_error().decode()
    assert project(lib, ws=None) == E['TD_E_ARG']
    assert 'null pointer' in lib.td_last_error().decode()
    assert project(lib, dtype=4) == E['TD_E_DTYPE']
    assert project(lib, Q=0) == 0  # nothing to compute
    assert project(lib, Q=0, ws=None) == 0


def test_head_major_entries_reject_on_host(lib):
    E = header_defines()
    p = 16
    # D = 4 float16 elements is an 8-byte head row: head-major needs a multiple of 16 bytes
    assert lib.td_value_proj_heads(1, p, p, None, p, 1, 100, 256, 64, 4, None) == E['TD_E_ARG']
    assert '16 bytes' in lib.td_last_error().decode()
    assert lib.td_value_proj_heads(1, p, p, None, p, 1, 100, 256, 0, 32, None) == E['TD_E_ARG']
    assert lib.td_value_proj_heads(1, None, None, None, None, 1, 100, 256, 8, 32, None) == E['TD_E_ARG']
    assert lib.td_value_proj_heads(6, p, p, None, p, 1, 100, 256, 8, 32, None) == E['TD_E_DTYPE']
    assert lib.td_value_proj_heads(1, p, p, None, p, 0, 100, 256, 8, 32, None) == 0  # nothing to compute
    assert lib.td_sample_forward_heads(1, p, p, p, p, p, None, 0, p, 1, 4, 100, 8, 32, 8, 9, None) == E['TD_E_ARG']
    assert 'levels x points' in lib.td_last_error().decode()
    assert lib.td_sample_forward_heads(1, p, p, p, p, p, None, 3, p, 1, 4, 100, 8, 32, 3, 4, None) == E['TD_E_ARG']
    assert lib.td_sample_forward_heads(1, None, p, p, p, p, None, 0, p, 1, 4, 100, 8, 32, 3, 4, None) == E['TD_E_ARG']
    assert lib.td_sample_forward_heads(1, p, p, p, p, p, None, 0, p, 1, 0, 100, 8, 32, 3, 4, None) == 0


def test_sample_v2_rejects_on_host(lib):
    import ctypes as ct
    p = 16
    pts = (ct.c_int64 * 3)(30, 30, 10)  # 70 samples > 64
    assert lib.td_sample_forward_v2(1, p, p, p, p, p, None, p, 1, 4, 100, 8, 32, 3, ct.cast(pts, ct.c_void_p), 0,
                                    None) == header_defines()['TD_E_ARG']
    assert 'levels x points' in lib.td_last_error().decode()
    ok = (ct.c_int64 * 3)(3, 6, 3)
    assert lib.td_sample_forward_v2(1, p, p, p, p, p, None, p, 1, 4, 100, 8, 32, 3, ct.cast(ok, ct.c_void_p), 2,
                                    None) == header_defines()['TD_E_ARG']
    assert 'method' in lib.td_last_error().decode()
    assert lib.td_sample_forward_v2(1, p, p, p, p, p, None, p, 1, 0, 100, 8, 32, 3, ct.cast(ok, ct.c_void_p), 1,
                                    None) == 0


def test_empty_work_returns_ok_without_launching(lib):
    # zero rows: nothing to launch, so no device is needed
    assert fused(lib, Q=0) == 0
    assert fused(lib, B=0) == 0
    assert sample(lib, Q=0) == 0
    assert lib.td_value_proj(1, 16, 16, None, 16, 0, 4, 4, None) == 0
    assert lib.td_last_error().decode() == ''


def sample_backward(lib, dtype=1, B=1, Q=4, N=100, H=8, D=32, L=3, P=4, ptr=16):
    p = ptr
    return lib.td_sample_backward(dtype, p, p, p, p, p, None, p, p, p, p, p, B, Q, N, H, D, L, P, None)


def test_backward_entries_reject_on_host(lib):
    E = header_defines()
    assert sample_backward(lib, L=8, P=9) == E['TD_E_ARG']
    assert 'levels x points' in lib.td_last_error().decode()
    assert sample_backward(lib, ptr=None) == E['TD_E_ARG']
    assert sample_backward(lib, D=300) == E['TD_E_ARG']
    assert 'head dim' in lib.td_last_error().decode()
    assert sample_backward(lib, dtype=5) == E['TD_E_DTYPE']
    assert lib.td_input_grad(1, None, None, None, None, 4, 4, 4, None) == E['TD_E_ARG']
    assert lib.td_input_grad(1, 16, 16, 16, 16, -1, 4, 4, None) == E['TD_E_ARG']
    assert lib.td_input_grad(1, 16, 16, 16, 16, 0, 4, 4, None) == 0  # nothing to compute
    # the weight gradient checks its workspace against td_weight_grad_workspace before launching anything
    need = lib.td_weight_grad_workspace(1, 8400, 256, 256)
    assert need > 0
    assert lib.td_weight_grad(1, 16, 16, 16, 16, 8400, 256, 256, 16, need - 1, None) == E['TD_E_WORKSPACE']
    assert 'workspace' in lib.td_last_error().decode()
    assert lib.td_weight_grad(1, None, None, None, None, 8400, 256, 256, 16, need, None) == E['TD_E_ARG']
    assert lib.td_weight_grad(1, 16, 16, 16, None, 8400, 0, 256, 16, need, None) == 0  # nothing to compute
    # both projection gradients in one call: the same checks, the workspace before anything is launched
    iwg = lib.td_input_weight_grad
    assert iwg(9, 16, 16, 16, 16, 16, 16, 16, 8400, 256, 256, 16, need, None) == E['TD_E_DTYPE']
    assert iwg(1, 16, 16, 16, 16, 16, 16, 16, -1, 256, 256, 16, need, None) == E['TD_E_ARG']
    assert iwg(1, 16, 16, 16, 16, 16, 16, 16, 8400, 256, 256, 16, need - 1, None) == E['TD_E_WORKSPACE']
    assert 'workspace' in lib.td_last_error().decode()
    assert iwg(1, 16, 16, 16, 16, None, 16, 16, 8400, 256, 256, 16, need, None) == E['TD_E_ARG']
    assert iwg(1, 16, 16, None, 16, 16, 16, 16, 8400, 256, 256, 16, need, None) == E['TD_E_ARG']


def test_probe_argument_errors(lib):
    # the measurement kernels refuse bad arguments before launching anything
    E = header_defines()
    assert lib.td_probe_empty(-1, None) == E['TD_E_ARG']
    assert lib.td_probe_gather(None, 1 << 20, 64, 8, 1, 1, 16, None) == E['TD_E_ARG']
    assert lib.td_probe_gather(16, 1 << 20, 48, 8, 1, 1, 16, None) == E['TD_E_ARG']  # not a power of two
    assert lib.td_probe_atomic(None, 1 << 20, 32, 1, 1, 1, None) == E['TD_E_ARG']
    assert lib.td_probe_atomic(16, 1 << 20, 24, 1, 1, 1, None) == E['TD_E_ARG']      # lanes
    assert lib.td_probe_atomic(16, 64, 32, 1, 1, 1, None) == E['TD_E_ARG']           # less than one chunk
    assert lib.td_probe_atomic(16, 1 << 20, 32, 0, 1, 1, None) == E['TD_E_ARG']
    assert lib.td_probe_atomic(16, 1 << 20, 32, 1, 0, 1, None) == E['TD_E_ARG']
    assert 'probe_atomic' in lib.td_last_error().decode()


@pytest.mark.parametrize('dtype,M,NO,K', [(1, 8400, 256, 256), (2, 43520, 1024, 1024), (0, 100, 48, 40),
                                          (3, 5, 16, 8), (1, 0, 64, 64), (0, 8400, 256, 256), (2, 20000, 256, 256),
                                          (1, 3000, 520, 600)])
def test_weight_grad_workspace_plan(lib, dtype, M, NO, K):
    # split-K plan: about 512 workgroups of 128 x 128 outputs (128 x 256 from K = 512 on, except float64; 1024
    # workgroups from 64 tiles), splits of at least four MFMA K steps (eight in 16 bits below 16384 tokens; 16 tokens
    # for float32, 32 otherwise) rounded up to the MFMA K, float32 partials (float64 for float64) plus bias partials;
    # the workspace covers the 128 x 128 plan as well (the launch combined with the input gradient)
    def splits(tw):
        tiles = -(-NO // 128) * -(-K // (128 * tw))
        kb = 16 if dtype == 0 else 32
        target = 1024 if tiles >= 64 else 512  # 1024 workgroups for 64 output tiles and more
        steps = 8 if dtype in (1, 2) and M < 16384 else 4
        s = max(1, min(-(-target // tiles), -(-M // (steps * kb))))
        chunk = -(-M // s) if M else 0
        chunk = -(-chunk // kb) * kb
        return -(-M // chunk) if chunk else 1
    s = max(splits(1), splits(2 if dtype != 3 and K >= 512 else 1))
    elem = 8 if dtype == 3 else 4
    assert lib.td_weight_grad_workspace(dtype, M, NO, K) == s * (NO * K + NO) * elem
