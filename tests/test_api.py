"""Python API and host logic (CPU only): the reference's CPU-runnable tests (tests/test_correctness.py:56-59,
141-163) and the host-side validation of csrc/ma_deform_fused.cu:236-266, 298-308, 333, exercised without a GPU."""

import numpy as np
import math

import pytest
import torch

import marearts_tinydeform_amd as td
from marearts_tinydeform_amd import _native
from oracle import bruteforce
from inputs import RTDETR_LEVELS, make


def test_public_names():
    assert set(td.__all__) >= {'ma_deform_attn', 'ma_deform_attn_reference', 'choose_mode'}
    assert td.MODES == ('auto', 'fused', 'project')


def test_cpu_path_is_reference():
    # reference tests/test_correctness.py:56-59
    args = make(1, 10, 2, 8, 16, [(6, 7), (3, 4)], 2)
    with torch.inference_mode():
        for mode in td.MODES:
            assert torch.equal(td.ma_deform_attn(*args, mode=mode), td.ma_deform_attn_reference(*args))


def test_reference_path_matches_oracle():
    args = make(2, 12, 4, 8, 32, [(10, 15), (5, 8)], 4)
    f64 = [t if t is None or t.dtype == torch.long else t.double() for t in args]
    assert np.abs(td.ma_deform_attn_reference(*f64).numpy() - bruteforce.deform_attn(*args)).max() <= 1e-12
    # float32 within float32 rounding
    got = td.ma_deform_attn_reference(*args).double().numpy()
    assert np.abs(got - bruteforce.deform_attn(*args)).max() <= 1e-5


def test_reference_path_supports_autograd():
    args = make(1, 4, 2, 4, 8, [(5, 6)], 2)
    args[0].requires_grad_(True)
    td.ma_deform_attn(*args).sum().backward()  # CPU tensors: the reference, with autograd
    assert args[0].grad is not None and args[0].grad.abs().sum() > 0


def test_unknown_mode_raises_value_error():
    args = make(1, 4, 2, 4, 8, [(5, 6)], 2)
    with pytest.raises(ValueError):
        td.ma_deform_attn(*args, mode='nope')


def test_auto_picks_fused_for_few_queries():
    # reference tests/test_correctness.py:149-153
    few = make(1, 50, 8, 32, 256, RTDETR_LEVELS, 4)
    many = make(8, 900, 8, 32, 256, RTDETR_LEVELS, 4)
    assert td.choose_mode(few[0], few[1], few[5]) == 'fused'
    assert td.choose_mode(many[0], many[1], many[5]) == 'project'


def test_auto_limits_follow_the_gpu_generation(monkeypatch):
    # reference tests/test_correctness.py:156-163: compute capability 8.x takes FUSED_LIMIT, 7.x FUSED_LIMIT_SM75 (no
    # device properties here: a CPU-only process falls back to FUSED_LIMIT)
    def no_props(i):
        raise RuntimeError('no device')
    monkeypatch.setattr(torch.cuda, 'get_device_properties', no_props)
    for cap, table in (((8, 9), td.FUSED_LIMIT), ((7, 5), td.FUSED_LIMIT_SM75)):
        monkeypatch.setattr(torch.cuda, 'get_device_capability', lambda device=None, cap=cap: cap)
        assert td._limits.__wrapped__(0) is table


def test_auto_limits_follow_the_gpu_architecture(monkeypatch):
    # on AMD GPUs (capability 9.x: gfx942, gfx950) the table is chosen by gcnArchName
    class Props:
        def __init__(self, arch):
            self.gcnArchName = arch

    monkeypatch.setattr(torch.cuda, 'get_device_capability', lambda device=None: (9, 5))
    for arch, table in (('gfx950:sramecc+:xnack-', td.FUSED_LIMIT), ('gfx942', td.FUSED_LIMIT)):
        monkeypatch.setattr(torch.cuda, 'get_device_properties', lambda i, arch=arch: Props(arch))
        assert td._limits.__wrapped__(0) is table
    assert td.ARCH_LIMITS['gfx950'] is td.FUSED_LIMIT


def test_reference_threshold_tables_keep_the_reference_rule(monkeypatch):
    # an (a, b) entry is the reference's rule: fused while Q * L * P * 4 / (N * D) < a + b / B
    # (marearts_tinydeform/__init__.py:39-46); FUSED_LIMIT_SM75 holds the reference's values
    assert td.FUSED_LIMIT_SM75[torch.float16] == (0.020, 0.0) and td.__version__ == '0.1.1'
    monkeypatch.setitem(td.FUSED_LIMIT, torch.float32, (0.073, 0.032))
    few = make(1, 50, 8, 32, 256, RTDETR_LEVELS, 4)    # r = 50 * 12 * 4 / (8400 * 32) = 0.0089 < 0.105
    many = make(1, 600, 8, 32, 256, RTDETR_LEVELS, 4)  # r = 0.107
    assert td.choose_mode(few[0], few[1], few[5]) == 'fused'
    assert td.choose_mode(many[0], many[1], many[5]) == 'project'
    with pytest.raises(ValueError):
        td.predict_us(few[0], few[1], few[5])


def test_cost_tables_are_sane():
    ff, fg, fs = td.cost_features(1, 300, 8, 32, 256, 8400, 3, 4, 2)
    gf = td.gap_features(1, 300, 8400, 8, 32, 3, 4, 2)
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        coef = td.FUSED_LIMIT[dtype]
        assert [len(coef[k]) for k in ('fused', 'gemm', 'sample', 'gap')] == [len(ff), len(fg), len(fs), len(gf)]
        assert all(c >= 0 for k in ('fused', 'gemm', 'sample', 'gap') for c in coef[k])


def test_cost_features_follow_the_launch_plans():
    # RT-DETR 640 fp16 B1 Q300: one balanced slice of 9-10 rows per CU (12 wavefronts), 256 workgroups; the GEMM takes
    # 64 x 64 tiles (528 of them: 3 on the busiest CU); the sampler 600 workgroups of 4 rows
    ff, fg, fs = td.cost_features(1, 300, 8, 32, 256, 8400, 3, 4, 2)
    assert _native.fused_plan(torch.float16, 1, 300, 8400, 256, 8, 32, 3, 4)[:6] == [0, 256, 12, 10, 32, 10]
    assert ff[1] == pytest.approx(10 * 48 * 256 * 2 / 1e6) and ff[2:6] == [0.0] * 4
    assert ff[8] == pytest.approx(16 * 256 * 32 * 2 / 1e6)
    assert _native.value_proj_plan(torch.float16, 8400, 256, 256, heads=8, N=8400) == 25
    assert fg[2] == pytest.approx(3 * 64 * 64 * 256 * 2 * 256 / 1e9) and fg[3] == pytest.approx(8400 * 512 * 2 / 1e6)
    assert _native.sample_plan(torch.float16, 1, 300, 8400, 8, 32, 3, 4, head_major=True)[:3] == [600, 2, 4]
    assert fs[1] == pytest.approx(300 * 8 * 48 * 32 * 2 / 1e6) and fs[2] == pytest.approx(3 * 4 * 48 * 32 * 2 / 1e6)
    # each XCD's L2 pulls in the rows its queries touch: 4800 corner reads per level over levels of 6400, 1600 and
    # 400 tokens (the 4:1 level sizes are exact here)
    touched = sum(n * (1 - math.exp(-4800 / n)) for n in (6400, 1600, 400))
    assert ff[6] == pytest.approx(touched * 512 / 1e6)
    # C = 1024 B2 (43520 x 1024 x 1024): the persistent GEMM's 680 tiles of 256 x 256, 85 per XCD over 32
    # workgroups: 3 rounds
    _, fg, _ = td.cost_features(2, 300, 16, 64, 1024, 21760, 4, 16, 2)
    assert fg[4] == 3 and fg[5] == pytest.approx(3 * 1.024) and fg[1:4] == [0.0] * 3
    # C = 256 B8 (67200 rows): the streaming GEMM, 263 tokens per CU in 9 steps of 32
    _, fg, _ = td.cost_features(8, 300, 8, 32, 256, 8400, 3, 4, 2)
    assert fg[1] == pytest.approx(9 * 32 * 512 * 2 * 256 / 1e6)


def test_auto_crossover_moves_with_queries_batch_and_channels():
    # RT-DETR 640, 16-bit (measured on MI355X): fused at batch 1 up to 900 queries (14.1 against 14.6 µs at 900),
    # project from 600 queries at batch 4; C=1024 / 16 heads / 64 samples (the limit shape) switches to project by
    # 300 queries
    def pick(B, Q, H, D, C, levels, P, dtype=torch.float16):
        mem = torch.empty(B, sum(h * w for h, w in levels), C, dtype=dtype)
        w = torch.empty(H * D, C, dtype=dtype)
        loc = torch.empty(B, Q, H, len(levels), P, 2, dtype=dtype)
        return td.choose_mode(mem, w, loc)
    assert pick(1, 300, 8, 32, 256, RTDETR_LEVELS, 4) == 'fused'
    assert pick(1, 600, 8, 32, 256, RTDETR_LEVELS, 4) == 'fused'
    assert pick(1, 900, 8, 32, 256, RTDETR_LEVELS, 4) == 'fused'
    assert pick(4, 300, 8, 32, 256, RTDETR_LEVELS, 4) == 'fused'
    assert pick(4, 600, 8, 32, 256, RTDETR_LEVELS, 4) == 'project'
    # batch 8, 300 queries, bfloat16: fused 22.5 against project 24.1 µs (1000-call graphs)
    assert pick(8, 300, 8, 32, 256, RTDETR_LEVELS, 4, torch.bfloat16) == 'fused'
    assert pick(8, 900, 8, 32, 256, RTDETR_LEVELS, 4) == 'project'
    limit = [(128, 128), (64, 64), (32, 32), (16, 16)]
    assert pick(2, 50, 16, 64, 1024, limit, 16, torch.bfloat16) == 'fused'
    assert pick(2, 300, 16, 64, 1024, limit, 16, torch.bfloat16) == 'project'


# ---- host validation (same rules and messages as the reference's host checks) ---------------------------------

def geometry_args():
    return make(1, 8, 2, 8, 16, [(6, 7), (3, 4)], 2)


@pytest.mark.parametrize('what,index,make_bad,message', [
    ('memory rank', 0, lambda a: a[0][0], 'memory / value must be [B, N, C]'),
    ('loc rank', 5, lambda a: a[5][..., 0], 'sampling_locations must be [B, Q, H, L, P, 2]'),
    ('attn rank', 6, lambda a: a[6][..., 0], 'attention_weights must be [B, Q, H, L, P]'),
    ('attn shape', 6, lambda a: a[6][:, :4], 'attention_weights must be [B, Q, H, L, P] like sampling_locations'),
    ('batch', 0, lambda a: torch.cat([a[0], a[0]]), 'batch size mismatch'),
    ('shapes dtype', 3, lambda a: a[3].int(), 'spatial_shapes must be int64 [L, 2]'),
    ('shapes size', 3, lambda a: a[3][:1], 'spatial_shapes must be int64 [L, 2]'),
    ('starts dtype', 4, lambda a: a[4].int(), 'level_start_index must be int64 [L]'),
    ('loc dtype', 5, lambda a: a[5].double(), 'all float tensors must have the same dtype'),
    ('attn dtype', 6, lambda a: a[6].half(), 'all float tensors must have the same dtype'),
])
def test_check_geometry_rejects(what, index, make_bad, message):
    a = geometry_args()
    a[index] = make_bad(a)
    with pytest.raises(RuntimeError, match=message.replace('[', r'\[').replace(']', r'\]')):
        _native.check_geometry(a[0], a[3], a[4], a[5], a[6], require_gpu=False)


def test_check_geometry_limits():
    a = geometry_args()
    loc = torch.rand(1, 8, 2, 2, 40, 2)
    attn = torch.ones(1, 8, 2, 2, 40) / 80
    with pytest.raises(RuntimeError, match='levels x points must be <= 64'):
        _native.check_geometry(a[0], a[3], a[4], loc, attn, require_gpu=False)
    loc0 = torch.rand(1, 8, 0, 2, 2, 2)
    with pytest.raises(RuntimeError, match='need at least one head'):
        _native.check_geometry(a[0], a[3], a[4], loc0, loc0[..., 0], require_gpu=False)
    assert _native.check_geometry(a[0], a[3], a[4], a[5], a[6], require_gpu=False) == (1, 8, 2, 2, 2)
    with pytest.raises(RuntimeError, match='inputs must be GPU tensors'):
        _native.check_geometry(a[0], a[3], a[4], a[5], a[6])


def test_check_projection_rejects():
    a = geometry_args()
    mem, w, b = a[0], a[1], a[2]
    assert _native.check_projection(mem, w, b, 2) == 16
    with pytest.raises(RuntimeError, match='value_weight must be'):
        _native.check_projection(mem, w[:, :8], b, 2)
    with pytest.raises(RuntimeError, match='multiple of the head count'):
        _native.check_projection(mem, w[:15], None, 2)
    with pytest.raises(RuntimeError, match='device and dtype'):
        _native.check_projection(mem, w.half(), b, 2)
    with pytest.raises(RuntimeError, match='value_bias must be'):
        _native.check_projection(mem, w, b[:4], 2)
    with pytest.raises(RuntimeError, match='value_bias must be'):
        _native.check_projection(mem, w, b.double(), 2)


def test_missing_extension_raises_for_device_entries(monkeypatch):
    monkeypatch.setattr(_native, 'lib', None)
    monkeypatch.setattr(_native, 'load_error', 'not built')
    a = geometry_args()
    with pytest.raises(RuntimeError, match='without its HIP extension'):
        _native.fused_forward(*a)
    with pytest.raises(RuntimeError, match='without its HIP extension'):
        _native.value_proj(a[0], a[1], a[2])
    with pytest.raises(RuntimeError, match='without its HIP extension'):
        td.ma_deform_sample(a[0], a[3], a[4], a[5], a[6])
    # CPU tensors still run the reference path (reference marearts_tinydeform/__init__.py:15-18, 62-64)
    assert td.ma_deform_attn(*a).shape == (1, 8, 16)
