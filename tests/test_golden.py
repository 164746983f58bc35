"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py): the oracle and this torch's
grid_sample must reproduce them on the CPU, and the HIP kernels must match them on the GPU in every element type
(the fixture inputs are exactly representable in bfloat16, float16 and float32)."""

import glob
import os

import numpy as np
import pytest
import torch

import marearts_tinydeform_amd as td
from oracle import bruteforce, gridsample

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, 'golden', '*.npz')))
NAMES = [os.path.splitext(os.path.basename(f))[0] for f in FIXTURES]
# cases whose result is fixed by the clamp and token-range rules rather than by grid_sample
RULE_CASES = {'nonfinite_locations', 'token_range'}


def load(path, dtype=torch.float64):
    z = np.load(path)
    t = lambda k: torch.from_numpy(z[k])  # noqa: E731
    args = [t('memory').to(dtype), t('weight').to(dtype), t('bias').to(dtype) if 'bias' in z else None,
            t('shapes'), t('starts'), t('loc').to(dtype), t('attn').to(dtype)]
    return args, z['expected']


def test_fixture_set_is_complete():
    assert len(FIXTURES) >= 12
    for name in ('three_levels', 'odd_channels', 'far_outside', 'max_level_points', 'nonfinite_locations',
                 'token_range'):
        assert name in NAMES


@pytest.mark.parametrize('path', FIXTURES, ids=NAMES)
def test_oracle_reproduces_fixture(path):
    args, expected = load(path)
    assert np.abs(bruteforce.deform_attn(*args) - expected).max() <= 1e-13
    assert np.abs(bruteforce.deform_attn_fused_order(*args) - expected).max() <= 1e-12
    name = os.path.splitext(os.path.basename(path))[0]
    if name not in RULE_CASES:
        assert np.abs(gridsample.deform_attn(*args).numpy() - expected).max() <= 1e-12


@pytest.mark.parametrize('path', FIXTURES, ids=NAMES)
def test_inputs_are_exact_in_every_dtype(path):
    for key, arr in np.load(path).items():
        if key in ('expected', 'shapes', 'starts'):
            continue
        t = torch.from_numpy(arr)
        fin = torch.isfinite(t)
        assert torch.equal(t[fin].to(torch.bfloat16).float(), t[fin]), key
        assert torch.equal(t[fin].half().float(), t[fin]), key


TOL = {torch.float32: 2e-5, torch.float16: 3e-3, torch.bfloat16: 2e-2, torch.float64: 1e-12}


@pytest.mark.gpu
@pytest.mark.parametrize('dtype', [torch.float32, torch.float16, torch.bfloat16, torch.float64])
def test_kernels_match_fixtures(dtype):
    for path, name in zip(FIXTURES, NAMES):
        args, expected = load(path, dtype)
        dev = [None if t is None else t.cuda() for t in args]
        for mode in ('fused', 'project'):
            with torch.inference_mode():
                out = td.ma_deform_attn(*dev, mode=mode)
            got = out.double().cpu().numpy()
            tol = TOL[dtype]
            err = np.abs(got - expected)
            assert (err <= tol + tol * np.abs(expected)).all(), f'{name} {dtype} [{mode}]: max |diff| {err.max():.3g}'
            if name == 'far_outside':
                assert np.array_equal(got == 0, expected == 0)
