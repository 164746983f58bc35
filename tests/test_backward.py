"""The backward on the CPU: the gradient oracle (oracle.gridsample.deform_attn_grads, PyTorch autograd through the
float64 grid_sample restatement) pinned against central finite differences of the independent numpy brute force
(oracle.bruteforce.deform_attn), a planted mistake the pin rejects, and the training entries' CPU routing.

Finite differences of a piecewise-bilinear function are exact up to O(eps^2) curvature (zero inside a cell for the
bilinear part, which is linear in each coordinate) plus float64 rounding, so the tolerance is tight: 1e-6 relative
to the largest gradient entry.
"""

import numpy as np
import pytest
import torch

import marearts_tinydeform_amd as td
from oracle import bruteforce, gridsample
from inputs import level_index

EPS = 1e-6
NAMES = ('memory', 'value_weight', 'value_bias', 'sampling_locations', 'attention_weights')


def tiny(seed=0, bias=True, mask=False):
    g = torch.Generator().manual_seed(seed)
    B, Q, H, D, C, P = 2, 3, 2, 3, 5, 2
    levels = [(4, 5), (3, 2)]
    shapes, starts, N = level_index(levels)
    L = len(levels)
    memory = torch.randn(B, N, C, generator=g, dtype=torch.float64)
    weight = torch.randn(H * D, C, generator=g, dtype=torch.float64) / C ** 0.5
    b = torch.randn(H * D, generator=g, dtype=torch.float64) * 0.1 if bias else None
    loc = torch.rand(B, Q, H, L, P, 2, generator=g, dtype=torch.float64) * 1.2 - 0.1
    attn = torch.randn(B, Q, H, L * P, generator=g, dtype=torch.float64).softmax(-1).view(B, Q, H, L, P)
    grad_out = torch.randn(B, Q, H * D, generator=g, dtype=torch.float64)
    pm = (torch.rand(B, N, generator=g) < 0.2) if mask else None
    return [memory, weight, b, shapes, starts, loc, attn], grad_out, pm


def finite_difference(args, grad_out, pm, name, idx):
    """d/dx_idx of sum(bruteforce.deform_attn(args) * grad_out), central difference."""
    k = NAMES.index(name)
    pos = (0, 1, 2, 5, 6)[k]
    vals = []
    for sgn in (1, -1):
        a = [t.clone() if isinstance(t, torch.Tensor) else t for t in args]
        a[pos].view(-1)[idx] += sgn * EPS
        out = bruteforce.deform_attn(*a, padding_mask=None if pm is None else pm.numpy())
        vals.append(float((out * grad_out.numpy()).sum()))
    return (vals[0] - vals[1]) / (2 * EPS)


@pytest.mark.parametrize('bias,mask', [(True, False), (False, False), (True, True)])
def test_gradient_oracle_matches_finite_differences(bias, mask):
    args, grad_out, pm = tiny(bias=bias, mask=mask)
    grads = gridsample.deform_attn_grads(*args, grad_out, padding_mask=pm)
    rng = np.random.default_rng(1)
    for name in NAMES:
        if grads[name] is None:
            assert name == 'value_bias' and not bias
            continue
        flat = grads[name].reshape(-1)
        scale = max(np.abs(flat).max(), 1e-3)
        for idx in rng.choice(flat.size, size=min(12, flat.size), replace=False):
            fd = finite_difference(args, grad_out, pm, name, int(idx))
            assert abs(fd - flat[idx]) <= 1e-6 * scale, f'{name}[{idx}]: autograd {flat[idx]} vs FD {fd}'


def test_planted_mistake_fails_against_finite_differences():
    # align_corners=True moves every sample by half a pixel: its location gradients disagree with the brute force
    args, grad_out, pm = tiny(seed=3)
    wrong = gridsample.deform_attn_grads(*args, grad_out, align_corners=True)['sampling_locations'].reshape(-1)
    fd = np.array([finite_difference(args, grad_out, pm, 'sampling_locations', i) for i in range(wrong.size)])
    assert np.abs(fd - wrong).max() > 1e-3 * np.abs(fd).max()


def test_closed_forms_of_the_gradients():
    args, grad_out, _ = tiny(seed=5)
    grads = gridsample.deform_attn_grads(*args, grad_out)
    memory, weight, b, shapes, starts, loc, attn = args
    # the bias gradient: grad_out weighted by each row's in-map weight sum, summed over (b, q); with every corner in
    # the map that is sum_{b,q} grad_out (softmaxed attention sums to 1 over a head's samples)
    inside = torch.full_like(loc, 0.5)
    g_in = gridsample.deform_attn_grads(memory, weight, b, shapes, starts, inside, attn, grad_out)
    np.testing.assert_allclose(g_in['value_bias'], grad_out.sum((0, 1)).numpy(), rtol=1e-12, atol=1e-12)
    # all samples far outside: every gradient is exactly zero
    far = torch.full_like(loc, 5.0)
    g_far = gridsample.deform_attn_grads(memory, weight, b, shapes, starts, far, attn, grad_out)
    for name in NAMES:
        assert not np.any(g_far[name]), name
    # linearity in memory: grad_W = G^T memory and grad_memory = G W for the value gradient G; check one identity
    # that ties them: sum(grad_W * W) = sum(grad_memory * memory) (both equal sum(G * (value - b)))
    lhs = float((grads['value_weight'] * weight.numpy()).sum())
    rhs = float((grads['memory'] * memory.numpy()).sum())
    assert abs(lhs - rhs) <= 1e-10 * max(abs(lhs), 1.0)


def test_training_entry_on_cpu_is_the_reference_under_autograd():
    args, grad_out, _ = tiny(seed=7)
    leaves = [t.clone().requires_grad_(True) if i in (0, 1, 2, 5, 6) else t for i, t in enumerate(args)]
    out = td.ma_deform_attn_train(*leaves)
    (out * grad_out).sum().backward()
    ref = gridsample.deform_attn_grads(*args, grad_out)
    for name, t in zip(NAMES, (leaves[0], leaves[1], leaves[2], leaves[5], leaves[6])):
        np.testing.assert_allclose(t.grad.numpy(), ref[name], rtol=1e-10, atol=1e-12, err_msg=name)


def test_inference_entry_still_rejects_grad():
    # ma_deform_attn stays inference only (reference tests/test_correctness.py:134-140); the CPU path is the
    # reference, which accepts grad, so the rejection is a GPU-path property; the training entry is separate
    assert td.ma_deform_attn_train is not td.ma_deform_attn
    assert 'ma_deform_attn_train' in td.__all__ and 'ma_deform_sample_train' in td.__all__
