"""Write the golden fixtures tests/golden/*.npz (run from the repository root: python tests/golden/make_golden.py).

Each fixture holds seeded inputs and the float64 output of value projection + multi-scale deformable attention.
Inputs are rounded to values exactly representable in bfloat16 (hence also in float16 and float32), so one expected
output serves every element type. The expected output comes from oracle.bruteforce and, where torch's grid_sample
defines the result (every fixture except the ones exercising the clamp and token-range rules), is checked at
generation time against oracle.gridsample in float64 (grid_sample is the library routine whose semantics the
reference operator reproduces, marearts_tinydeform/reference.py:37). The reference repository itself ships no
golden vectors.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import bruteforce, gridsample  # noqa: E402

# name, B, Q, H, D, C, levels, P, spread, bias
CASES = [
    ('three_levels', 1, 6, 4, 8, 32, [(8, 8), (4, 4), (2, 2)], 4, 1.0, True),
    ('batch2_two_levels', 2, 5, 4, 8, 32, [(8, 8), (4, 4)], 2, 1.0, True),
    ('four_levels_nonsquare', 2, 4, 2, 16, 32, [(10, 15), (5, 8), (3, 4), (2, 2)], 2, 1.0, True),
    ('narrow_heads_p8', 1, 4, 4, 4, 16, [(6, 9), (3, 5)], 8, 1.0, True),
    ('one_level_p16', 1, 4, 2, 16, 32, [(5, 7)], 16, 1.0, True),
    ('odd_channels', 2, 5, 3, 10, 30, [(7, 9), (3, 4)], 4, 1.0, True),
    ('channels_36', 1, 5, 4, 9, 36, [(5, 6)], 4, 1.0, True),
    ('no_bias', 1, 6, 4, 8, 32, [(8, 8), (4, 4)], 4, 1.0, False),
    ('far_outside', 2, 5, 4, 8, 32, [(9, 11), (5, 6)], 4, 200.0, True),
    ('max_level_points', 1, 3, 2, 8, 16, [(4, 4), (3, 3), (2, 2), (1, 1)], 16, 1.0, True),
]


def bf16_exact(t):
    return t.to(torch.bfloat16).to(torch.float32)


def make(B, Q, H, D, C, levels, P, spread, bias, seed):
    g = torch.Generator().manual_seed(seed)
    shapes = torch.tensor(levels, dtype=torch.long)
    sizes = shapes[:, 0] * shapes[:, 1]
    starts = torch.cat([torch.zeros(1, dtype=torch.long), sizes.cumsum(0)[:-1]])
    N, L = int(sizes.sum()), len(levels)
    memory = bf16_exact(torch.randn(B, N, C, generator=g))
    weight = bf16_exact(torch.randn(H * D, C, generator=g) / C ** 0.5)
    b = bf16_exact(torch.randn(H * D, generator=g) * 0.1) if bias else None
    loc = bf16_exact(torch.rand(B, Q, 1, 1, 1, 2, generator=g) + spread * 0.3 * torch.randn(B, Q, H, L, P, 2,
                                                                                            generator=g))
    attn = bf16_exact(torch.randn(B, Q, H, L * P, generator=g).softmax(-1).view(B, Q, H, L, P))
    return [memory, weight, b, shapes, starts, loc, attn]


def save(name, args, expected):
    memory, weight, b, shapes, starts, loc, attn = args
    out = dict(memory=memory.numpy(), weight=weight.numpy(), shapes=shapes.numpy(), starts=starts.numpy(),
               loc=loc.numpy(), attn=attn.numpy(), expected=expected)
    if b is not None:
        out['bias'] = b.numpy()
    np.savez_compressed(os.path.join(HERE, f'{name}.npz'), **out)


def main():
    for i, (name, B, Q, H, D, C, levels, P, spread, bias) in enumerate(CASES):
        args = make(B, Q, H, D, C, levels, P, spread, bias, seed=100 + i)
        expected = bruteforce.deform_attn(*args)
        f64 = [t if t is None or t.dtype == torch.long else t.double() for t in args]
        gs = gridsample.deform_attn(*f64).numpy()
        assert np.abs(expected - gs).max() <= 1e-12, name
        save(name, args, expected)
        print(f'{name:24s} max |out| {np.abs(expected).max():.3f}')

    # clamp rule: infinite, NaN and huge coordinates sample nothing (reference csrc/ma_deform_fused.cu:87-89)
    args = make(1, 6, 2, 8, 16, [(7, 9), (4, 5)], 2, 1.0, True, seed=200)
    loc = args[5]
    loc[0, 0, :, :, :, 0] = float('inf')
    loc[0, 1, :, :, :, 1] = float('-inf')
    loc[0, 2, :, 0, 0, 0] = float('nan')
    loc[0, 3] = 4096.0  # far outside, exact in bfloat16 and float16
    expected = bruteforce.deform_attn(*args)
    assert np.isfinite(expected).all() and not expected[0, 0].any() and not expected[0, 3].any()
    save('nonfinite_locations', args, expected)
    print('nonfinite_locations')

    # token range rule: the second level claims 16 tokens but memory ends after 24, so tokens 24..31 drop
    # (reference csrc/ma_deform_fused.cu:95-96)
    args = make(1, 6, 2, 8, 16, [(4, 4), (4, 4)], 4, 0.5, True, seed=201)
    args[0] = args[0][:, :24].contiguous()
    expected = bruteforce.deform_attn(*args)
    save('token_range', args, expected)
    print('token_range')


if __name__ == '__main__':
    main()
