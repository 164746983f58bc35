"""Seeded input factories shared by the tests and bench.py.

make() follows the reference test's factory (tests/test_correctness.py:13-26): CPU torch.Generator, memory randn,
weight randn / sqrt(C), bias randn * 0.1, locations = per-query centre rand + spread * 0.3 * randn per
(head, level, point), attention = softmax of randn over L * P, floats cast to dtype.

workload() builds the benchmark configurations: RT-DETR 640 / DINO 4-level / C=1024 shapes with uniform
locations (U[-0.05, 1.05], or U[0, 1] with 10% of samples pushed outside), weight ~ N(0, 1/C), bias ~ N(0, 0.02)
(variance), softmaxed N(0, 1) attention logits.
"""

import torch

# name, B, Q, H, D, C, levels, P   (reference tests/test_correctness.py:33-43)
CASES = [
    ('rtdetr-640', 1, 300, 8, 32, 256, [(80, 80), (40, 40), (20, 20)], 4),
    ('rtdetr-640 b4 few queries', 4, 40, 8, 32, 256, [(80, 80), (40, 40), (20, 20)], 4),
    ('deformable-detr 4 levels non-square', 2, 100, 8, 32, 256, [(100, 152), (50, 76), (25, 38), (13, 19)], 4),
    ('narrow heads', 2, 50, 4, 16, 64, [(32, 48), (16, 24)], 8),
    ('one level many points', 1, 64, 2, 64, 128, [(20, 30)], 16),
    ('wide channels', 1, 40, 12, 64, 768, [(40, 40), (20, 20), (10, 10)], 4),
    ('odd channels (scalar kernel)', 2, 33, 3, 10, 30, [(13, 17), (7, 9)], 4),
    ('channels % 8 != 0, % 4 == 0', 1, 25, 4, 9, 36, [(11, 12)], 4),
]

RTDETR_LEVELS = [(80, 80), (40, 40), (20, 20)]
DINO_LEVELS = [(100, 167), (50, 84), (25, 42), (13, 21)]
LIMIT_LEVELS = [(128, 128), (64, 64), (32, 32), (16, 16)]


def level_index(levels):
    shapes = torch.tensor(levels, dtype=torch.long).reshape(-1, 2)
    sizes = shapes[:, 0] * shapes[:, 1]
    starts = torch.cat([torch.zeros(1, dtype=torch.long), sizes.cumsum(0)[:-1]])
    return shapes, starts, int(sizes.sum())


def make(B, Q, H, D, C, levels, P, dtype=torch.float32, spread=1.0, bias=True, seed=0):
    g = torch.Generator().manual_seed(seed)
    shapes, starts, N = level_index(levels)
    L = len(levels)
    memory = torch.randn(B, N, C, generator=g)
    weight = torch.randn(H * D, C, generator=g) / C ** 0.5
    b = torch.randn(H * D, generator=g) * 0.1 if bias else None
    loc = torch.rand(B, Q, 1, 1, 1, 2, generator=g) + spread * 0.3 * torch.randn(B, Q, H, L, P, 2, generator=g)
    attn = torch.randn(B, Q, H, L * P, generator=g).softmax(-1).view(B, Q, H, L, P)
    return [t if t is None or t.dtype == torch.long else t.to(dtype) for t in
            (memory, weight, b, shapes, starts, loc, attn)]


def workload(B, Q, H, D, C, levels, P, dtype, bias=True, loc_dist='uniform', seed=0):
    """Benchmark inputs (CPU tensors): loc_dist 'uniform' = U[-0.05, 1.05]; 'outside10' = U[0, 1] with a
    seeded 10% of samples moved to U[-0.5, 0) or (1, 1.5]; 'clustered' = per-query centre + 0.05 randn;
    'encoder' = encoder self-attention (Deformable-DETR / DINO): query q is memory token q % N and samples every
    level around that token's normalized centre, 2 randn pixels of the level away."""
    g = torch.Generator().manual_seed(seed)
    shapes, starts, N = level_index(levels)
    L = len(levels)
    memory = torch.randn(B, N, C, generator=g)
    weight = torch.randn(H * D, C, generator=g) / C ** 0.5
    b = torch.randn(H * D, generator=g) * 0.02 ** 0.5 if bias else None
    if loc_dist == 'uniform':
        loc = torch.rand(B, Q, H, L, P, 2, generator=g) * 1.1 - 0.05
    elif loc_dist == 'outside10':
        loc = torch.rand(B, Q, H, L, P, 2, generator=g)
        moved = torch.rand(B, Q, H, L, P, 1, generator=g) < 0.1
        side = torch.rand(B, Q, H, L, P, 2, generator=g) < 0.5
        far = torch.rand(B, Q, H, L, P, 2, generator=g) * 0.5
        outside = torch.where(side, -far - 1e-3, 1.0 + 1e-3 + far)  # U[-0.5, 0) or (1, 1.5]
        loc = torch.where(moved, outside, loc)
    elif loc_dist == 'clustered':
        loc = torch.rand(B, Q, 1, 1, 1, 2, generator=g) + 0.05 * torch.randn(B, Q, H, L, P, 2, generator=g)
    elif loc_dist == 'encoder':
        ref = token_centres(levels)[torch.arange(Q) % N]                          # [Q, 2] (x, y)
        pix = torch.tensor([[w, h] for h, w in levels], dtype=torch.float32)     # [L, 2] (width, height)
        off = 2.0 * torch.randn(B, Q, H, L, P, 2, generator=g)
        loc = ref[None, :, None, None, None, :] + off / pix[None, None, None, :, None, :]
    else:
        raise ValueError(loc_dist)
    attn = torch.randn(B, Q, H, L * P, generator=g).softmax(-1).view(B, Q, H, L, P)
    return [t if t is None or t.dtype == torch.long else t.to(dtype) for t in
            (memory, weight, b, shapes, starts, loc, attn)]


def token_centres(levels):
    """Normalized (x, y) centre of every memory token, level by level: [N, 2]."""
    out = []
    for h, w in levels:
        y, x = torch.meshgrid((torch.arange(h) + 0.5) / h, (torch.arange(w) + 0.5) / w, indexing='ij')
        out.append(torch.stack([x.flatten(), y.flatten()], -1))
    return torch.cat(out)


def to(args, device):
    return [None if t is None else t.to(device) for t in args]


def as_f64(args):
    return [t if t is None or t.dtype == torch.long else t.double() for t in args]


# name, B, Q, H, D, C, levels, P, ref_dim, ref_levels ('1' or 'L')
LAYER_CASES = [
    ('rt-detr decoder boxes', 1, 300, 8, 32, 256, [(80, 80), (40, 40), (20, 20)], 4, 4, '1'),
    ('deformable-detr points per level', 2, 100, 8, 32, 256, [(100, 152), (50, 76), (25, 38), (13, 19)], 4, 2, 'L'),
    ('points shared by levels', 2, 37, 4, 16, 64, [(32, 48), (16, 24)], 8, 2, '1'),
    ('boxes per level, one level', 1, 50, 2, 64, 128, [(20, 30)], 16, 4, 'L'),
    ('wide channels', 1, 40, 12, 64, 768, [(40, 40), (20, 20), (10, 10)], 4, 4, '1'),
    ('odd channels (fallback)', 2, 33, 3, 10, 30, [(13, 17), (7, 9)], 4, 2, 'L'),
]


def make_layer(B, Q, H, D, C, levels, P, ref_dim=4, ref_levels='1', dtype=torch.float32, pos=True, bias=True,
               out_proj=True, seed=0):
    """Inputs of a deformable cross-attention layer (CPU tensors), in ma_deform_attn_layer's argument order up to
    num_points: hidden, memory, reference points, shapes, starts, offsets W/b, attention W/b, value W/b,
    output W/b, H, P; plus position embeddings (or None) last. Offsets are a few pixels (points) or a fraction
    of the box (boxes); attention logits N(0, ~1)."""
    g = torch.Generator().manual_seed(seed)
    shapes, starts, N = level_index(levels)
    L = len(levels)
    HD = H * D
    hidden = torch.randn(B, Q, C, generator=g)
    memory = torch.randn(B, N, C, generator=g)
    RL = 1 if ref_levels == '1' else L
    if ref_dim == 2:
        ref = torch.rand(B, Q, RL, 2, generator=g)
        off_scale = 3.0
    else:
        centre = torch.rand(B, Q, RL, 2, generator=g)
        size = torch.rand(B, Q, RL, 2, generator=g) * 0.3 + 0.02
        ref = torch.cat([centre, size], -1)
        off_scale = 1.0
    off_w = torch.randn(H * L * P * 2, C, generator=g) * (off_scale / C ** 0.5)
    off_b = torch.randn(H * L * P * 2, generator=g) * off_scale if bias else None
    aw_w = torch.randn(H * L * P, C, generator=g) / C ** 0.5
    aw_b = torch.randn(H * L * P, generator=g) * 0.3 if bias else None
    v_w = torch.randn(HD, C, generator=g) / C ** 0.5
    v_b = torch.randn(HD, generator=g) * 0.1 if bias else None
    o_w = torch.randn(C, HD, generator=g) / HD ** 0.5 if out_proj else None
    o_b = torch.randn(C, generator=g) * 0.1 if (out_proj and bias) else None
    position = torch.randn(B, Q, C, generator=g) * 0.5 if pos else None
    cast = [t if t is None or t.dtype == torch.long else t.to(dtype) for t in
            (hidden, memory, ref, shapes, starts, off_w, off_b, aw_w, aw_b, v_w, v_b, o_w, o_b)]
    return cast + [H, P, None if position is None else position.to(dtype)]
