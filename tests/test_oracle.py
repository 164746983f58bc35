"""Pins of the oracle (CPU only). The reference ships no golden vectors, so the float64 brute force
(oracle.bruteforce) is pinned by:
  1. torch's grid_sample (bilinear, zeros, align_corners=False), the library routine whose result the reference
     operator reproduces (marearts_tinydeform/reference.py:37), on the reference test's 8 geometries;
  2. an independent route on tiny inputs: bilinear interpolation of an explicitly zero-padded image (no in-map
     tests at all), written from the definition;
  3. closed forms: pixel-centre locations, one-hot attention, all samples outside, identity weight, bias share,
     empty queries, non-finite locations, the token-range guard;
  4. invariants: linearity, fused order == project order;
  5. planted mistakes (in wrapped copies of the oracle) that each of these checks must reject.
"""

import math

import numpy as np
import pytest
import torch

from oracle import bruteforce, gridsample
from inputs import CASES, as_f64, level_index, make


def gs64(args):
    return gridsample.deform_attn(*as_f64(args)).numpy()


@pytest.mark.parametrize('case', CASES, ids=[c[0] for c in CASES])
def test_bruteforce_matches_grid_sample(case):
    name, B, Q, H, D, C, levels, P = case
    args = make(B, min(Q, 24), H, D, C, levels, P)
    assert np.abs(bruteforce.deform_attn(*args) - gs64(args)).max() <= 1e-12


@pytest.mark.parametrize('spread', [0.3, 1.0, 3.0])
def test_bruteforce_matches_grid_sample_near_and_outside_edges(spread):
    args = make(2, 16, 4, 8, 16, [(7, 5), (3, 9), (1, 2)], 4, spread=spread, seed=7)
    assert np.abs(bruteforce.deform_attn(*args) - gs64(args)).max() <= 1e-12


def padded_image_route(args):
    """out[b, q, h*D:(h+1)*D] by interpolating each level image after padding it with zeros, from the definition of
    bilinear interpolation; pure Python loops, tiny inputs only."""
    memory, weight, bias, shapes, starts, loc, attn = [None if t is None else t.double() if t.is_floating_point()
                                                       else t for t in args]
    B, N, _ = memory.shape
    _, Q, H, L, P, _ = loc.shape
    value = memory @ weight.T + (0 if bias is None else bias)
    D = value.shape[-1] // H
    out = torch.zeros(B, Q, H * D, dtype=torch.float64)
    pad = 4
    for b in range(B):
        for h in range(H):
            for lvl in range(L):
                hl, wl, st = int(shapes[lvl, 0]), int(shapes[lvl, 1]), int(starts[lvl])
                img = torch.zeros(hl + 2 * pad, wl + 2 * pad, D, dtype=torch.float64)
                img[pad:pad + hl, pad:pad + wl] = value[b, st:st + hl * wl, h * D:(h + 1) * D].reshape(hl, wl, D)
                for q in range(Q):
                    for p in range(P):
                        x = float(loc[b, q, h, lvl, p, 0]) * wl - 0.5 + pad
                        y = float(loc[b, q, h, lvl, p, 1]) * hl - 0.5 + pad
                        if not (0 <= x < wl + 2 * pad - 1 and 0 <= y < hl + 2 * pad - 1):
                            continue  # every corner lies in the zero padding
                        x0, y0 = math.floor(x), math.floor(y)
                        fx, fy = x - x0, y - y0
                        v = ((1 - fx) * (1 - fy) * img[y0, x0] + fx * (1 - fy) * img[y0, x0 + 1]
                             + (1 - fx) * fy * img[y0 + 1, x0] + fx * fy * img[y0 + 1, x0 + 1])
                        out[b, q, h * D:(h + 1) * D] += float(attn[b, q, h, lvl, p]) * v
    return out.numpy()


@pytest.mark.parametrize('seed', [0, 1, 2])
def test_bruteforce_matches_zero_padded_interpolation(seed):
    args = make(2, 5, 3, 4, 6, [(4, 6), (3, 2)], 3, spread=0.8, seed=seed)
    assert np.abs(bruteforce.deform_attn(*args) - padded_image_route(args)).max() <= 1e-12


def test_pixel_centre_location_reads_exactly_one_token():
    # power-of-two map sizes: (i + 0.5) / W is exact in binary, so x = loc * W - 0.5 lands exactly on i
    B, Q, H, D, C, levels, P = 1, 6, 2, 4, 8, [(4, 8), (2, 4)], 2
    args = make(B, Q, H, D, C, levels, P, seed=3)
    shapes, starts, N = level_index(levels)
    g = torch.Generator().manual_seed(11)
    loc = torch.empty(B, Q, H, len(levels), P, 2, dtype=torch.float64)
    expect_tok = torch.empty(B, Q, H, len(levels), P, dtype=torch.long)
    for lvl, (hl, wl) in enumerate(levels):
        i = torch.randint(0, wl, (B, Q, H, P), generator=g)
        j = torch.randint(0, hl, (B, Q, H, P), generator=g)
        loc[:, :, :, lvl, :, 0] = (i + 0.5) / wl
        loc[:, :, :, lvl, :, 1] = (j + 0.5) / hl
        expect_tok[:, :, :, lvl] = int(starts[lvl]) + j * wl + i
    args = as_f64(args)
    args[5] = loc
    tok, wt = bruteforce.corner_table(args[3], args[4], args[5], args[6], N)
    w = wt.reshape(B, Q, H, len(levels), P, 4)
    t = tok.reshape(B, Q, H, len(levels), P, 4)
    np.testing.assert_array_equal(t[..., 0], expect_tok.numpy())
    np.testing.assert_array_equal(w[..., 0], args[6].numpy())
    assert not w[..., 1:].any()
    value = bruteforce.project(args[0], args[1], args[2]).reshape(B, N, H, D)
    out = bruteforce.deform_attn(*args).reshape(B, Q, H, D)
    manual = np.zeros((B, Q, H, D))
    for q in range(Q):
        for h in range(H):
            for lvl in range(len(levels)):
                for p in range(P):
                    manual[0, q, h] += args[6][0, q, h, lvl, p].item() * value[0, expect_tok[0, q, h, lvl, p], h]
    assert np.abs(out - manual).max() <= 1e-13


def test_one_hot_attention_is_one_bilinear_sample():
    B, Q, H, D, C, levels, P = 1, 4, 2, 3, 6, [(6, 5), (3, 3)], 3
    args = as_f64(make(B, Q, H, D, C, levels, P, seed=4))
    attn = torch.zeros_like(args[6])
    attn[..., 1, 2] = 1.0  # level 1, point 2 only
    args[6] = attn
    loc = args[5]
    hl, wl = levels[1]
    value = bruteforce.project(args[0], args[1], args[2]).reshape(B, -1, H, D)
    st = levels[0][0] * levels[0][1]
    out = bruteforce.deform_attn(*args).reshape(B, Q, H, D)
    for q in range(Q):
        for h in range(H):
            x = loc[0, q, h, 1, 2, 0].item() * wl - 0.5
            y = loc[0, q, h, 1, 2, 1].item() * hl - 0.5
            x0, y0 = math.floor(x), math.floor(y)
            acc = np.zeros(D)
            for yy, wy in ((y0, 1 - (y - y0)), (y0 + 1, y - y0)):
                for xx, wx in ((x0, 1 - (x - x0)), (x0 + 1, x - x0)):
                    if 0 <= xx < wl and 0 <= yy < hl:
                        acc += wx * wy * value[0, st + yy * wl + xx, h]
            assert np.abs(out[0, q, h] - acc).max() <= 1e-13


def test_all_samples_outside_give_exact_zero_bias_included():
    args = make(2, 7, 4, 8, 16, [(9, 11), (5, 6)], 4, seed=5)
    for far in (-3.0, 5.0, 1e6, float('inf')):
        args[5] = torch.full_like(args[5], far)
        out = bruteforce.deform_attn(*args)
        assert out.shape == (2, 7, 32) and not out.any()
        assert not bruteforce.deform_attn_fused_order(*args).any()


def test_identity_weight_samples_raw_memory():
    B, Q, H, D, levels, P = 2, 5, 4, 6, [(6, 7), (3, 3)], 4
    args = make(B, Q, H, D, H * D, levels, P, bias=False, seed=6)
    args[1] = torch.eye(H * D)
    direct = bruteforce.sample(args[0], H, *args[3:])
    assert np.abs(bruteforce.deform_attn(*args) - direct).max() <= 1e-15


def test_bias_share_is_bias_times_weight_sum():
    # memory = 0 and every corner inside the map: out = bias * sum(attention) = bias (softmax sums to 1)
    levels = [(6, 8), (4, 5)]
    args = as_f64(make(1, 9, 3, 4, 8, levels, 4, seed=8))
    args[0] = torch.zeros_like(args[0])
    g = torch.Generator().manual_seed(9)
    args[5] = (0.2 + 0.6 * torch.rand(args[5].shape, generator=g)).double()
    args[6] = args[6] / args[6].sum(dim=(-2, -1), keepdim=True)  # sums to 1 in float64
    out = bruteforce.deform_attn(*args).reshape(1, 9, 3, 4)
    np.testing.assert_allclose(out, np.broadcast_to(args[2].numpy().reshape(3, 4), out.shape), atol=1e-14)


def test_empty_queries():
    args = make(2, 0, 4, 8, 32, [(9, 11)], 4)
    assert bruteforce.deform_attn(*args).shape == (2, 0, 32)
    assert gs64(args).shape == (2, 0, 32)


def test_linear_in_memory_and_attention():
    a = make(1, 8, 2, 4, 8, [(6, 6), (3, 3)], 2, bias=False, seed=10)
    b = make(1, 8, 2, 4, 8, [(6, 6), (3, 3)], 2, bias=False, seed=11)
    mix = list(a)
    mix[0] = 2.0 * a[0].double() - 3.0 * b[0].double()
    lhs = bruteforce.deform_attn(*mix)
    rhs = 2.0 * bruteforce.deform_attn(*a) - 3.0 * bruteforce.deform_attn(*[b[0]] + a[1:])
    assert np.abs(lhs - rhs).max() <= 1e-12
    mix = list(a)
    mix[6] = 0.5 * a[6].double() + 4.0 * b[6].double()
    lhs = bruteforce.deform_attn(*mix)
    rhs = 0.5 * bruteforce.deform_attn(*a) + 4.0 * bruteforce.deform_attn(*a[:6] + [b[6]])
    assert np.abs(lhs - rhs).max() <= 1e-12


def test_fused_order_equals_project_order():
    for name, B, Q, H, D, C, levels, P in CASES:
        args = make(B, min(Q, 16), H, D, C, levels, P)
        assert np.abs(bruteforce.deform_attn(*args) - bruteforce.deform_attn_fused_order(*args)).max() <= 1e-12


def test_nonfinite_and_huge_locations_sample_nothing():
    args = as_f64(make(1, 6, 2, 4, 8, [(7, 9), (4, 5)], 2, seed=12))
    loc = args[5]
    loc[0, 0, :, :, :, 0] = float('inf')
    loc[0, 1, :, :, :, 1] = float('-inf')
    loc[0, 2, :, :, :, :] = float('nan')
    loc[0, 3] = 1e300
    out = bruteforce.deform_attn(*args)
    assert np.isfinite(out).all()
    assert not out[0, :4].any()
    clean = [t.clone() if t is not None else None for t in args]
    clean[5] = clean[5][:, 4:].contiguous()
    clean[6] = clean[6][:, 4:].contiguous()
    assert np.abs(out[:, 4:] - bruteforce.deform_attn(*clean)).max() == 0


def test_token_range_guard_drops_tokens_past_n():
    # level 1 claims 16 tokens starting at 16, memory holds 24: tokens 24..31 must contribute nothing, which equals
    # keeping them with zero rows (bias off, so a zero row contributes zero)
    args = as_f64(make(1, 10, 2, 4, 8, [(4, 4), (4, 4)], 4, spread=0.5, bias=False, seed=13))
    padded = list(args)
    zeros = args[0].clone()
    zeros[:, 24:] = 0
    padded[0] = zeros
    truncated = list(args)
    truncated[0] = args[0][:, :24].contiguous()
    a = bruteforce.deform_attn(*truncated)
    b = bruteforce.deform_attn(*padded)
    assert np.abs(a - b).max() <= 1e-15
    tok, _ = bruteforce.corner_table(args[3], args[4], args[5], args[6], 24)
    assert tok.max() < 24


# ---- planted mistakes: each wrapped copy of the oracle must fail a pin above ---------------------------------

def _mutants():
    orig = bruteforce.corner_table

    def no_half_pixel(shapes, starts, loc, attn, n, mask=None):  # x = loc * W (align_corners mix-up)
        wh = torch.as_tensor(np.asarray(shapes))[:, [1, 0]].double()
        return orig(shapes, starts, torch.as_tensor(np.asarray(loc)) + 0.5 / wh[:, None, :], attn, n, mask)

    def swapped_xy(shapes, starts, loc, attn, n, mask=None):
        return orig(shapes, starts, torch.as_tensor(np.asarray(loc)).flip(-1), attn, n, mask)

    def dropped_corner(shapes, starts, loc, attn, n, mask=None):
        tok, wt = orig(shapes, starts, loc, attn, n, mask)
        wt = wt.copy()
        wt[..., 3::4] = 0.0
        return tok, wt

    def transposed_bilinear(shapes, starts, loc, attn, n, mask=None):  # corner k=1 and k=2 weights exchanged
        tok, wt = orig(shapes, starts, loc, attn, n, mask)
        wt = wt.copy()
        wt[..., 1::4], wt[..., 2::4] = wt[..., 2::4].copy(), wt[..., 1::4].copy()
        return tok, wt

    def wrong_level_start(shapes, starts, loc, attn, n, mask=None):
        return orig(shapes, np.roll(np.asarray(starts), 1), loc, attn, n, mask)

    return {'no half-pixel offset': no_half_pixel, 'swapped x/y': swapped_xy, 'dropped corner': dropped_corner,
            'transposed bilinear weights': transposed_bilinear, 'wrong level start': wrong_level_start}


@pytest.mark.parametrize('mutant', sorted(_mutants()))
def test_planted_mistake_fails_grid_sample_pin(mutant, monkeypatch):
    args = make(2, 12, 4, 8, 16, [(10, 15), (5, 8)], 4, seed=14)
    ref = gs64(args)
    monkeypatch.setattr(bruteforce, 'corner_table', _mutants()[mutant])
    assert np.abs(bruteforce.deform_attn(*args) - ref).max() > 1e-3


def test_planted_bias_mistake_fails_outside_zero_pin():
    # adding the bias once per row instead of bias * (sum of in-map weights)
    args = make(2, 7, 4, 8, 16, [(9, 11), (5, 6)], 4, seed=15)
    args[5] = torch.full_like(args[5], 5.0)
    no_bias = list(args)
    no_bias[2] = None
    wrong = bruteforce.deform_attn_fused_order(*no_bias) + args[2].double().numpy()
    assert wrong.any()  # the closed form (exact zero) rejects it
    assert not bruteforce.deform_attn_fused_order(*args).any()


# ---- value padding mask -------------------------------------------------------------------------------------

def random_mask(B, N, seed, frac=0.3):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(B, N, generator=g) < frac


@pytest.mark.parametrize('case', CASES[:4], ids=[c[0] for c in CASES[:4]])
def test_padding_mask_drops_corners_like_zeroed_values(case):
    # dropping corners on padded tokens == zeroing their value rows after the projection (the decoder's
    # value.masked_fill(mask[..., None], 0)), checked three ways: corner-dropping brute force, zeroed-value brute
    # force, grid_sample on zeroed values
    name, B, Q, H, D, C, levels, P = case
    args = make(B, min(Q, 16), H, D, C, levels, P, seed=21)
    mask = random_mask(B, args[0].shape[1], 22)
    dropped = bruteforce.deform_attn(*args, padding_mask=mask)
    value = bruteforce.project(args[0], args[1], args[2])
    value[mask.numpy()] = 0.0
    zeroed = bruteforce.sample(value, H, *args[3:])
    gs = gridsample.deform_attn(*as_f64(args), padding_mask=mask).numpy()
    assert np.abs(dropped - zeroed).max() <= 1e-13
    assert np.abs(dropped - gs).max() <= 1e-12
    assert np.abs(dropped - bruteforce.deform_attn(*args)).max() > 1e-3  # the mask matters


def test_padding_mask_all_and_none():
    args = make(2, 6, 2, 4, 8, [(5, 6), (3, 3)], 2, seed=23)
    N = args[0].shape[1]
    full = bruteforce.deform_attn(*args, padding_mask=torch.ones(2, N, dtype=torch.bool))
    assert not full.any()  # every token padded: exact zero, bias included
    none = bruteforce.deform_attn(*args, padding_mask=torch.zeros(2, N, dtype=torch.bool))
    assert np.abs(none - bruteforce.deform_attn(*args)).max() == 0


# ---- per-level point counts and D-FINE's discrete method -----------------------------------------------------

def dfine_inputs(B, Q, H, D, levels, points, seed, spread=0.4):
    g = torch.Generator().manual_seed(seed)
    shapes, starts, N = level_index(levels)
    J = sum(points)
    value = torch.randn(B, N, H, D, generator=g, dtype=torch.float64)
    loc = (torch.rand(B, Q, 1, 1, 2, generator=g) + spread * torch.randn(B, Q, H, J, 2, generator=g)).double()
    attn = torch.randn(B, Q, H, J, generator=g).softmax(-1).double()
    return value, shapes, starts, loc, attn


@pytest.mark.parametrize('points', [[3, 6, 3], [4, 4, 4], [2, 1, 5, 3], [8]])
@pytest.mark.parametrize('method', ['default', 'discrete'])
def test_sample_v2_matches_dfine_restatement(points, method):
    levels = [(12, 9), (6, 5), (3, 3), (2, 2)][:len(points)]
    value, shapes, starts, loc, attn = dfine_inputs(2, 7, 3, 4, levels, points, seed=31)
    ref = gridsample.deform_sample_v2(value, shapes, loc, attn, points, method).numpy()
    got = bruteforce.sample_v2(value, shapes, starts, loc, attn, points, method)
    assert np.abs(got - ref).max() <= 1e-12


@pytest.mark.parametrize('points', [[3, 6, 3], [4, 4, 4], [2, 1, 5, 3], [8]])
@pytest.mark.parametrize('method', ['default', 'discrete'])
def test_sample_v2_matches_transformers(points, method):
    # the library routine itself: transformers' D-FINE core (models/d_fine/modeling_d_fine.py:150-216, installed in
    # this image), run in float64 on the CPU, with locations that reach past every edge of the maps
    dfine = pytest.importorskip('transformers.models.d_fine.modeling_d_fine')
    levels = [(12, 9), (6, 5), (3, 3), (2, 2)][:len(points)]
    value, shapes, starts, loc, attn = dfine_inputs(2, 7, 3, 4, levels, points, seed=41, spread=0.6)
    assert (loc < 0).any() and (loc > 1).any()
    ref = dfine.multi_scale_deformable_attention_v2(value, [tuple(int(v) for v in s) for s in shapes], loc, attn,
                                                    points, method).numpy()
    got = bruteforce.sample_v2(value, shapes, starts, loc, attn, points, method)
    assert got.shape == ref.shape
    assert np.abs(got - ref).max() <= 1e-12


def test_sample_v2_uniform_points_equals_sample():
    levels = [(12, 9), (6, 5), (3, 3)]
    value, shapes, starts, loc, attn = dfine_inputs(2, 5, 3, 4, levels, [4, 4, 4], seed=32)
    v1 = bruteforce.sample(value.reshape(2, -1, 12), 3, shapes, starts, loc.reshape(2, 5, 3, 3, 4, 2),
                           attn.reshape(2, 5, 3, 3, 4))
    assert np.abs(bruteforce.sample_v2(value, shapes, starts, loc, attn, [4, 4, 4]) - v1).max() == 0


def test_discrete_pixel_closed_form():
    # a location inside pixel (i, j) reads exactly value[start + j * W + i]; outside the map it clamps to the edge
    levels = [(4, 8)]
    value, shapes, starts, loc, attn = dfine_inputs(1, 3, 1, 2, levels, [2], seed=33)
    loc = loc.clone()
    loc[0, 0, 0, 0] = torch.tensor([(5 + 0.3) / 8, (2 + 0.6) / 4])   # pixel x=5 (rounds up from 5.8: 5.3 + 0.5)
    loc[0, 0, 0, 1] = torch.tensor([-3.0, 9.0])                       # clamps to x=0, y=3
    attn = torch.zeros_like(attn)
    attn[0, 0, 0, 0], attn[0, 0, 0, 1] = 0.25, 0.75
    out = bruteforce.sample_v2(value, shapes, starts, loc, attn, [2], 'discrete')
    # x = int(5.3 + 0.5) = 5, y = int(2.6 + 0.5) = 3
    expect = 0.25 * value[0, 3 * 8 + 5, 0].numpy() + 0.75 * value[0, 3 * 8 + 0, 0].numpy()
    assert np.abs(out[0, 0] - expect).max() <= 1e-15


def test_planted_discrete_mistake_fails_restatement_pin(monkeypatch):
    # rounding without the + 0.5 (floor instead of nearest) must disagree with the D-FINE restatement
    levels = [(12, 9), (6, 5)]
    value, shapes, starts, loc, attn = dfine_inputs(2, 7, 3, 4, levels, [3, 5], seed=34)
    ref = gridsample.deform_sample_v2(value, shapes, loc, attn, [3, 5], 'discrete').numpy()
    orig = bruteforce.corner_table_v2

    def floor_not_round(shapes_, starts_, loc_, attn_, n, pts, method='default', mask=None):
        wh = torch.as_tensor(np.asarray(shapes_))[:, [1, 0]].double()
        level_of = np.repeat(np.arange(len(pts)), pts)
        return orig(shapes_, starts_, torch.as_tensor(np.asarray(loc_)) - 0.5 / wh[level_of], attn_, n, pts, method,
                    mask)

    monkeypatch.setattr(bruteforce, 'corner_table_v2', floor_not_round)
    assert np.abs(bruteforce.sample_v2(value, shapes, starts, loc, attn, [3, 5], 'discrete') - ref).max() > 1e-3
