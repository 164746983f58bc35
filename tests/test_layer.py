"""The decoder-layer entries on the CPU: the float64 layer oracle pinned against HF transformers' own
RTDetrMultiscaleDeformableAttention (models/rt_detr/modeling_rt_detr.py:623-727, run here in float64 on the CPU),
against closed forms and against planted mistakes; the package's PyTorch layer path and MSDeformAttnLayer
against the oracle; and the C ABI's host-side checks of the layer entries."""

import ctypes

import numpy as np
import pytest
import torch

import marearts_tinydeform_amd as td
from marearts_tinydeform_amd import _native
from oracle import layer as olayer
from inputs import LAYER_CASES, level_index, make_layer

transformers = pytest.importorskip('transformers')


def hf_module(C, H, L, P):
    from transformers import RTDetrConfig
    from transformers.models.rt_detr.modeling_rt_detr import RTDetrMultiscaleDeformableAttention
    cfg = RTDetrConfig(d_model=C, num_feature_levels=L, decoder_attention_heads=H, decoder_n_points=P)
    cfg.disable_custom_kernels = True
    return RTDetrMultiscaleDeformableAttention(cfg, num_heads=H, n_points=P).double().eval()


def load_hf(m, a):
    hidden, memory, ref, shapes, starts, ow, ob, aw, ab, vw, vb, o_w, o_b, H, P, pos = a
    with torch.no_grad():
        m.sampling_offsets.weight.copy_(ow)
        m.sampling_offsets.bias.copy_(ob)
        m.attention_weights.weight.copy_(aw)
        m.attention_weights.bias.copy_(ab)
        m.value_proj.weight.copy_(vw)
        m.value_proj.bias.copy_(vb)
        m.output_proj.weight.copy_(o_w)
        m.output_proj.bias.copy_(o_b)


def run_hf(a, valid=None):
    hidden, memory, ref, shapes, starts, ow, ob, aw, ab, vw, vb, o_w, o_b, H, P, pos = a
    L = shapes.shape[0]
    m = hf_module(hidden.shape[-1], H, L, P)
    load_hf(m, a)
    with torch.no_grad():
        out, attn = m(hidden_states=hidden, attention_mask=valid, encoder_hidden_states=memory,
                      position_embeddings=pos, reference_points=ref, spatial_shapes=shapes,
                      spatial_shapes_list=[tuple(int(v) for v in s) for s in shapes], level_start_index=starts)
    return out.numpy(), attn.numpy()


def oracle(a, padding_mask=None):
    return olayer.layer(*a[:15], position_embeddings=a[15], padding_mask=padding_mask)


SMALL = [c for c in LAYER_CASES if c[1] * c[2] * c[3] <= 2400]


@pytest.mark.parametrize('case', SMALL, ids=[c[0] for c in SMALL])
def test_oracle_matches_transformers(case):
    name, B, Q, H, D, C, levels, P, rd, rl = case
    if H * D != C:  # HF's value_proj / output_proj are C x C
        D = C // H
    a = make_layer(B, min(Q, 40), H, D, C, levels, P, rd, rl, dtype=torch.float64)
    got, got_attn = oracle(a)
    want, want_attn = run_hf(a)
    np.testing.assert_allclose(got_attn, want_attn, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-10)


def test_oracle_matches_transformers_with_mask_and_no_position():
    a = make_layer(2, 30, 4, 16, 64, [(12, 18), (6, 9)], 4, 2, 'L', dtype=torch.float64, pos=False)
    N = a[1].shape[1]
    g = torch.Generator().manual_seed(3)
    padded = torch.rand(2, N, generator=g) < 0.3
    got, _ = oracle(a, padding_mask=padded)
    want, _ = run_hf(a, valid=~padded)
    np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-10)


def test_planted_mistakes_fail_against_transformers():
    a = make_layer(1, 20, 4, 16, 64, [(12, 18), (6, 9)], 4, 2, 'L', dtype=torch.float64)
    want, _ = run_hf(a)
    good, _ = oracle(a)
    assert np.abs(good - want).max() < 1e-9
    # (width, height) normaliser swapped to (height, width)
    b = list(a)
    b[3] = a[3].flip(-1)
    loc_swapped, attn = olayer.locations(a[0], a[2], b[3], a[5], a[6], a[7], a[8], a[13], a[14], a[15])
    from oracle import bruteforce
    core = bruteforce.deform_attn(a[1], a[9], a[10], a[3], a[4], loc_swapped, attn)
    wrong = core @ a[11].double().numpy().T + a[12].double().numpy()
    assert np.abs(wrong - want).max() > 1e-3
    # position embeddings dropped
    wrong2, _ = olayer.layer(*a[:15], position_embeddings=None)
    assert np.abs(wrong2 - want).max() > 1e-3
    # box half-size factor dropped
    c = make_layer(1, 20, 4, 16, 64, [(12, 18), (6, 9)], 4, 4, '1', dtype=torch.float64)
    want_c, _ = run_hf(c)
    ref2 = c[2].clone()
    ref2[..., 2:] *= 2.0
    wrong3, _ = olayer.layer(c[0], c[1], ref2, *c[3:15], position_embeddings=c[15])
    assert np.abs(wrong3 - want_c).max() > 1e-3


def test_closed_forms():
    B, Q, H, C, P = 1, 6, 2, 16, 3
    levels = [(8, 10), (4, 5)]
    shapes, starts, N = level_index(levels)
    L = len(levels)
    hidden = torch.randn(B, Q, C, dtype=torch.float64)
    ref = torch.rand(B, Q, 1, 2, dtype=torch.float64)
    zero_w = torch.zeros(H * L * P * 2, C, dtype=torch.float64)
    zero_a = torch.zeros(H * L * P, C, dtype=torch.float64)
    # no offsets: every sample sits on its reference point; equal logits: uniform attention 1 / (L * P)
    loc, attn = olayer.locations(hidden, ref, shapes, zero_w, None, zero_a, None, H, P)
    np.testing.assert_array_equal(loc, np.broadcast_to(ref.numpy()[:, :, None, :, None, :], loc.shape))
    np.testing.assert_allclose(attn, 1.0 / (L * P), rtol=0, atol=1e-15)
    # a bias-only offset of (W_l, H_l) pixels moves a point by exactly (1, 1) in normalised units
    ob = torch.tensor([[float(w), float(h)] for h, w in levels], dtype=torch.float64)
    ob = ob[None, :, None, :].expand(H, L, P, 2).reshape(-1)
    loc, _ = olayer.locations(hidden, ref, shapes, zero_w, ob, zero_a, None, H, P)
    np.testing.assert_allclose(loc, np.broadcast_to(ref.numpy()[:, :, None, :, None, :] + 1.0, loc.shape), atol=1e-15)
    # a box with bias offset P moves by half its size
    box = torch.cat([ref, torch.full_like(ref, 0.25)], -1)
    ob2 = torch.full((H * L * P * 2,), float(P), dtype=torch.float64)
    loc, _ = olayer.locations(hidden, box, shapes, zero_w, ob2, zero_a, None, H, P)
    np.testing.assert_allclose(loc, np.broadcast_to(ref.numpy()[:, :, None, :, None, :] + 0.125, loc.shape),
                               atol=1e-15)
    # one dominant logit: that sample takes all the weight
    ab = torch.full((H * L * P,), -1e3, dtype=torch.float64)
    ab[::L * P] = 0.0
    _, attn = olayer.locations(hidden, ref, shapes, zero_w, None, zero_a, ab, H, P)
    flat = attn.reshape(B, Q, H, L * P)
    np.testing.assert_allclose(flat[..., 0], 1.0)
    np.testing.assert_allclose(flat[..., 1:], 0.0, atol=1e-300)


@pytest.mark.parametrize('rd,rl', [(2, 'L'), (4, '1')])
def test_reference_layer_matches_oracle(rd, rl):
    a = make_layer(2, 25, 4, 16, 64, [(12, 18), (6, 9)], 4, rd, rl, dtype=torch.float64)
    want, want_attn = oracle(a)
    out, attn = td.ma_deform_attn_layer(*a[:15], position_embeddings=a[15], return_attention_weights=True)
    np.testing.assert_allclose(out.numpy(), want, rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(attn.numpy(), want_attn, rtol=1e-12, atol=1e-13)


def test_module_loads_transformers_state_dict():
    C, H, L, P = 64, 4, 2, 4
    a = make_layer(1, 20, H, C // H, C, [(12, 18), (6, 9)], P, 4, '1', dtype=torch.float64)
    m = hf_module(C, H, L, P)
    load_hf(m, a)
    ours = td.MSDeformAttnLayer(d_model=C, n_levels=L, n_heads=H, n_points=P).double()
    ours.load_state_dict(m.state_dict())
    hidden, memory, ref, shapes, starts = a[:5]
    kw = dict(hidden_states=hidden, encoder_hidden_states=memory, position_embeddings=a[15], reference_points=ref,
              spatial_shapes=shapes, spatial_shapes_list=[tuple(int(v) for v in s) for s in shapes],
              level_start_index=starts)
    with torch.no_grad():
        want = m(**kw)
        got = ours(**kw)
    torch.testing.assert_close(got[0], want[0], rtol=1e-9, atol=1e-10)
    torch.testing.assert_close(got[1], want[1], rtol=1e-12, atol=1e-13)


def test_module_default_init_is_deformable_detr_grid():
    m = td.MSDeformAttnLayer(d_model=32, n_levels=2, n_heads=4, n_points=3)
    b = m.sampling_offsets.bias.view(4, 2, 3, 2)
    # head 0 looks along +x, head 1 along +y; point p at distance p + 1, the same on every level
    torch.testing.assert_close(b[0, 0, :, 0], torch.tensor([1.0, 2.0, 3.0]))
    torch.testing.assert_close(b[1, 1, :, 1], torch.tensor([1.0, 2.0, 3.0]))
    assert torch.equal(b[:, 0], b[:, 1])
    assert torch.count_nonzero(m.sampling_offsets.weight) == 0
    assert torch.count_nonzero(m.attention_weights.weight) == 0


def test_layer_rejects_bad_arguments():
    a = make_layer(1, 4, 2, 8, 16, [(4, 4)], 2, 2, 'L')
    with pytest.raises(ValueError):
        td.ma_deform_attn_layer(*a[:15], mode='fast')
    bad = list(a)
    bad[2] = a[2][..., :1]
    with pytest.raises(RuntimeError, match='reference_points'):
        _native.check_layer(a[1], *[bad[i] for i in (0, 2, 5, 6, 7, 8)], None, a[3], 2, 2, require_gpu=False)
    with pytest.raises(RuntimeError, match='sampling_offsets weight'):
        _native.check_layer(a[1], a[0], a[2], a[5][:-1], a[6], a[7], a[8], None, a[3], 2, 2, require_gpu=False)
    with pytest.raises(RuntimeError, match='levels x points'):
        _native.check_layer(a[1], a[0], a[2], a[5], a[6], a[7], a[8], None, a[3], 2, 65, require_gpu=False)


def test_abi_layer_entries_reject_on_host():
    lib = _native.load()
    assert lib is not None, _native.load_error
    p = 16
    E_ARG = -1
    # reference points with 3 coordinates
    rc = lib.td_layer_fused_forward(1, p, None, p, 1, 3, p, None, p, None, p, p, None, p, p, None, p, None, None,
                                    1, 4, 100, 256, 256, 8, 32, 3, 4, None)
    assert rc == E_ARG and 'coordinates' in lib.td_last_error().decode()
    # reference points with 2 levels when L = 3
    rc = lib.td_layer_fused_forward(1, p, None, p, 2, 2, p, None, p, None, p, p, None, p, p, None, p, None, None,
                                    1, 4, 100, 256, 256, 8, 32, 3, 4, None)
    assert rc == E_ARG and 'levels' in lib.td_last_error().decode()
    # too many query channels
    rc = lib.td_layer_prologue(1, p, None, p, 1, 4, p, None, p, None, p, p, p, 1, 4, 9000, 8, 3, 4, None)
    assert rc == E_ARG and 'query channels' in lib.td_last_error().decode()
    # L * P over the limit
    rc = lib.td_layer_sample_forward(1, p, p, p, p, p, None, p, 1, 4, 100, 8, 32, 4, 20, None)
    assert rc == E_ARG and 'levels x points' in lib.td_last_error().decode()
    # no rows: nothing to do, no device needed
    assert lib.td_layer_fused_forward(1, p, None, p, 1, 4, p, None, p, None, p, p, None, p, p, None, p, None, None,
                                      1, 0, 100, 256, 256, 8, 32, 3, 4, None) == 0
    assert lib.td_layer_prologue(1, p, None, p, 1, 4, p, None, p, None, p, p, p, 1, 0, 256, 8, 3, 4, None) == 0
