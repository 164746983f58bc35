"""Torch restatement of the reference's PyTorch path. TEST INFRASTRUCTURE ONLY: imported by tests/ and by
bench.py's cpu_baseline leg (it is the CPU path the reference runs for CPU tensors), never by the product.

deform_attn follows marearts_tinydeform/reference.py:13-40: value = F.linear(memory, W, b), then for each level
F.grid_sample(bilinear, zeros, align_corners=False) of that level's [B*H, D, h, w] map at 2 * loc - 1, then the
attention-weighted sum over levels and points. Runs in the dtype it is given (float32 for the CPU baseline,
float64 to cross-check the brute force).

deform_attn_grads is the gradient oracle of the backward: PyTorch's autograd through deform_attn in float64
(grid_sample's and F.linear's own backward), pinned in tests/test_backward.py against central finite differences
of the numpy brute force (oracle.bruteforce.deform_attn).
"""

import torch
import torch.nn.functional as F


def deform_attn(memory, value_weight, value_bias, spatial_shapes, level_start_index, sampling_locations,
                attention_weights, padding_mask=None):
    """padding_mask ([B, N] bool, True = padded) zeroes those value rows after the projection, the way
    Deformable-DETR decoders mask padded tokens."""
    B, N, _ = memory.shape
    _, Q, H, L, P, _ = sampling_locations.shape
    value = F.linear(memory, value_weight, value_bias)
    if padding_mask is not None:
        value = value.masked_fill(padding_mask.bool()[..., None], 0)
    value = value.view(B, N, H, -1)
    D = value.shape[-1]
    grids = 2 * sampling_locations - 1
    acc = torch.zeros(B * H, D, Q, dtype=value.dtype)
    for lvl in range(L):
        h, w = int(spatial_shapes[lvl, 0]), int(spatial_shapes[lvl, 1])
        s = int(level_start_index[lvl])
        v = value[:, s:s + h * w].permute(0, 2, 3, 1).reshape(B * H, D, h, w)
        g = grids[:, :, :, lvl].transpose(1, 2).reshape(B * H, Q, P, 2)
        smp = F.grid_sample(v, g, mode='bilinear', padding_mode='zeros', align_corners=False)  # [B*H, D, Q, P]
        a = attention_weights[:, :, :, lvl].transpose(1, 2).reshape(B * H, 1, Q, P)
        acc = acc + torch.einsum('ndqp,ndqp->ndq', smp, a.expand_as(smp))
    return acc.view(B, H * D, Q).transpose(1, 2).contiguous()


def deform_sample_v2(value, spatial_shapes, sampling_locations, attention_weights, num_points_list,
                     method='default'):
    """D-FINE's deformable attention core, restating transformers models/d_fine/modeling_d_fine.py:150-216
    (multi_scale_deformable_attention_v2): value [B, N, H, D], loc [B, Q, H, sum(P), 2], attn [B, Q, H, sum(P)];
    per level, grid_sample (method 'default') or the nearest-pixel gather of (loc * [W, H] + 0.5) cast to int64
    and clamped into the map ('discrete'), then the attention-weighted sum -> [B, Q, H * D]."""
    B, N, H, D = value.shape
    _, Q, _, J, _ = sampling_locations.shape
    levels = [(int(h), int(w)) for h, w in spatial_shapes]
    per_level = value.permute(0, 2, 3, 1).flatten(0, 1).split([h * w for h, w in levels], dim=-1)
    grids = 2 * sampling_locations - 1 if method == 'default' else sampling_locations
    grids = grids.permute(0, 2, 1, 3, 4).flatten(0, 1).split(list(num_points_list), dim=-2)  # [B*H, Q, P_l, 2]
    sampled = []
    for lvl, (h, w) in enumerate(levels):
        v = per_level[lvl].reshape(B * H, D, h, w)
        g = grids[lvl]
        if method == 'default':
            sampled.append(F.grid_sample(v, g, mode='bilinear', padding_mode='zeros', align_corners=False))
        else:
            coord = (g * torch.tensor([[w, h]], dtype=g.dtype) + 0.5).to(torch.int64)
            x = coord[..., 0].clamp(0, w - 1)
            y = coord[..., 1].clamp(0, h - 1)
            n = torch.arange(B * H)[:, None, None]
            sampled.append(v[n, :, y, x].permute(0, 3, 1, 2))  # [B*H, D, Q, P_l]
    a = attention_weights.permute(0, 2, 1, 3).reshape(B * H, 1, Q, J)
    out = (torch.cat(sampled, dim=-1) * a).sum(-1)  # [B*H, D, Q]
    return out.view(B, H * D, Q).transpose(1, 2).contiguous()


def deform_attn_grads(memory, value_weight, value_bias, spatial_shapes, level_start_index, sampling_locations,
                      attention_weights, grad_out, padding_mask=None, align_corners=False):
    """float64 gradients of sum(deform_attn(...) * grad_out) with respect to memory, value_weight, value_bias,
    sampling_locations and attention_weights, as numpy arrays keyed by those names (value_bias: None without one).
    align_corners=True exists only to plant a mistake the finite-difference pin must reject."""
    def leaf(t):
        return None if t is None else t.detach().cpu().double().requires_grad_(True)

    mem, w, b, loc, attn = (leaf(t) for t in (memory, value_weight, value_bias, sampling_locations,
                                              attention_weights))
    shapes, starts = spatial_shapes.cpu(), level_start_index.cpu()
    mask = None if padding_mask is None else padding_mask.cpu()
    if align_corners:
        out = _deform_attn_aligned(mem, w, b, shapes, starts, loc, attn, mask)
    else:
        out = deform_attn(mem, w, b, shapes, starts, loc, attn, padding_mask=mask)
    (out * grad_out.detach().cpu().double()).sum().backward()
    grads = {'memory': mem.grad, 'value_weight': w.grad, 'value_bias': None if b is None else b.grad,
             'sampling_locations': loc.grad, 'attention_weights': attn.grad}
    return {k: None if v is None else v.numpy() for k, v in grads.items()}


def _deform_attn_aligned(memory, value_weight, value_bias, spatial_shapes, level_start_index, sampling_locations,
                         attention_weights, padding_mask=None):
    """deform_attn with align_corners=True: a deliberate mistake, used only by the oracle's planted-mistake test."""
    B, N, _ = memory.shape
    _, Q, H, L, P, _ = sampling_locations.shape
    value = F.linear(memory, value_weight, value_bias)
    if padding_mask is not None:
        value = value.masked_fill(padding_mask.bool()[..., None], 0)
    value = value.view(B, N, H, -1)
    D = value.shape[-1]
    grids = 2 * sampling_locations - 1
    acc = torch.zeros(B * H, D, Q, dtype=value.dtype)
    for lvl in range(L):
        h, w = int(spatial_shapes[lvl, 0]), int(spatial_shapes[lvl, 1])
        s = int(level_start_index[lvl])
        v = value[:, s:s + h * w].permute(0, 2, 3, 1).reshape(B * H, D, h, w)
        g = grids[:, :, :, lvl].transpose(1, 2).reshape(B * H, Q, P, 2)
        smp = F.grid_sample(v, g, mode='bilinear', padding_mode='zeros', align_corners=True)
        a = attention_weights[:, :, :, lvl].transpose(1, 2).reshape(B * H, 1, Q, P)
        acc = acc + (smp * a).sum(-1)
    return acc.view(B, H * D, Q).transpose(1, 2).contiguous()
