"""The standard path in plain PyTorch: project every memory token, then sample each level with grid_sample.

This is the public `ma_deform_attn_reference` of the API (reference marearts_tinydeform/reference.py:13-40):
the computation Deformable-DETR-style decoders run, usable on CPU and GPU, with autograd. `ma_deform_attn` routes
CPU tensors here. Bilinear interpolation, zero padding, align_corners=False.
"""

import torch
import torch.nn.functional as F


def ma_deform_attn_reference(memory, value_weight, value_bias, spatial_shapes, level_start_index,
                             sampling_locations, attention_weights, padding_mask=None):
    """value = memory @ value_weight.T + value_bias, then multi-scale deformable attention.

    memory              [B, N, C]
    value_weight        [H * D, C]      (an nn.Linear weight)
    value_bias          [H * D] or None
    spatial_shapes      [L, 2] int64    (height, width) of each level, tokens laid out level by level
    level_start_index   [L] int64       first token of each level
    sampling_locations  [B, Q, H, L, P, 2]  (x, y) normalised to [0, 1]
    attention_weights   [B, Q, H, L, P]     already normalised (softmax over L * P)
    padding_mask        [B, N] bool or None  True = padded token: its value row is zeroed after the projection
    returns             [B, Q, H * D]
    """
    B, N, _ = memory.shape
    _, Q, H, L, P, _ = sampling_locations.shape
    value = F.linear(memory, value_weight, value_bias)  # [B, N, H * D]
    if padding_mask is not None:
        value = value.masked_fill(padding_mask.bool()[..., None], 0)
    D = value.shape[-1] // H
    # heads to the batch dimension: [B * H, D, N]
    per_head = value.view(B, N, H, D).permute(0, 2, 3, 1).reshape(B * H, D, N)
    # grid_sample's normalised coordinates for align_corners=False: -1 is the left edge of pixel 0
    grid = (sampling_locations * 2 - 1).permute(0, 2, 1, 3, 4, 5).reshape(B * H, Q, L, P, 2)
    out = None
    for lvl in range(L):
        h, w = int(spatial_shapes[lvl, 0]), int(spatial_shapes[lvl, 1])
        s = int(level_start_index[lvl])
        image = per_head[:, :, s:s + h * w].reshape(B * H, D, h, w)
        sampled = F.grid_sample(image, grid[:, :, lvl], mode='bilinear', padding_mode='zeros',
                                align_corners=False)  # [B * H, D, Q, P]
        weights = attention_weights[:, :, :, lvl].permute(0, 2, 1, 3).reshape(B * H, 1, Q, P)
        part = (sampled * weights).sum(-1)  # [B * H, D, Q]
        out = part if out is None else out + part
    if out is None:  # no levels
        out = memory.new_zeros(B * H, D, Q)
    return out.view(B, H, D, Q).permute(0, 3, 1, 2).reshape(B, Q, H * D)
