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


def layer_locations_reference(hidden_states, reference_points, spatial_shapes, sampling_offsets_weight,
                              sampling_offsets_bias, attention_weights_weight, attention_weights_bias, num_heads,
                              num_points, position_embeddings=None):
    """Sampling locations [B, Q, H, L, P, 2] and attention weights [B, Q, H, L, P] of a deformable-attention layer,
    in PyTorch (HF transformers RTDetrMultiscaleDeformableAttention.forward, models/rt_detr/modeling_rt_detr.py:673-713).

    reference_points [B, Q, 1 or L, 2] are points, [B, Q, 1 or L, 4] boxes (centre, size): a point's offsets are
    divided by the level's (width, height); a box's by num_points, scaled by half its size.
    """
    if position_embeddings is not None:
        hidden_states = hidden_states + position_embeddings
    B, Q, _ = hidden_states.shape
    H, P, L = num_heads, num_points, spatial_shapes.shape[0]
    offsets = F.linear(hidden_states, sampling_offsets_weight, sampling_offsets_bias).view(B, Q, H, L, P, 2)
    logits = F.linear(hidden_states, attention_weights_weight, attention_weights_bias).view(B, Q, H, L * P)
    attention = F.softmax(logits, -1).view(B, Q, H, L, P)
    ref = reference_points[:, :, None, :, None, :]  # [B, Q, 1, 1 or L, 1, 2 or 4]
    if reference_points.shape[-1] == 2:
        normalizer = torch.stack([spatial_shapes[..., 1], spatial_shapes[..., 0]], -1)  # (width, height)
        locations = ref + offsets / normalizer[None, None, None, :, None, :]
    elif reference_points.shape[-1] == 4:
        locations = ref[..., :2] + offsets / P * ref[..., 2:] * 0.5
    else:
        raise ValueError(f'reference_points must end in 2 or 4 coordinates, got {reference_points.shape[-1]}')
    return locations, attention


def ma_deform_attn_layer_reference(hidden_states, encoder_hidden_states, reference_points, spatial_shapes,
                                   level_start_index, sampling_offsets_weight, sampling_offsets_bias,
                                   attention_weights_weight, attention_weights_bias, value_weight, value_bias,
                                   output_weight, output_bias, num_heads, num_points, position_embeddings=None,
                                   padding_mask=None, return_attention_weights=False):
    """One deformable cross-attention layer of a DETR decoder in PyTorch: the query prologue
    (layer_locations_reference), value projection and multi-scale deformable attention (ma_deform_attn_reference),
    then output_proj (skipped when output_weight is None). Returns [B, Q, C_out] (and the attention weights with
    return_attention_weights)."""
    locations, attention = layer_locations_reference(
        hidden_states, reference_points, spatial_shapes, sampling_offsets_weight, sampling_offsets_bias,
        attention_weights_weight, attention_weights_bias, num_heads, num_points, position_embeddings)
    out = ma_deform_attn_reference(encoder_hidden_states, value_weight, value_bias, spatial_shapes, level_start_index,
                                   locations, attention, padding_mask=padding_mask)
    if output_weight is not None:
        out = F.linear(out, output_weight, output_bias)
    return (out, attention) if return_attention_weights else out
