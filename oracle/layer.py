"""Float64 oracle of a deformable cross-attention decoder layer (numpy). TEST INFRASTRUCTURE ONLY: imported by
tests/, smoke() and bench.py's CPU baseline, never by the product.

Restates, in float64, HF transformers RTDetrMultiscaleDeformableAttention.forward
(models/rt_detr/modeling_rt_detr.py:673-727), the decoder code the layer entries fuse:
  x          = hidden_states + position_embeddings                                   :674-675
  offsets    = x @ Woff^T + boff, viewed [B, Q, H, L, P, 2]                          :690-692
  attention  = softmax over L * P of (x @ Wattn^T + battn), viewed [B, Q, H, L, P]   :693-698
  locations  = ref + offsets / (W_l, H_l)                  (ref [B, Q, 1 or L, 2])   :700-706
             = ref[..., :2] + offsets / P * ref[..., 2:] * 0.5   (ref [..., 4])      :707-711
  out        = output_proj(deform_attn(memory, value_proj, locations, attention))    :685-689, :715-725
with the core from oracle.bruteforce (padded tokens' value rows zeroed, :686-688).
"""

import numpy as np

from . import bruteforce
from .bruteforce import _f64, _i64


def locations(hidden_states, reference_points, spatial_shapes, offsets_weight, offsets_bias, attn_weight, attn_bias,
              num_heads, num_points, position_embeddings=None):
    """Sampling locations [B, Q, H, L, P, 2] and attention weights [B, Q, H, L, P], float64."""
    x = _f64(hidden_states)
    if position_embeddings is not None:
        x = x + _f64(position_embeddings)
    shapes = _i64(spatial_shapes)
    B, Q, _ = x.shape
    H, P, L = num_heads, num_points, shapes.shape[0]
    off = x @ _f64(offsets_weight).T
    if offsets_bias is not None:
        off = off + _f64(offsets_bias)
    off = off.reshape(B, Q, H, L, P, 2)
    logit = x @ _f64(attn_weight).T
    if attn_bias is not None:
        logit = logit + _f64(attn_bias)
    logit = logit.reshape(B, Q, H, L * P)
    e = np.exp(logit - logit.max(-1, keepdims=True))
    attn = (e / e.sum(-1, keepdims=True)).reshape(B, Q, H, L, P)
    ref = _f64(reference_points)[:, :, None, :, None, :]  # [B, Q, 1, 1 or L, 1, 2 or 4]
    if ref.shape[-1] == 2:
        norm = np.stack([shapes[:, 1], shapes[:, 0]], -1).astype(np.float64)  # (width, height)
        loc = ref + off / norm[None, None, None, :, None, :]
    else:
        loc = ref[..., :2] + off / P * ref[..., 2:] * 0.5
    return loc, attn


def layer(hidden_states, memory, reference_points, spatial_shapes, level_start_index, offsets_weight, offsets_bias,
          attn_weight, attn_bias, value_weight, value_bias, output_weight, output_bias, num_heads, num_points,
          position_embeddings=None, padding_mask=None):
    """The layer's output [B, Q, C_out] (the core [B, Q, H * D] when output_weight is None) and the attention
    weights, float64."""
    loc, attn = locations(hidden_states, reference_points, spatial_shapes, offsets_weight, offsets_bias, attn_weight,
                          attn_bias, num_heads, num_points, position_embeddings)
    mask = None if padding_mask is None else np.asarray(_f64(padding_mask) != 0)
    out = bruteforce.deform_attn(memory, value_weight, value_bias, spatial_shapes, level_start_index, loc, attn,
                                 padding_mask=mask)
    if output_weight is not None:
        out = out @ _f64(output_weight).T
        if output_bias is not None:
            out = out + _f64(output_bias)
    return out, attn
