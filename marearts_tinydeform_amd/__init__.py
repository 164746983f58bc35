"""marearts_tinydeform_amd: value projection + multi-scale deformable attention for DETR-style decoders on MI355X.

Drop-in for marearts_tinydeform (same functions, arguments, results and errors; reference
marearts_tinydeform/__init__.py:12-79). GPU tensors run hand-written HIP kernels for gfx950 through the C ABI of
libtinydeform.so; CPU tensors run the PyTorch reference path. Inference only.
"""

import functools

import torch

from . import _native
from .reference import layer_locations_reference, ma_deform_attn_layer_reference, ma_deform_attn_reference

__all__ = ['ma_deform_attn', 'ma_deform_attn_reference', 'choose_mode', 'ma_deform_sample', 'ma_deform_sample_v2',
           'predict_us', 'cost_features', 'ma_deform_attn_layer', 'ma_deform_attn_layer_reference', 'layer_locations_reference',
           'MSDeformAttnLayer', 'ma_deform_attn_train', 'ma_deform_sample_train']
__version__ = '0.1.0'

MODES = ('auto', 'fused', 'project')

# 'auto' compares predicted times of the two orders (reference marearts_tinydeform/__init__.py:21-46 uses one
# threshold on queries * levels * points * 4 / (tokens * head_dim); on MI355X the value GEMM is cheap next to
# gathering C-wide rows, so the crossover also moves with C and one threshold cannot place it). Per dtype, each
# mode's time in µs is a linear function of the work it does (cost_features), fitted to MI355X (gfx950)
# measurements of both modes (bench.py --fit-auto: RT-DETR 640 shapes at batch 1/2/4/8 and 50..900 queries, C = 512
# at batch 1/2/4, DINO 4-level and C = 1024 shapes; checked on shapes outside that grid with bench.py --holdout).
# The coefficients were kept when the deep-K GEMM became persistent 256 x 256 tiles (and gemm_rounds_k began counting
# them): a refit on the new measurements matched them on the fit grid (worst auto/best 1.044) and did worse on the
# held-out grid (1.36 against 1.07). When the fused kernel's projection took every N tile per job (3-4% faster at
# small problems), the 16-bit fused line was scaled by 0.96, and when both gathers moved to buffer loads with
# multiply-high index arithmetic (fused 10-17% faster, the sampler 15-30%) by 0.90 more: every case of the fit grid
# within 10% again (worst 1.094; unscaled 1.123) and 101 to 103 of the 108 held-out cases over two runs (unscaled
# 101; a least-squares refit 99).
#   fused   = f0 + f1 * gathered_mb
#   project = p0 + p1 * gemm_mb + p2 * gemm_gflop + p3 * gemm_rounds_k + p4 * sample_mb
FUSED_LIMIT = {
    torch.float32: {'fused': (7.4791, 0.0478), 'project': (13.9906, 0.6181, 0.0000, 0.0000, 0.0877)},
    torch.float16: {'fused': (4.9276, 0.0503), 'project': (11.5020, 0.1554, 0.0000, 10.1974, 0.0925)},
    torch.bfloat16: {'fused': (4.9276, 0.0503), 'project': (11.5020, 0.1554, 0.0000, 10.1974, 0.0925)},
}


def cost_features(B, Q, H, D, C, N, L, P, s):
    """The work each mode does, the terms of its cost line: ([1, gathered_mb], [1, gemm_mb, gemm_gflop,
    gemm_rounds_k, sample_mb]) with s the element size in bytes:
      gathered_mb    B*Q*H*L*P*4*C*s / 1e6   C-wide corner rows read by 'fused'
      gemm_mb        B*N*(C + H*D)*s / 1e6   value GEMM traffic of 'project'
      gemm_gflop     2*B*N*C*H*D / 1e9       value GEMM work of 'project' for C < 512 (the bandwidth-bound kernels)
      gemm_rounds_k  rounds of 256 x 256 output tiles over MI355X's 256 CUs, times C / 1e3, for C >= 512 (the
                     direct-to-LDS kernels, whose time goes by the busiest CU's count of tiles, each as long as K)
      sample_mb      B*Q*H*L*P*4*D*s / 1e6   D-wide corner rows read by 'project'"""
    samples = B * Q * H * L * P * 4
    HD, M = H * D, B * N
    if C >= 512:
        tiles = -(-M // 256) * -(-HD // 256)
        narrow, deep = 0.0, -(-tiles // 256) * C / 1e3
    else:
        narrow, deep = 2 * M * C * HD / 1e9, 0.0
    return ([1.0, samples * C * s / 1e6], [1.0, M * (C + HD) * s / 1e6, narrow, deep, samples * D * s / 1e6])


# cost tables by GPU architecture (gcnArchName without feature suffixes)
ARCH_LIMITS = {'gfx950': FUSED_LIMIT}


def _arch(device_index):
    return torch.cuda.get_device_properties(device_index).gcnArchName.split(':')[0]


@functools.lru_cache(maxsize=None)
def _limits(device_index):
    return ARCH_LIMITS.get(_arch(device_index), FUSED_LIMIT)


def predict_us(memory, value_weight, sampling_locations, table=None):
    """Predicted µs of mode 'fused' and 'project' for these shapes: {'fused': t, 'project': t}."""
    _, Q, H, L, P, _ = sampling_locations.shape
    return _predict(memory, value_weight, Q, H, L, P, table)


def _predict(memory, value_weight, Q, H, L, P, table=None):
    B, N, C = memory.shape
    HD = value_weight.shape[0]
    D = HD // max(H, 1)
    s = memory.element_size()
    if table is None:
        table = _limits(memory.get_device()) if memory.is_cuda else FUSED_LIMIT
    coef = table.get(memory.dtype, table[torch.float16])
    ff, fp = cost_features(B, Q, H, D, C, N, L, P, s)
    return {'fused': sum(c * x for c, x in zip(coef['fused'], ff)),
            'project': sum(c * x for c, x in zip(coef['project'], fp))}


def choose_mode(memory, value_weight, sampling_locations):
    """The mode 'auto' runs: 'fused' for few queries per image, 'project' (project every token first) for many."""
    t = predict_us(memory, value_weight, sampling_locations)
    return 'fused' if t['fused'] <= t['project'] else 'project'


def _reject_grad(*tensors):
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise RuntimeError('ma_deform_attn is inference only: run it under torch.no_grad() / '
                           'torch.inference_mode(), or use ma_deform_attn_reference for training')


def _on_device(t, fn, *args):
    if t.device.index is None or t.device.index == torch.cuda.current_device():
        return fn(*args)
    with torch.cuda.device(t.device):
        return fn(*args)


def ma_deform_attn(memory, value_weight, value_bias, spatial_shapes, level_start_index,
                   sampling_locations, attention_weights, mode='auto', padding_mask=None):
    """value = memory @ value_weight.T + value_bias, then multi-scale deformable attention; [B, Q, H * D].

    Same arguments, shapes and result as ma_deform_attn_reference (grid_sample, bilinear, zero padding,
    align_corners=False). GPU tensors (float32, float16, bfloat16, float64; float32 accumulation for the
    16/32-bit types):
      mode='fused'    gather the sampled memory rows first, then project per (query, head) on MFMA
      mode='project'  project all tokens (the library's MFMA GEMM), then sample
      mode='auto'     choose_mode() picks one by size (default)
    padding_mask: optional bool [B, N], True for padded tokens, whose value is zero
    (value.masked_fill(padding_mask[..., None], 0) after the projection, as Deformable-DETR decoders do; HF RT-DETR
    passes ~attention_mask). Not in the reference operator, which has no mask.
    CPU tensors run the reference. Inference only: inputs that require grad are rejected.
    """
    if mode not in MODES:
        raise ValueError(f'mode must be one of {MODES}, got {mode!r}')
    if not memory.is_cuda:
        return ma_deform_attn_reference(memory, value_weight, value_bias, spatial_shapes, level_start_index,
                                        sampling_locations, attention_weights, padding_mask=padding_mask)
    _native._require()
    _reject_grad(memory, value_weight, value_bias, sampling_locations, attention_weights)
    if mode == 'auto':
        mode = choose_mode(memory, value_weight, sampling_locations)
    if mode == 'fused':
        return _on_device(memory, _native.fused_forward, memory, value_weight, value_bias, spatial_shapes,
                          level_start_index, sampling_locations, attention_weights, padding_mask)
    return _on_device(memory, _project, memory, value_weight, value_bias, spatial_shapes, level_start_index,
                      sampling_locations, attention_weights, padding_mask)


def _project(memory, value_weight, value_bias, spatial_shapes, level_start_index, sampling_locations,
             attention_weights, padding_mask):
    # padded tokens: the sampler drops their corners, the same as zeroing their value rows
    return _native.project_forward(memory, value_weight, value_bias, spatial_shapes, level_start_index,
                                   sampling_locations, attention_weights, padding_mask)


def ma_deform_sample(value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                     padding_mask=None):
    """Multi-scale deformable attention on already projected values [B, N, H * D] -> [B, Q, H * D].

    The sampling half of mode='project' on its own (for decoders whose value projection is done elsewhere, e.g.
    D-FINE). padding_mask as in ma_deform_attn. GPU tensors only.
    """
    _native._require()
    _reject_grad(value, sampling_locations, attention_weights)
    H = sampling_locations.shape[2] if sampling_locations.dim() == 6 else 0
    return _on_device(value, _native.sample_forward, value, H, spatial_shapes, level_start_index,
                      sampling_locations, attention_weights, padding_mask)


def ma_deform_sample_v2(value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                        num_points_list, method='default', padding_mask=None):
    """D-FINE's deformable attention core on the GPU: per-level point counts and the 'default' (bilinear, zero
    padding, align_corners=False) or 'discrete' (nearest pixel, clamped) method; the result of transformers'
    multi_scale_deformable_attention_v2 (models/d_fine/modeling_d_fine.py:150-216) with the value padding already
    applied by padding_mask.

    value               [B, N, H, D] or [B, N, H * D]   (D-FINE has no value projection)
    sampling_locations  [B, Q, H, sum(num_points_list), 2]
    attention_weights   [B, Q, H, sum(num_points_list)]
    returns             [B, Q, H * D]
    """
    _native._require()
    _reject_grad(value, sampling_locations, attention_weights)
    return _on_device(value, _native.sample_forward_v2, value, spatial_shapes, level_start_index, sampling_locations,
                      attention_weights, num_points_list, method, padding_mask)


def ma_deform_attn_layer(hidden_states, encoder_hidden_states, reference_points, spatial_shapes, level_start_index,
                         sampling_offsets_weight, sampling_offsets_bias, attention_weights_weight,
                         attention_weights_bias, value_weight, value_bias, output_weight, output_bias, num_heads,
                         num_points, position_embeddings=None, padding_mask=None, mode='auto',
                         return_attention_weights=False):
    """One deformable cross-attention layer of a DETR decoder (HF transformers RTDetrMultiscaleDeformableAttention,
    models/rt_detr/modeling_rt_detr.py:673-727) with its producers fused on the GPU:

      x          = hidden_states (+ position_embeddings)                        [B, Q, C]
      offsets    = x @ sampling_offsets_weight.T + bias    -> [B, Q, H, L, P, 2]
      attention  = softmax over L * P of (x @ attention_weights_weight.T + bias)
      locations  = reference_points + offsets / (W_l, H_l)          (points, [B, Q, 1 or L, 2])
                 = ref[..., :2] + offsets / P * ref[..., 2:] * 0.5  (boxes, [B, Q, 1 or L, 4])
      out        = output_proj(ma_deform_attn(encoder_hidden_states, value_weight, value_bias, ...))

    mode='fused': one kernel computes each (query tile, head)'s offsets and attention on MFMA, keeps the locations
    in float32 in LDS and gathers the memory rows; mode='project': the query prologue kernel, the value GEMM and
    the sampler; 'auto' picks by size as ma_deform_attn does. output_proj runs on the library's GEMM (skipped when
    output_weight is None). padding_mask: bool [B, N], True = padded token (HF passes ~attention_mask).
    Returns [B, Q, C_out], and the attention weights [B, Q, H, L, P] too with return_attention_weights.
    CPU tensors run ma_deform_attn_layer_reference. Inference only.
    """
    if mode not in MODES:
        raise ValueError(f'mode must be one of {MODES}, got {mode!r}')
    args = (hidden_states, encoder_hidden_states, reference_points, spatial_shapes, level_start_index,
            sampling_offsets_weight, sampling_offsets_bias, attention_weights_weight, attention_weights_bias,
            value_weight, value_bias, output_weight, output_bias, num_heads, num_points)
    if not encoder_hidden_states.is_cuda:
        return ma_deform_attn_layer_reference(*args, position_embeddings=position_embeddings,
                                              padding_mask=padding_mask,
                                              return_attention_weights=return_attention_weights)
    _native._require()
    _reject_grad(hidden_states, encoder_hidden_states, reference_points, sampling_offsets_weight,
                 sampling_offsets_bias, attention_weights_weight, attention_weights_bias, value_weight, value_bias,
                 output_weight, output_bias, position_embeddings)
    return _on_device(encoder_hidden_states, _layer, *args, position_embeddings, padding_mask, mode,
                      return_attention_weights)


def _layer(hidden_states, memory, reference_points, spatial_shapes, level_start_index, ow, ob, aw, ab, value_weight,
           value_bias, output_weight, output_bias, num_heads, num_points, position, padding_mask, mode, want_attn):
    B, Q, Cq, H, L, P = _native.check_layer(memory, hidden_states, reference_points, ow, ob, aw, ab, position,
                                            spatial_shapes, num_heads, num_points)
    if mode == 'auto':
        t = _predict(memory, value_weight, Q, H, L, P)
        mode = 'fused' if t['fused'] <= t['project'] else 'project'
    if mode == 'fused':
        core, la = _native.layer_fused_forward(hidden_states, position, reference_points, ow, ob, aw, ab, memory,
                                               value_weight, value_bias, spatial_shapes, level_start_index, H, P,
                                               padding_mask, return_locations=want_attn)
        attn = la[1] if want_attn else None
    else:
        _native.check_projection(memory, value_weight, value_bias, H)
        _native.check_padding_mask(memory, padding_mask)
        loc, attn = _native.layer_prologue(hidden_states, position, reference_points, ow, ob, aw, ab, spatial_shapes,
                                           H, P)
        core = _native.project_forward(memory, value_weight, value_bias, spatial_shapes, level_start_index, loc, attn,
                                       padding_mask, loc_acc=True)
    out = core if output_weight is None else _native.value_proj(core, output_weight, output_bias)
    if want_attn:
        return out, attn.to(memory.dtype)
    return out


class _DeformAttnFunction(torch.autograd.Function):
    """value = memory @ W^T + b, then sampling, on the library's kernels, with gradients for memory, W, b, the
    locations and the attention weights (td_sample_backward, td_input_grad, td_weight_grad)."""

    @staticmethod
    def forward(ctx, memory, value_weight, value_bias, spatial_shapes, level_start_index, sampling_locations,
                attention_weights, padding_mask):
        H = sampling_locations.shape[2] if sampling_locations.dim() == 6 else 0
        _native.check_geometry(memory, spatial_shapes, level_start_index, sampling_locations, attention_weights)
        _native.check_padding_mask(memory, padding_mask)
        value = _native.value_proj(memory, value_weight, value_bias)
        out = _native.sample_forward(value, H, spatial_shapes, level_start_index, sampling_locations,
                                     attention_weights, padding_mask)
        ctx.save_for_backward(memory, value_weight, value, spatial_shapes, level_start_index, sampling_locations,
                              attention_weights, padding_mask)
        ctx.has_bias = value_bias is not None
        return out

    @staticmethod
    def backward(ctx, grad_out):
        memory, weight, value, shapes, starts, loc, attn, mask = ctx.saved_tensors
        need = ctx.needs_input_grad
        gv, gl, ga = _native.sample_backward(value, loc.shape[2], shapes, starts, loc, attn, grad_out, mask)
        gm = _native.input_grad(gv, weight) if need[0] else None
        gw = gb = None
        if need[1] or (need[2] and ctx.has_bias):
            gw, gb = _native.weight_grad(gv, memory, with_bias=ctx.has_bias and need[2])
        return (gm, gw if need[1] else None, gb, None, None, gl if need[5] else None, ga if need[6] else None, None)


class _DeformSampleFunction(torch.autograd.Function):
    """Sampling of projected values with gradients for the values, the locations and the attention weights."""

    @staticmethod
    def forward(ctx, value, spatial_shapes, level_start_index, sampling_locations, attention_weights, padding_mask):
        H = sampling_locations.shape[2] if sampling_locations.dim() == 6 else 0
        out = _native.sample_forward(value, H, spatial_shapes, level_start_index, sampling_locations,
                                     attention_weights, padding_mask)
        ctx.save_for_backward(value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                              padding_mask)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        value, shapes, starts, loc, attn, mask = ctx.saved_tensors
        need = ctx.needs_input_grad
        gv, gl, ga = _native.sample_backward(value, loc.shape[2], shapes, starts, loc, attn, grad_out, mask)
        return gv if need[0] else None, None, None, gl if need[3] else None, ga if need[4] else None, None


def ma_deform_attn_train(memory, value_weight, value_bias, spatial_shapes, level_start_index, sampling_locations,
                         attention_weights, padding_mask=None):
    """ma_deform_attn with autograd, for training: the same arguments and result (project order: the value
    projection, then sampling), differentiable in memory, value_weight, value_bias, sampling_locations and
    attention_weights. GPU tensors run the library's forward and backward kernels (float32 accumulation for the
    16/32-bit types); CPU tensors run ma_deform_attn_reference under PyTorch's autograd. ma_deform_attn itself stays
    inference only, as in the reference."""
    if not memory.is_cuda:
        return ma_deform_attn_reference(memory, value_weight, value_bias, spatial_shapes, level_start_index,
                                        sampling_locations, attention_weights, padding_mask=padding_mask)
    _native._require()
    return _on_device(memory, _DeformAttnFunction.apply, memory, value_weight, value_bias, spatial_shapes,
                      level_start_index, sampling_locations, attention_weights, padding_mask)


def ma_deform_sample_train(value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                           padding_mask=None):
    """ma_deform_sample with autograd: differentiable in value [B, N, H * D], sampling_locations and
    attention_weights (Deformable-DETR's MSDeformAttnFunction, for decoders that project the values themselves).
    GPU tensors only."""
    _native._require()
    return _on_device(value, _DeformSampleFunction.apply, value, spatial_shapes, level_start_index,
                      sampling_locations, attention_weights, padding_mask)


def _grid_offsets_bias(n_heads, n_levels, n_points):
    """Deformable-DETR's initial sampling-offset bias: head h looks along direction 2 pi h / H (scaled so the larger
    coordinate is 1), point p at distance p + 1, on every level."""
    theta = torch.arange(n_heads, dtype=torch.float32) * (2.0 * torch.pi / n_heads)
    grid = torch.stack([theta.cos(), theta.sin()], -1)
    grid = grid / grid.abs().max(-1, keepdim=True)[0]
    grid = grid.view(n_heads, 1, 1, 2).repeat(1, n_levels, n_points, 1)
    grid = grid * torch.arange(1, n_points + 1, dtype=torch.float32).view(1, 1, n_points, 1)
    return grid.flatten()


class MSDeformAttnLayer(torch.nn.Module):
    """Deformable cross-attention module of a DETR decoder, running ma_deform_attn_layer.

    Same submodules as HF transformers' RTDetrMultiscaleDeformableAttention (sampling_offsets, attention_weights,
    value_proj, output_proj; models/rt_detr/modeling_rt_detr.py:623-658), so its state dict loads unchanged, and the
    same forward arguments and results: (output [B, Q, d_model], attention_weights [B, Q, H, L, P]).
    attention_mask is the encoder's validity mask (True = real token), as HF passes it.
    """

    def __init__(self, d_model=256, n_levels=4, n_heads=8, n_points=4, mode='auto'):
        super().__init__()
        if d_model % n_heads != 0:
            raise ValueError(f'd_model ({d_model}) must be divisible by n_heads ({n_heads})')
        self.d_model, self.n_levels, self.n_heads, self.n_points, self.mode = d_model, n_levels, n_heads, n_points, mode
        self.sampling_offsets = torch.nn.Linear(d_model, n_heads * n_levels * n_points * 2)
        self.attention_weights = torch.nn.Linear(d_model, n_heads * n_levels * n_points)
        self.value_proj = torch.nn.Linear(d_model, d_model)
        self.output_proj = torch.nn.Linear(d_model, d_model)
        self.reset_parameters()

    @torch.no_grad()
    def reset_parameters(self):
        torch.nn.init.zeros_(self.sampling_offsets.weight)
        self.sampling_offsets.bias.copy_(_grid_offsets_bias(self.n_heads, self.n_levels, self.n_points))
        torch.nn.init.zeros_(self.attention_weights.weight)
        torch.nn.init.zeros_(self.attention_weights.bias)
        for lin in (self.value_proj, self.output_proj):
            torch.nn.init.xavier_uniform_(lin.weight)
            torch.nn.init.zeros_(lin.bias)

    def forward(self, hidden_states, attention_mask=None, encoder_hidden_states=None, encoder_attention_mask=None,
                position_embeddings=None, reference_points=None, spatial_shapes=None, spatial_shapes_list=None,
                level_start_index=None, **kwargs):
        if level_start_index is None:
            sizes = spatial_shapes[:, 0] * spatial_shapes[:, 1]
            level_start_index = torch.cat([sizes.new_zeros(1), sizes.cumsum(0)[:-1]])
        padding_mask = None if attention_mask is None else ~attention_mask.bool()
        if torch.is_grad_enabled() and (any(t.requires_grad for t in self.parameters()) or any(
                t is not None and t.requires_grad for t in (hidden_states, encoder_hidden_states, position_embeddings,
                                                            reference_points))):
            # training: the query prologue and output_proj under PyTorch's autograd, the operator on the library's
            # forward and backward kernels
            loc, attn = layer_locations_reference(
                hidden_states, reference_points, spatial_shapes, self.sampling_offsets.weight,
                self.sampling_offsets.bias, self.attention_weights.weight, self.attention_weights.bias, self.n_heads,
                self.n_points, position_embeddings)
            core = ma_deform_attn_train(encoder_hidden_states, self.value_proj.weight, self.value_proj.bias,
                                        spatial_shapes, level_start_index, loc, attn, padding_mask=padding_mask)
            return self.output_proj(core), attn
        return ma_deform_attn_layer(
            hidden_states, encoder_hidden_states, reference_points, spatial_shapes, level_start_index,
            self.sampling_offsets.weight, self.sampling_offsets.bias, self.attention_weights.weight,
            self.attention_weights.bias, self.value_proj.weight, self.value_proj.bias, self.output_proj.weight,
            self.output_proj.bias, self.n_heads, self.n_points, position_embeddings=position_embeddings,
            padding_mask=padding_mask, mode=self.mode, return_attention_weights=True)
